// The BF16 decode GEMV as device functions shared by the standalone kernels
// (decode.hip) and the persistent decode kernel (persistent.hip).
//
// Reference: matmul_w_into (src/tensor.rs:331-460), hot loop dot_bf16_avx2
// (src/tensor.rs:78-96).  A 256-thread workgroup owns R output rows ("a
// block") and covers the whole input dimension; thread t streams 16 B (8 BF16)
// of every row per 2048-element chunk, so one wavefront load is a contiguous
// 1 KiB of a row.  The row loads of a block are issued before the activation
// prologue (they do not depend on it), the activation lives in registers, and
// the per-row reduction is a transposed shuffle butterfly plus a 4-wave LDS
// sum.
//
// COH selects device-coherent (sc1) accesses for activations, for use inside a
// persistent kernel where other workgroups wrote them in the same launch.
#pragma once

#include "coh.cuh"
#include "common.cuh"
#include "kernels.hpp"

namespace tmg {

constexpr int kChunk = kBlock * 8;  // elements per chunk: 8 per thread

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int KC>
__host__ __device__ constexpr int gemv_rows() {
    return KC <= 2 ? 8 : 4;
}

template <int KC, int R>
struct WeightRegs {
    u32x4 w[R][KC];
};

// Issue the loads of block `blk` (rows blk*R .. blk*R+R-1, clamped).
template <int KC, int R>
__device__ __forceinline__ void gemv_load(const GemvArgs &a, int blk, WeightRegs<KC, R> &W) {
    const int t = threadIdx.x;
    const int row0 = blk * R;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = min(row0 + r, a.out - 1);
        const u32x4 *wr = reinterpret_cast<const u32x4 *>(a.W + (size_t)row * a.in);
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const int k = c * kChunk + t * 8;
            W.w[r][c] = (k < a.in) ? __builtin_nontemporal_load(wr + (k >> 3)) : u32x4{0u, 0u, 0u, 0u};
        }
    }
}

template <int KC, bool COH>
__device__ __forceinline__ void load_act(const float *src, const uint16_t *src_bf, int in, float (&xv)[KC][8]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int c = 0; c < KC; c++) {
        const int k = c * kChunk + t * 8;
        if (k < in) {
            if (src_bf) {
                const uint4 u = *reinterpret_cast<const uint4 *>(src_bf + k);
                xv[c][0] = bf16_lo(u.x);
                xv[c][1] = bf16_hi(u.x);
                xv[c][2] = bf16_lo(u.y);
                xv[c][3] = bf16_hi(u.y);
                xv[c][4] = bf16_lo(u.z);
                xv[c][5] = bf16_hi(u.z);
                xv[c][6] = bf16_lo(u.w);
                xv[c][7] = bf16_hi(u.w);
            } else {
                const float4 p = ldf4<COH>(src + k);
                const float4 q = ldf4<COH>(src + k + 4);
                xv[c][0] = p.x;
                xv[c][1] = p.y;
                xv[c][2] = p.z;
                xv[c][3] = p.w;
                xv[c][4] = q.x;
                xv[c][5] = q.y;
                xv[c][6] = q.z;
                xv[c][7] = q.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) xv[c][j] = 0.0f;
        }
    }
}

// Split count of a decode attention row at context n_ctx: the same formula in
// the attention kernel, its combine kernel and the fused combine prologue.
__device__ __forceinline__ int active_splits(int n_ctx, int nsplit, int min_chunk) {
    return min(nsplit, (n_ctx + min_chunk - 1) / min_chunk);
}

// The attention output for this thread's 8 consecutive dims (one head),
// merged from the active splits: o = sum_s e^(m_s-M) o_s / sum_s e^(m_s-M) l_s.
template <int KC, bool COH>
__device__ __forceinline__ void load_attn(const GemvArgs &a, int pos, float (&xv)[KC][8]) {
    const int t = threadIdx.x;
    const int active = active_splits(pos + 1, a.nsplit, a.min_chunk);
#pragma unroll
    for (int c = 0; c < KC; c++) {
        const int k = c * kChunk + t * 8;
#pragma unroll
        for (int j = 0; j < 8; j++) xv[c][j] = 0.0f;
        if (k >= a.in) continue;
        const int h = k / a.hd, d = k - h * a.hd;
        const int g = h / a.group, hq = h - g * a.group;
        const size_t base = (size_t)g * a.nsplit * a.group + hq;  // + split * group
        float M = -INFINITY;
        for (int sp = 0; sp < active; sp++) M = fmaxf(M, ldf<COH>(a.part_ml + (base + (size_t)sp * a.group) * 2));
        float L = 0.0f;
        for (int sp = 0; sp < active; sp++) {
            const size_t pi = base + (size_t)sp * a.group;
            const float m = ldf<COH>(a.part_ml + pi * 2);
            const float w = (m == -INFINITY) ? 0.0f : expf(m - M);
            L = fmaf(ldf<COH>(a.part_ml + pi * 2 + 1), w, L);
            const float4 o0 = ldf4<COH>(a.part + pi * a.hd + d);
            const float4 o1 = ldf4<COH>(a.part + pi * a.hd + d + 4);
            xv[c][0] = fmaf(o0.x, w, xv[c][0]);
            xv[c][1] = fmaf(o0.y, w, xv[c][1]);
            xv[c][2] = fmaf(o0.z, w, xv[c][2]);
            xv[c][3] = fmaf(o0.w, w, xv[c][3]);
            xv[c][4] = fmaf(o1.x, w, xv[c][4]);
            xv[c][5] = fmaf(o1.y, w, xv[c][5]);
            xv[c][6] = fmaf(o1.z, w, xv[c][6]);
            xv[c][7] = fmaf(o1.w, w, xv[c][7]);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) xv[c][j] = xv[c][j] / L;
    }
}

// Activation prologue: gather / load, then RMSNorm when PRO asks for it
// (reference rms_norm_into, src/tensor.rs:969-977; batch association
// src/tensor.rs:946-954).  `scratch` holds 4 floats of LDS.  `tok` and `pos`
// are the step's token and position (read once by the caller).
template <int KC, int PRO, bool COH>
__device__ __forceinline__ void gemv_prologue(const GemvArgs &a, int tok, int pos, float (&xv)[KC][8], float *scratch,
                                              bool store_x) {
    const int t = threadIdx.x;
    const int in = a.in;
    if constexpr (PRO == PRO_ATTN_COMBINE) {
        load_attn<KC, COH>(a, pos, xv);
        return;
    } else if constexpr (PRO == PRO_EMBED_NORM) {
        if (a.embed_bf16)
            load_act<KC, false>(nullptr, a.embed_bf16 + (size_t)tok * in, in, xv);
        else
            load_act<KC, false>(a.embed_f32 + (size_t)tok * in, nullptr, in, xv);
        if (store_x) {
#pragma unroll
            for (int c = 0; c < KC; c++) {
                const int k = c * kChunk + t * 8;
                if (k < in)
#pragma unroll
                    for (int j = 0; j < 8; j++) stf<COH>(a.x_store + k + j, xv[c][j]);
            }
        }
    } else {
        load_act<KC, COH>(a.x, nullptr, in, xv);
    }
    if constexpr (PRO != PRO_PLAIN) {
        float ss[1] = {0.0f};
#pragma unroll
        for (int c = 0; c < KC; c++)
#pragma unroll
            for (int j = 0; j < 8; j++) ss[0] += xv[c][j] * xv[c][j];
        block_sum_n<1>(ss, scratch);
        const float inv = 1.0f / sqrtf(ss[0] / (float)in + a.eps);
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const int k = c * kChunk + t * 8;
            if (k < in) {
                const float4 w0 = *reinterpret_cast<const float4 *>(a.norm_w + k);
                const float4 w1 = *reinterpret_cast<const float4 *>(a.norm_w + k + 4);
                const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    // decode (v*inv)*w; batch v*(inv*w) (src/tensor.rs:975 vs :951)
                    if constexpr (PRO == PRO_NORM_BATCH)
                        xv[c][j] = __fmul_rn(xv[c][j], __fmul_rn(inv, w[j]));
                    else
                        xv[c][j] = __fmul_rn(__fmul_rn(xv[c][j], inv), w[j]);
                }
            }
        }
    }
}

// FMAs over a loaded block, the block reduction and the epilogue.
// `red` is LDS of 4*R floats.  Returns after the epilogue; the caller
// separates consecutive calls with a __syncthreads (red is reused).
template <int KC, int R, int EPI, bool COH>
__device__ __forceinline__ void gemv_finish(const GemvArgs &a, int blk, int pos, const WeightRegs<KC, R> &W,
                                            const float (&xv)[KC][8], float (*red)[R]) {
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const u32x4 u = W.w[r][c];
            s0 = fmaf(xv[c][0], bf16_lo(u.x), s0);
            s1 = fmaf(xv[c][1], bf16_hi(u.x), s1);
            s0 = fmaf(xv[c][2], bf16_lo(u.y), s0);
            s1 = fmaf(xv[c][3], bf16_hi(u.y), s1);
            s0 = fmaf(xv[c][4], bf16_lo(u.z), s0);
            s1 = fmaf(xv[c][5], bf16_hi(u.z), s1);
            s0 = fmaf(xv[c][6], bf16_lo(u.w), s0);
            s1 = fmaf(xv[c][7], bf16_hi(u.w), s1);
        }
        acc[r] = s0 + s1;
    }
    {
        constexpr int LR = R == 8 ? 3 : R == 4 ? 2 : R == 2 ? 1 : 0;
        const float s = multi_wave_sum<R>(acc, lane);
        if ((lane & ((64 >> LR) - 1)) == 0) red[wave][lane >> (6 - LR)] = s;
    }
    __syncthreads();
    const int row0 = blk * R;
    if constexpr (EPI == EPI_STORE || EPI == EPI_RESID || EPI == EPI_LOGITS) {
        if (t < R) {
            const int row = row0 + t;
            const float v = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
            const bool ok = row < a.out;
            if (ok) {
                if constexpr (EPI == EPI_RESID)
                    stf<COH>(a.y + row, ldf<COH>(a.y + row) + v);
                else
                    a.y[row] = v;  // logits / plain output: read after the launch
            }
            if constexpr (EPI == EPI_LOGITS) {
                if (a.argmax_part) {
                    unsigned long long key = (ok && v == v) ? argmax_key(v, (uint32_t)row) : 0ull;
#pragma unroll
                    for (int off = R / 2; off > 0; off >>= 1) {
                        const unsigned long long o = shfl_xor_u64(key, off);
                        key = o > key ? o : key;
                    }
                    if (t == 0) stu64<COH>(a.argmax_part + blk, key);
                }
            }
        }
    } else {
        if (t < R / 2) {
            const int P = row0 / 2 + t;  // global pair index
            const float va = (red[0][2 * t] + red[1][2 * t]) + (red[2][2 * t] + red[3][2 * t]);
            const float vb = (red[0][2 * t + 1] + red[1][2 * t + 1]) + (red[2][2 * t + 1] + red[3][2 * t + 1]);
            if (2 * P + 1 < a.out) {
                if constexpr (EPI == EPI_SWIGLU) {
                    stf<COH>(a.y + P, swiglu(va, vb));
                } else {  // EPI_QKV: pair (j, j + hd/2) of head P / (hd/2)
                    const int half = a.hd >> 1;
                    const int head = P / half, j = P - head * half;
                    const int kvd = a.nkv * a.hd;
                    if (head < a.nq + a.nkv) {
                        float oa, ob;
                        rope_pair(va, vb, a.rope_cos[(size_t)pos * half + j], a.rope_sin[(size_t)pos * half + j], &oa,
                                  &ob);
                        if (head < a.nq) {
                            stf<COH>(a.q_out + head * a.hd + j, oa);
                            stf<COH>(a.q_out + head * a.hd + j + half, ob);
                        } else {
                            float *kr = a.k_cache + (size_t)pos * kvd + (head - a.nq) * a.hd;
                            stf<COH>(kr + j, oa);
                            stf<COH>(kr + j + half, ob);
                        }
                    } else {
                        float *vr = a.v_cache + (size_t)pos * kvd + (head - a.nq - a.nkv) * a.hd;
                        stf<COH>(vr + j, va);
                        stf<COH>(vr + j + half, vb);
                    }
                }
            }
        }
    }
}

}  // namespace tmg
