// The BF16 decode GEMV as device functions of the decode kernels
// (decode.hip): weight loads, activation prologues, dots, the block
// reduction and the fused epilogues.
//
// Reference: matmul_w_into (src/tensor.rs:331-460), hot loop dot_bf16_avx2
// (src/tensor.rs:78-96).  A 256-thread workgroup owns R output rows ("a
// block") and covers the whole input dimension; thread t streams 16 B (8 BF16)
// of every row per 2048-element chunk, so one wavefront load is a contiguous
// 1 KiB of a row.  The row loads of a block are issued before the activation
// prologue (they do not depend on it), the activation lives in registers, and
// the per-row reduction is a transposed shuffle butterfly plus a 4-wave LDS
// sum.
#pragma once

#include "attn.cuh"
#include "common.cuh"
#include "kernels.hpp"

namespace tmg {

constexpr int kChunk = kBlock * 8;  // elements per chunk: 8 per thread

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int KC>
__host__ __device__ constexpr int gemv_rows() {
    return KC <= 3 ? 8 : 4;
}

template <int KC, int R>
struct WeightRegs {
    u32x4 w[R][KC];
};

// Issue the loads of block `blk` (rows blk*R .. blk*R+R-1, clamped).  NT
// threads per workgroup: a chunk is NT * 8 elements of a row.
template <int KC, int R, int NT = kBlock>
__device__ __forceinline__ void gemv_load(const GemvArgs &a, int blk, WeightRegs<KC, R> &W) {
    const int t = threadIdx.x;
    const int row0 = blk * R;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = min(row0 + r, a.out - 1);
        const u32x4 *wr = reinterpret_cast<const u32x4 *>(a.W + (size_t)row * a.in);
#pragma unroll
        for (int c = 0; c < KC; c++) {
            // clamped instead of branched, so all loads issue back to back;
            // gemv_finish zeroes the chunks past the row end
            const int k = c * NT * 8 + t * 8;
            W.w[r][c] = __builtin_nontemporal_load(wr + (min(k, a.in - 8) >> 3));
        }
    }
}

template <int KC, int NT = kBlock>
__device__ __forceinline__ void load_act(const float *src, const uint16_t *src_bf, int in, float (&xv)[KC][8]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int c = 0; c < KC; c++) {
        const int k = c * NT * 8 + t * 8;
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
                const float4 p = *reinterpret_cast<const float4 *>(src + k);
                const float4 q = *reinterpret_cast<const float4 *>(src + k + 4);
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

template <int KC, int NT = kBlock>
__device__ __forceinline__ void load_norm_w(const GemvArgs &a, float (&wv)[KC][8]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int c = 0; c < KC; c++) {
        const int k = c * NT * 8 + t * 8;
        float4 w0 = make_float4(0.f, 0.f, 0.f, 0.f), w1 = w0;
        if (k < a.in) {
            w0 = *reinterpret_cast<const float4 *>(a.norm_w + k);
            w1 = *reinterpret_cast<const float4 *>(a.norm_w + k + 4);
        }
        wv[c][0] = w0.x;
        wv[c][1] = w0.y;
        wv[c][2] = w0.z;
        wv[c][3] = w0.w;
        wv[c][4] = w1.x;
        wv[c][5] = w1.y;
        wv[c][6] = w1.z;
        wv[c][7] = w1.w;
    }
}

// RMSNorm of the block's activation in registers (reference rms_norm_into,
// src/tensor.rs:969-977; batch association src/tensor.rs:946-954).
// `scratch` holds NT / 64 floats of LDS.
template <int KC, int PRO, int NT = kBlock>
__device__ __forceinline__ void rms_scale(const GemvArgs &a, float (&xv)[KC][8], const float (&wv)[KC][8],
                                          float *scratch) {
    const int t = threadIdx.x;
    float ss[1] = {0.0f};
#pragma unroll
    for (int c = 0; c < KC; c++)
#pragma unroll
        for (int j = 0; j < 8; j++) ss[0] += xv[c][j] * xv[c][j];
    block_sum_n<1, NT / 64>(ss, scratch);
    const float inv = 1.0f / sqrtf(ss[0] / (float)a.in + a.eps);
#pragma unroll
    for (int c = 0; c < KC; c++) {
        const int k = c * NT * 8 + t * 8;
        if (k < a.in) {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                // decode (v*inv)*w; batch v*(inv*w) (src/tensor.rs:975 vs :951)
                if constexpr (PRO == PRO_NORM_BATCH)
                    xv[c][j] = __fmul_rn(xv[c][j], __fmul_rn(inv, wv[c][j]));
                else
                    xv[c][j] = __fmul_rn(__fmul_rn(xv[c][j], inv), wv[c][j]);
            }
        }
    }
}

// Prologue of the layer-0 QKV GEMV: the embedding row of token `tok`
// (src/model.rs:401-403; BF16 rows widen exactly), stored as the residual
// stream by one workgroup, then RMSNorm (rms_norm_into, src/tensor.rs:969-977).
// `scratch` holds NT / 64 floats of LDS.
template <int KC, int NT = kBlock>
__device__ __forceinline__ void gemv_embed_prologue(const GemvArgs &a, int tok, float (&xv)[KC][8], float *scratch,
                                                    bool store_x) {
    const int t = threadIdx.x;
    const int in = a.in;
    if (a.embed_bf16)
        load_act<KC, NT>(nullptr, a.embed_bf16 + (size_t)tok * in, in, xv);
    else
        load_act<KC, NT>(a.embed_f32 + (size_t)tok * in, nullptr, in, xv);
    if (store_x) {
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const int k = c * NT * 8 + t * 8;
            if (k < in)
#pragma unroll
                for (int j = 0; j < 8; j++) a.x_store[k + j] = xv[c][j];
        }
    }
    float wv[KC][8];
    load_norm_w<KC, NT>(a, wv);
    rms_scale<KC, PRO_NORM, NT>(a, xv, wv, scratch);
}

// Epilogue inputs loaded ahead of the weights: the residual of row blk*R+t
// (thread t < R) and the RoPE cos/sin of the block's R/2 rotation pairs.
struct EpiIn {
    float resid;
    // RoPE cos/sin: all R/2 pairs of the block (uniform scalar loads) when
    // R <= 8; with R = 16, entry 0 holds this thread's own pair
    float rc[4], rs[4];
    float sc[2];  // int8 rows: the scales of the thread's epilogue rows
};

__device__ __forceinline__ float pick4(const float (&v)[4], int i) {
    return i == 0 ? v[0] : i == 1 ? v[1] : i == 2 ? v[2] : v[3];
}

// Value of local row i of a block from the NW per-wave partials in `red`:
// the f32 sum ((w0 + w1) + (w2 + w3)) + w4 ... (BF16 and f32 rows), or for
// int8 rows (four waves) the exact integer dot times the activation scale
// and the row scale, y = (dot as f32) * xs * scale[o] (matmul_w_into's
// WMat::I8 arm, src/tensor.rs:349-353).
template <int R, bool Q8, int NW = 4>
__device__ __forceinline__ float row_value(float (*red)[R], int i, float xs, float sc) {
    // the product is rounded before any residual add, as the reference
    // stores y and adds it afterwards (no contraction into an FMA)
#pragma clang fp contract(off)
    if constexpr (Q8) {
        static_assert(NW == 4, "int8 rows run four waves");
        const int d = (__float_as_int(red[0][i]) + __float_as_int(red[1][i])) +
                      (__float_as_int(red[2][i]) + __float_as_int(red[3][i]));
        return ((float)d * xs) * sc;
    } else {
        float v = (red[0][i] + red[1][i]) + (red[2][i] + red[3][i]);
#pragma unroll
        for (int w = 4; w < NW; w++) v += red[w][i];
        return v;
    }
}

// FMAs over a loaded block of BF16 rows and the per-wave reduction into
// `red` (LDS of NT / 64 * R floats).
template <int KC, int R, int NT = kBlock>
__device__ __forceinline__ void gemv_dot(const GemvArgs &a, const WeightRegs<KC, R> &W, const float (&xv)[KC][8],
                                         float (*red)[R]) {
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int c = 0; c < KC; c++) {
            // the clamped loads of a partial last chunk are zeroed (a
            // duplicated Inf or NaN weight would survive a zero activation);
            // the test is uniform, so full chunks keep their registers
            u32x4 u = W.w[r][c];
            if ((c + 1) * NT * 8 > a.in && c * NT * 8 + t * 8 >= a.in) u = u32x4{0u, 0u, 0u, 0u};
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
    constexpr int LR = log2_pow2<R>();  // row i's sum lands in the lanes whose top LR bits are i
    const float sum = multi_wave_sum<R>(acc, lane);
    if ((lane & ((64 >> LR) - 1)) == 0) red[wave][lane >> (6 - LR)] = sum;
}

// The epilogue of a block whose per-wave partials are in `red` (after a
// __syncthreads).  With PRE the residual / RoPE inputs come from `pre`
// instead of memory; with Q8 the rows are int8 (row scales in pre.sc, xs the
// activation scale).
template <int R, int EPI, bool PRE, bool Q8, int NW = 4>
__device__ __forceinline__ void gemv_epilogue(const GemvArgs &a, int blk, int pos, float (*red)[R], const EpiIn &pre,
                                              float xs) {
    const int t = threadIdx.x;
    const int row0 = blk * R;
    if constexpr (EPI == EPI_STORE || EPI == EPI_RESID || EPI == EPI_LOGITS) {
        if (t < R) {
            const int row = row0 + t;
            const float v = row_value<R, Q8, NW>(red, t, xs, pre.sc[0]);
            const bool ok = row < a.out;
            if (ok) {
                if constexpr (EPI == EPI_RESID)
                    a.y[row] = (PRE ? pre.resid : a.y[row]) + v;
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
                    if (t == 0) a.argmax_part[blk] = key;
                }
            }
        }
    } else {
        if (t < R / 2) {
            const int P = row0 / 2 + t;  // global pair index
            const float va = row_value<R, Q8, NW>(red, 2 * t, xs, pre.sc[0]);
            const float vb = row_value<R, Q8, NW>(red, 2 * t + 1, xs, pre.sc[1]);
            if (2 * P + 1 < a.out) {
                if constexpr (EPI == EPI_SWIGLU) {
                    a.y[P] = swiglu(va, vb);
                } else {  // EPI_QKV: pair (j, j + hd/2) of head P / (hd/2)
                    const int half = a.hd >> 1;
                    const int head = P / half, j = P - head * half;
                    const int kvd = a.nkv * a.hd;
                    if (head < a.nq + a.nkv) {
                        float oa, ob;
                        const float rc = !PRE ? a.rope_cos[(size_t)pos * half + j] : R == 16 ? pre.rc[0] : pick4(pre.rc, t);
                        const float rs = !PRE ? a.rope_sin[(size_t)pos * half + j] : R == 16 ? pre.rs[0] : pick4(pre.rs, t);
                        rope_pair(va, vb, rc, rs, &oa, &ob);
                        if (head < a.nq) {
                            a.q_out[head * a.hd + j] = oa;
                            a.q_out[head * a.hd + j + half] = ob;
                        } else {
                            float *kr = a.k_cache + (size_t)pos * kvd + (head - a.nq) * a.hd;
                            kr[j] = oa;
                            kr[j + half] = ob;
                        }
                    } else {
                        float *vr = a.v_cache + (size_t)pos * kvd + (head - a.nq - a.nkv) * a.hd;
                        vr[j] = va;
                        vr[j + half] = vb;
                    }
                }
            }
        }
    }
}

// FMAs over a loaded block, the block reduction and the epilogue.
// `red` is LDS of 4*R floats.  Returns after the epilogue; the caller
// separates consecutive calls with a __syncthreads (red is reused).  With
// PRE the residual / RoPE inputs come from `pre` instead of memory.
template <int KC, int R, int EPI, bool PRE = false, int NT = kBlock>
__device__ __forceinline__ void gemv_finish(const GemvArgs &a, int blk, int pos, const WeightRegs<KC, R> &W,
                                            const float (&xv)[KC][8], float (*red)[R], const EpiIn &pre = EpiIn{}) {
    gemv_dot<KC, R, NT>(a, W, xv, red);
    __syncthreads();
    gemv_epilogue<R, EPI, PRE, false, NT / 64>(a, blk, pos, red, pre, 0.0f);
}

// ---------------------------------------------------------------------------
// f32 rows (WMat::F32: F32 or F16 weight matrices converted to f32 at load,
// reference src/model.rs:49-55; dot_f32_avx2, src/tensor.rs:58-74).  Same
// element mapping as the BF16 rows -- thread t takes elements c*2048 + 8t ..
// +7 of every row -- as two 16-byte loads; fewer rows per workgroup, as each
// row holds twice the registers.
// ---------------------------------------------------------------------------

typedef float f32x4v __attribute__((ext_vector_type(4)));

template <int KC>
__host__ __device__ constexpr int gemv_rows_f32() {
    return KC <= 1 ? 8 : KC <= 3 ? 4 : 2;
}

template <int KC, int R>
struct WeightRegsF {
    f32x4v w[R][KC][2];
};

template <int KC, int R>
__device__ __forceinline__ void gemv_loadf(const GemvArgs &a, int blk, WeightRegsF<KC, R> &W) {
    const int t = threadIdx.x;
    const int row0 = blk * R;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = min(row0 + r, a.out - 1);
        const f32x4v *wr = reinterpret_cast<const f32x4v *>(a.Wf + (size_t)row * a.in);
#pragma unroll
        for (int c = 0; c < KC; c++) {
            // clamped like gemv_load; gemv_dotf zeroes the chunks past the row end
            const int k = min(c * kChunk + t * 8, a.in - 8) >> 2;
            W.w[r][c][0] = __builtin_nontemporal_load(wr + k);
            W.w[r][c][1] = __builtin_nontemporal_load(wr + k + 1);
        }
    }
}

template <int KC, int R>
__device__ __forceinline__ void gemv_dotf(const GemvArgs &a, const WeightRegsF<KC, R> &W, const float (&xv)[KC][8],
                                          float (*red)[R]) {
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int c = 0; c < KC; c++) {
            f32x4v u0 = W.w[r][c][0], u1 = W.w[r][c][1];
            if ((c + 1) * kChunk > a.in && c * kChunk + t * 8 >= a.in) u0 = u1 = f32x4v{0.f, 0.f, 0.f, 0.f};
            s0 = fmaf(xv[c][0], u0.x, s0);
            s1 = fmaf(xv[c][1], u0.y, s1);
            s0 = fmaf(xv[c][2], u0.z, s0);
            s1 = fmaf(xv[c][3], u0.w, s1);
            s0 = fmaf(xv[c][4], u1.x, s0);
            s1 = fmaf(xv[c][5], u1.y, s1);
            s0 = fmaf(xv[c][6], u1.z, s0);
            s1 = fmaf(xv[c][7], u1.w, s1);
        }
        acc[r] = s0 + s1;
    }
    constexpr int LR = log2_pow2<R>();  // row i's sum lands in the lanes whose top LR bits are i
    const float sum = multi_wave_sum<R>(acc, lane);
    if ((lane & ((64 >> LR) - 1)) == 0) red[wave][lane >> (6 - LR)] = sum;
}

// ---------------------------------------------------------------------------
// int8 rows (the TMG_I8 weight-only mode, reference src/model.rs:57-76):
// W8 [out, in] int8 with one f32 scale per row.  Same element mapping as the
// BF16 rows -- thread t takes elements c*2048 + 8t .. +7 of every row -- with
// 8-byte loads.  The activation is quantized like quantize_row_i8
// (src/tensor.rs:125-139) by every workgroup from the registers it already
// holds, and the dots are exact int32 v_dot4_i32_i8 sums, as dot_i8's i16
// madd sums are (src/tensor.rs:144-170).
// ---------------------------------------------------------------------------

// Rows per workgroup of the int8 GEMV: every workgroup reads the whole
// activation (and, with a fused RMSNorm, the norm weights) and reduces it
// twice, so at 1 byte per weight a normalizing single-chunk GEMV takes 16
// rows to keep that per-workgroup cost small against its weight bytes.
template <int KC, int PRO>
__host__ __device__ constexpr int gemv_rows8() {
    return (KC == 1 && (PRO == PRO_NORM || PRO == PRO_EMBED_NORM)) ? 16 : gemv_rows<KC>();
}

template <int KC, int R>
struct WeightRegs8 {
    u32x2 w[R][KC];
};

template <int KC, int R>
__device__ __forceinline__ void gemv_load8(const GemvArgs &a, int blk, WeightRegs8<KC, R> &W) {
    const int t = threadIdx.x;
    const int row0 = blk * R;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = min(row0 + r, a.out - 1);
        const u32x2 *wr = reinterpret_cast<const u32x2 *>(a.W8 + (size_t)row * a.in);
#pragma unroll
        for (int c = 0; c < KC; c++) {
            // clamped like gemv_load; the activation codes past the row end
            // are zero, so those lanes add nothing
            const int k = c * kChunk + t * 8;
            W.w[r][c] = __builtin_nontemporal_load(wr + (min(k, a.in - 8) >> 3));
        }
    }
}

// Scales of the rows this thread's epilogue writes: row blk*R + t (t < R), or
// the pair 2t, 2t+1 (t < R/2) for the pair epilogues.
template <int R, int EPI>
__device__ __forceinline__ void epi_issue_scale(const GemvArgs &a, int blk, EpiIn &pre) {
    const int t = threadIdx.x;
    const int row0 = blk * R;
    pre.sc[0] = pre.sc[1] = 0.0f;
    if constexpr (EPI == EPI_SWIGLU || EPI == EPI_QKV) {
        const int r = row0 + 2 * t;
        if (t < R / 2 && r + 1 < a.out) {
            const float2 v = *reinterpret_cast<const float2 *>(a.wscale + r);
            pre.sc[0] = v.x;
            pre.sc[1] = v.y;
        }
    } else {
        const int r = row0 + t;
        if (t < R && r < a.out) pre.sc[0] = a.wscale[r];
    }
}

// round(a * b) with the product rounded to f32 first, as the reference
// computes (x * inv).round(): the subtraction inside round() is not allowed
// to fuse with the multiply.
__device__ __forceinline__ float round_product(float a, float b) {
#pragma clang fp contract(off)
    const float p = a * b;
    return roundf(p);
}

// quantize_row_i8 of the activation held in registers: xs = max|x| / 127,
// q = round(x * (1 / xs)) (half away from zero) clamped to [-127, 127], four
// codes per int; an all-zero vector gives zero codes and xs = 0.  Every
// thread returns xs.  `scratch` holds 4 floats of LDS.
template <int KC>
__device__ __forceinline__ float quantize_act(const float (&xv)[KC][8], int (&xq)[KC][2], float *scratch) {
    float m[1] = {0.0f};
#pragma unroll
    for (int c = 0; c < KC; c++)
#pragma unroll
        for (int j = 0; j < 8; j++) m[0] = fmaxf(fabsf(xv[c][j]), m[0]);
    block_max_n<1>(m, scratch);
    const float maxabs = m[0];
    const float s = __fdiv_rn(maxabs, 127.0f);
    const float inv = maxabs == 0.0f ? 0.0f : __fdiv_rn(1.0f, s);
#pragma unroll
    for (int c = 0; c < KC; c++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint32_t packed = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float r = round_product(xv[c][4 * h + j], inv);
                // `as i8` after clamp: NaN becomes 0
                const int q = r == r ? (int)fminf(fmaxf(r, -127.0f), 127.0f) : 0;
                packed |= ((uint32_t)q & 0xffu) << (8 * j);
            }
            xq[c][h] = (int)packed;
        }
    return maxabs == 0.0f ? 0.0f : s;
}

// Exact integer dots of a loaded int8 block and the per-wave reduction into
// `red` (int32 bit patterns in LDS of 4*R floats).
template <int KC, int R>
__device__ __forceinline__ void gemv_dot8(const WeightRegs8<KC, R> &W, const int (&xq)[KC][2], float (*red)[R]) {
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    int acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        int d = 0;
#pragma unroll
        for (int c = 0; c < KC; c++) {
            d = __builtin_amdgcn_sdot4(xq[c][0], (int)W.w[r][c].x, d, false);
            d = __builtin_amdgcn_sdot4(xq[c][1], (int)W.w[r][c].y, d, false);
        }
        acc[r] = d;
    }
    constexpr int LR = log2_pow2<R>();  // row i's sum lands in the lanes whose top LR bits are i
    const int sum = multi_wave_sum<R>(acc, lane);
    if ((lane & ((64 >> LR) - 1)) == 0) red[wave][lane >> (6 - LR)] = __int_as_float(sum);
}

// ---------------------------------------------------------------------------
// Load order of the standalone decode GEMV.  Vector loads of a wavefront
// complete in issue order, so an activation loaded after the weights could
// only be used once every weight load had arrived.  The kernels therefore
// issue the activation-side loads (x and the norm weights, or the split-K
// attention partials, and the residual) first, then the weights, and run the
// prologue (RMSNorm reduction, split merge) while the weights stream in.
// ---------------------------------------------------------------------------

template <int KC, int PRO>
struct ActIn {
    static constexpr bool kAttn = PRO == PRO_ATTN_COMBINE;
    static constexpr bool kNorm = PRO == PRO_NORM || PRO == PRO_NORM_BATCH;
    static constexpr int NS = kAttn ? kFusedSplits : 1;
    float xv[KC][8];
    float wv[kNorm ? KC : 1][8];
    float2 ml[kAttn ? KC : 1][NS];
    float4 o[kAttn ? KC : 1][NS][2];
};

// PRO in {PLAIN, NORM, NORM_BATCH, ATTN_COMBINE}; ATTN_COMBINE requires
// a.nsplit <= kFusedSplits.
template <int KC, int PRO, int NT = kBlock>
__device__ __forceinline__ void act_issue(const GemvArgs &a, ActIn<KC, PRO> &in) {
    const int t = threadIdx.x;
    if constexpr (PRO == PRO_ATTN_COMBINE) {
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const int k = c * NT * 8 + t * 8;
            const bool ok = k < a.in;
            const int h = k / a.hd, d = k - h * a.hd;
            const int g = h / a.group, hq = h - g * a.group;
            const size_t base = (size_t)g * a.nsplit * a.group + hq;
#pragma unroll
            for (int sp = 0; sp < kFusedSplits; sp++) {
                const size_t pi = base + (size_t)sp * a.group;
                if (ok && sp < a.nsplit) {
                    in.ml[c][sp] = *reinterpret_cast<const float2 *>(a.part_ml + pi * 2);
                    in.o[c][sp][0] = *reinterpret_cast<const float4 *>(a.part + pi * a.hd + d);
                    in.o[c][sp][1] = *reinterpret_cast<const float4 *>(a.part + pi * a.hd + d + 4);
                } else {
                    in.ml[c][sp] = make_float2(-INFINITY, 0.0f);
                    in.o[c][sp][0] = in.o[c][sp][1] = make_float4(0.f, 0.f, 0.f, 0.f);
                }
            }
        }
    } else {
        load_act<KC, NT>(a.x, nullptr, a.in, in.xv);
        if constexpr (ActIn<KC, PRO>::kNorm) load_norm_w<KC, NT>(a, in.wv);
    }
}

// The prologue's arithmetic: the split merge, or the copy of x and its RMSNorm.
template <int KC, int PRO, int NT = kBlock>
__device__ __forceinline__ void act_finish(const GemvArgs &a, int pos, ActIn<KC, PRO> &in, float (&xv)[KC][8],
                                           float *scratch) {
    const int t = threadIdx.x;
    if constexpr (PRO == PRO_ATTN_COMBINE) {
        const int active = active_splits(pos + 1, a.nsplit, a.attn_block);
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const int k = c * NT * 8 + t * 8;
#pragma unroll
            for (int j = 0; j < 8; j++) xv[c][j] = 0.0f;
            if (k >= a.in) continue;
            float M = -INFINITY;
#pragma unroll
            for (int sp = 0; sp < kFusedSplits; sp++)
                if (sp < active) M = fmaxf(M, in.ml[c][sp].x);
            float L = 0.0f;
#pragma unroll
            for (int sp = 0; sp < kFusedSplits; sp++) {
                if (sp >= active) continue;
                const float m = in.ml[c][sp].x;
                const float w = (m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - M);
                L = fmaf(in.ml[c][sp].y, w, L);
                const float4 o0 = in.o[c][sp][0], o1 = in.o[c][sp][1];
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
    } else {
#pragma unroll
        for (int c = 0; c < KC; c++)
#pragma unroll
            for (int j = 0; j < 8; j++) xv[c][j] = in.xv[c][j];
        if constexpr (ActIn<KC, PRO>::kNorm) rms_scale<KC, PRO, NT>(a, xv, in.wv, scratch);
    }
}

// Residual rows of block blk (issued before the weights).
template <int R>
__device__ __forceinline__ void epi_issue_resid(const GemvArgs &a, int blk, EpiIn &pre) {
    const int t = threadIdx.x;
    pre.resid = 0.0f;
    if (t < R) {
        const int row = blk * R + t;
        if (row < a.out) pre.resid = a.y[row];
    }
}

// RoPE cos/sin of the block's pairs at position pos: the R/2 pairs of a block
// are consecutive frequencies of one head (hd/2 is a multiple of R/2), so the
// addresses are uniform over the workgroup.
template <int R>
__device__ __forceinline__ void epi_load_rope(const GemvArgs &a, int blk, int pos, EpiIn &pre) {
    const int half = a.hd >> 1;
    const int P0 = (blk * R) >> 1;
    const int j0 = P0 - (P0 / half) * half;
    const float *cb = a.rope_cos + (size_t)pos * half + j0;
    const float *sb = a.rope_sin + (size_t)pos * half + j0;
    if constexpr (R == 16) {
        // eight pairs: one vector load per thread; eight scalar pairs and a
        // per-thread select would be kept in LDS by the compiler
        const int t = threadIdx.x;
        pre.rc[0] = t < 8 ? cb[t] : 0.0f;
        pre.rs[0] = t < 8 ? sb[t] : 0.0f;
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            pre.rc[i] = i < R / 2 ? cb[i] : 0.0f;
            pre.rs[i] = i < R / 2 ? sb[i] : 0.0f;
        }
        // pin the (scalar) loads here rather than letting them sink into the
        // epilogue, where their latency would add to the kernel's tail
#pragma unroll
        for (int i = 0; i < 4; i++) asm volatile("" ::"s"(pre.rc[i]), "s"(pre.rs[i]));
    }
}

// ---------------------------------------------------------------------------
// Several activation rows per launch (batched decode of up to kMtMaxSeq
// sequences).  A workgroup loads its R weight rows once (as gemv_load does)
// and walks the sequences in groups of TG: per group it loads the TG
// activation rows (KC chunks of 8 per thread each), applies each row's
// RMSNorm (forward_token's (v*inv)*w), forms the R*TG dots, reduces them in
// one transposed butterfly, and runs the epilogue per (row, sequence).
// ---------------------------------------------------------------------------

// Activation rows per group: 2 for two sequences; rows of one chunk take
// all of five to eight sequences in one group (one load round trip, one norm
// and one dot reduction per launch; 8 sequences of the 1B model 1.537 ->
// 1.518 ms per step); else 4 (2 above three chunks).  Activation registers
// TG * KC * 8.
__host__ __device__ constexpr int gemv_mt_group(int KC, int nb) {
    return (nb <= 2 || KC > 3) ? 2 : (KC == 1 && nb > 4) ? 8 : 4;
}
// Rows per workgroup: every workgroup reads each group's activation rows
// from L2, so more rows per workgroup mean fewer re-reads per weight byte;
// R * TG dots stay within 32 (registers, and two waves per SIMD), 64 for a
// group of eight over one chunk (4 rows there were slower: 1.71 ms).
__host__ __device__ constexpr int gemv_mt_rows(int KC, int TG) {
    return KC == 1 ? (TG == 8 ? 8 : 32 / TG) : KC <= 3 ? 16 / TG : 4;
}

// Raw loads of activation rows b0 .. b0+TG-1 (zeros past a.nb).
template <int KC, int TG>
__device__ __forceinline__ void mt_issue(const GemvArgs &a, int b0, float (&xv)[TG][KC][8]) {
    const int t = threadIdx.x;
#pragma unroll
    for (int u = 0; u < TG; u++) {
        const bool live = b0 + u < a.nb;
        const float *src = a.x + (size_t)(live ? b0 + u : 0) * a.in;
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const int k = c * kChunk + t * 8;
            if (live && k < a.in) {
                const float4 p = *reinterpret_cast<const float4 *>(src + k);
                const float4 q = *reinterpret_cast<const float4 *>(src + k + 4);
                xv[u][c][0] = p.x;
                xv[u][c][1] = p.y;
                xv[u][c][2] = p.z;
                xv[u][c][3] = p.w;
                xv[u][c][4] = q.x;
                xv[u][c][5] = q.y;
                xv[u][c][6] = q.z;
                xv[u][c][7] = q.w;
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) xv[u][c][j] = 0.0f;
            }
        }
    }
}

// Each row's RMSNorm (PRO_NORM); `scratch` holds 4*TG floats of LDS.
template <int KC, int TG, int PRO>
__device__ __forceinline__ void mt_norm(const GemvArgs &a, const float (&wv)[KC][8], float (&xv)[TG][KC][8],
                                        float *scratch) {
    if constexpr (PRO == PRO_NORM) {
        float ss[TG];
#pragma unroll
        for (int u = 0; u < TG; u++) {
            ss[u] = 0.0f;
#pragma unroll
            for (int c = 0; c < KC; c++)
#pragma unroll
                for (int j = 0; j < 8; j++) ss[u] += xv[u][c][j] * xv[u][c][j];
        }
        block_sum_n<TG>(ss, scratch);
#pragma unroll
        for (int u = 0; u < TG; u++) {
            const float inv = 1.0f / sqrtf(ss[u] / (float)a.in + a.eps);
#pragma unroll
            for (int c = 0; c < KC; c++)
#pragma unroll
                for (int j = 0; j < 8; j++) xv[u][c][j] = (xv[u][c][j] * inv) * wv[c][j];
        }
    }
}

// Dots of the R loaded rows with the TG activation rows, reduced into
// red[wave][r * TG + u].
template <int KC, int R, int TG>
__device__ __forceinline__ void mt_dot(const GemvArgs &a, const WeightRegs<KC, R> &W, const float (&xv)[TG][KC][8],
                                       float (*red)[R * TG]) {
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    float acc[R * TG];
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
        for (int u = 0; u < TG; u++) {
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int c = 0; c < KC; c++) {
                const u32x4 w = (c * kChunk + t * 8 < a.in) ? W.w[r][c] : u32x4{0u, 0u, 0u, 0u};
                s0 = fmaf(xv[u][c][0], bf16_lo(w.x), s0);
                s1 = fmaf(xv[u][c][1], bf16_hi(w.x), s1);
                s0 = fmaf(xv[u][c][2], bf16_lo(w.y), s0);
                s1 = fmaf(xv[u][c][3], bf16_hi(w.y), s1);
                s0 = fmaf(xv[u][c][4], bf16_lo(w.z), s0);
                s1 = fmaf(xv[u][c][5], bf16_hi(w.z), s1);
                s0 = fmaf(xv[u][c][6], bf16_lo(w.w), s0);
                s1 = fmaf(xv[u][c][7], bf16_hi(w.w), s1);
            }
            acc[r * TG + u] = s0 + s1;
        }
    }
    constexpr int N = R * TG;
    constexpr int LN = log2_pow2<N>();
    const float sum = multi_wave_sum<N>(acc, lane);
    if ((lane & ((64 >> LN) - 1)) == 0) red[wave][lane >> (6 - LN)] = sum;
}

// Epilogue of sequences b0 .. b0+TG-1 (those below a.nb) for block blk.
// LOGITS: argmax key of the block's rows per sequence.
template <int R, int TG, int EPI>
__device__ __forceinline__ void mt_epilogue(const GemvArgs &a, int blk, int b0, float (*red)[R * TG]) {
    const int t = threadIdx.x;
    const int row0 = blk * R;
    auto val = [&](int r, int u) {
        const int i = r * TG + u;
        return (red[0][i] + red[1][i]) + (red[2][i] + red[3][i]);
    };
    if constexpr (EPI == EPI_RESID) {
        if (t < R * TG) {
            const int r = t / TG, u = t % TG, row = row0 + r, b = b0 + u;
            if (row < a.out && b < a.nb) {
                float *y = a.y + (size_t)b * a.out + row;
                *y = *y + val(r, u);
            }
        }
    } else if constexpr (EPI == EPI_LOGITS) {
        if (t < TG) {
            const int b = b0 + t;
            unsigned long long key = 0ull;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float v = val(r, t);
                const int row = row0 + r;
                if (row < a.out && v == v) {
                    const unsigned long long k = argmax_key(v, (uint32_t)row);
                    key = k > key ? k : key;
                }
            }
            if (b < a.nb) a.argmax_part[(size_t)b * gridDim.x + blk] = key;
        }
    } else {
        if (t < (R / 2) * TG) {
            const int pr = t / TG, u = t % TG, b = b0 + u;
            const int P = row0 / 2 + pr;
            if (2 * P + 1 < a.out && b < a.nb) {
                const float va = val(2 * pr, u), vb = val(2 * pr + 1, u);
                if constexpr (EPI == EPI_SWIGLU) {
                    a.y[(size_t)b * (a.out / 2) + P] = swiglu(va, vb);
                } else {  // EPI_QKV
                    const int half = a.hd >> 1;
                    const int head = P / half, j = P - head * half;
                    const int kvd = a.nkv * a.hd;
                    const int pos = a.pos_seq[b];
                    if (head < a.nq + a.nkv) {
                        float oa, ob;
                        rope_pair(va, vb, a.rope_cos[(size_t)pos * half + j], a.rope_sin[(size_t)pos * half + j],
                                  &oa, &ob);
                        if (head < a.nq) {
                            float *q = a.q_out + (size_t)b * a.nq * a.hd + head * a.hd;
                            q[j] = oa;
                            q[j + half] = ob;
                        } else {
                            float *kr = a.k_seq[b] + a.kv_layer_off + (size_t)pos * kvd + (head - a.nq) * a.hd;
                            kr[j] = oa;
                            kr[j + half] = ob;
                        }
                    } else {
                        float *vr = a.v_seq[b] + a.kv_layer_off + (size_t)pos * kvd + (head - a.nq - a.nkv) * a.hd;
                        vr[j] = va;
                        vr[j + half] = vb;
                    }
                }
            }
        }
    }
}

}  // namespace tmg
