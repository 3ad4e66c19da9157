// Decode-step kernels for gfx950: the fused BF16 GEMV, split-K GQA
// attention and the step finalizer.
//
// GEMV (reference matmul_w_into, src/tensor.rs:331-460, hot loop
// dot_bf16_avx2 at src/tensor.rs:78-96): one 256-thread workgroup owns R
// output rows and covers the whole input dimension, each thread streaming
// 16 B (8 BF16) per 2048-element chunk of every row.  A wavefront load is one
// contiguous 1 KiB segment of a row, the activation stays in registers, all
// R*KC row loads are issued before the FMAs, and the per-row reduction is a
// transposed DPP/shuffle butterfly followed by a 4-way LDS sum.  Prologues
// fuse the RMSNorm (reference rms_norm_into, src/tensor.rs:969-977) or the
// embedding gather; epilogues fuse the residual add, SwiGLU, RoPE + KV-cache
// append, or logits + a running argmax.
#include "common.cuh"
#include "kernels.hpp"

namespace tmg {
namespace {

constexpr int kChunk = kBlock * 8;  // elements per chunk: 8 per thread
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int KC>
__device__ __forceinline__ void load_act(const float *src, const uint16_t *src_bf, int in, int t,
                                         float (&xv)[KC][8]) {
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
                const float4 a = *reinterpret_cast<const float4 *>(src + k);
                const float4 b = *reinterpret_cast<const float4 *>(src + k + 4);
                xv[c][0] = a.x;
                xv[c][1] = a.y;
                xv[c][2] = a.z;
                xv[c][3] = a.w;
                xv[c][4] = b.x;
                xv[c][5] = b.y;
                xv[c][6] = b.z;
                xv[c][7] = b.w;
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
template <int KC>
__device__ __forceinline__ void load_attn(const GemvArgs &a, int t, float (&xv)[KC][8]) {
    const int n_ctx = *a.pos + 1;
    const int active = active_splits(n_ctx, a.nsplit, a.min_chunk);
#pragma unroll
    for (int c = 0; c < KC; c++) {
        const int k = c * kChunk + t * 8;
#pragma unroll
        for (int j = 0; j < 8; j++) xv[c][j] = 0.0f;
        if (k >= a.in) continue;
        const int h = k / a.hd, d = k - h * a.hd;
        const int g = h / a.group, hq = h - g * a.group;
        const size_t base = (size_t)g * a.nsplit * a.group + hq;  // + s * group
        float M = -INFINITY;
        for (int sp = 0; sp < active; sp++) M = fmaxf(M, a.part_ml[(base + (size_t)sp * a.group) * 2]);
        float L = 0.0f;
        for (int sp = 0; sp < active; sp++) {
            const size_t pi = base + (size_t)sp * a.group;
            const float m = a.part_ml[pi * 2];
            const float w = (m == -INFINITY) ? 0.0f : expf(m - M);
            L = fmaf(a.part_ml[pi * 2 + 1], w, L);
            const float4 o0 = *reinterpret_cast<const float4 *>(a.part + pi * a.hd + d);
            const float4 o1 = *reinterpret_cast<const float4 *>(a.part + pi * a.hd + d + 4);
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

template <int KC, int R, int PRO, int EPI>
__global__ __launch_bounds__(kBlock) void gemv_kernel(const GemvArgs a) {
    __shared__ float red[4][R];
    __shared__ float scratch[4];
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int in = a.in;

    // ---- prologue: activation into registers ------------------------------
    float xv[KC][8];
    const float *src = a.x;
    const uint16_t *src_bf = nullptr;
    if constexpr (PRO == PRO_EMBED_NORM) {
        const int tok = *a.token;
        if (a.embed_bf16) {
            src_bf = a.embed_bf16 + (size_t)tok * in;
        } else {
            src = a.embed_f32 + (size_t)tok * in;
        }
    }
    if constexpr (PRO == PRO_ATTN_COMBINE) {
        load_attn<KC>(a, t, xv);
    } else {
        load_act<KC>(src, src_bf, in, t, xv);
    }
    if constexpr (PRO == PRO_EMBED_NORM) {
        if (blockIdx.x == 0) {
#pragma unroll
            for (int c = 0; c < KC; c++) {
                const int k = c * kChunk + t * 8;
                if (k < in) {
                    *reinterpret_cast<float4 *>(a.x_store + k) = make_float4(xv[c][0], xv[c][1], xv[c][2], xv[c][3]);
                    *reinterpret_cast<float4 *>(a.x_store + k + 4) =
                        make_float4(xv[c][4], xv[c][5], xv[c][6], xv[c][7]);
                }
            }
        }
    }
    if constexpr (PRO != PRO_PLAIN && PRO != PRO_ATTN_COMBINE) {
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
                    // decode: (v*inv)*w; batch (prefill): v*(inv*w) -- the
                    // reference's two associations (src/tensor.rs:951, :975)
                    if constexpr (PRO == PRO_NORM_BATCH)
                        xv[c][j] = __fmul_rn(xv[c][j], __fmul_rn(inv, w[j]));
                    else
                        xv[c][j] = __fmul_rn(__fmul_rn(xv[c][j], inv), w[j]);
                }
            }
        }
    }

    // ---- main loop: issue every row load, then the FMAs --------------------
    const int row0 = blockIdx.x * R;
    u32x4 wv[R][KC];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = min(row0 + r, a.out - 1);
        const u32x4 *wr = reinterpret_cast<const u32x4 *>(a.W + (size_t)row * in);
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const int k = c * kChunk + t * 8;
            wv[r][c] = (k < in) ? __builtin_nontemporal_load(wr + (k >> 3)) : u32x4{0u, 0u, 0u, 0u};
        }
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int c = 0; c < KC; c++) {
            const u32x4 u = wv[r][c];
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

    // ---- reduction --------------------------------------------------------
    {
        constexpr int LR = R == 8 ? 3 : R == 4 ? 2 : R == 2 ? 1 : 0;
        const float s = multi_wave_sum<R>(acc, lane);
        if ((lane & ((64 >> LR) - 1)) == 0) red[wave][lane >> (6 - LR)] = s;
    }
    __syncthreads();

    // ---- epilogue ---------------------------------------------------------
    if constexpr (EPI == EPI_STORE || EPI == EPI_RESID || EPI == EPI_LOGITS) {
        if (t < R) {
            const int row = row0 + t;
            const float v = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
            const bool ok = row < a.out;
            if (ok) {
                if constexpr (EPI == EPI_RESID)
                    a.y[row] += v;
                else
                    a.y[row] = v;
            }
            if constexpr (EPI == EPI_LOGITS) {
                if (a.argmax_part) {
                    unsigned long long key = (ok && v == v) ? argmax_key(v, (uint32_t)row) : 0ull;
#pragma unroll
                    for (int off = R / 2; off > 0; off >>= 1) {
                        const unsigned long long o = shfl_xor_u64(key, off);
                        key = o > key ? o : key;
                    }
                    if (t == 0) a.argmax_part[blockIdx.x] = key;
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
                    a.y[P] = swiglu(va, vb);
                } else {  // EPI_QKV: pair (j, j + hd/2) of head P / (hd/2)
                    const int half = a.hd >> 1;
                    const int head = P / half, j = P - head * half;
                    const int pos = *a.pos;
                    const int kvd = a.nkv * a.hd;
                    if (head < a.nq + a.nkv) {
                        float oa, ob;
                        rope_pair(va, vb, a.rope_cos[(size_t)pos * half + j], a.rope_sin[(size_t)pos * half + j], &oa,
                                  &ob);
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

template <int KC, int PRO, int EPI>
hipError_t launch_kc(const GemvArgs &a, hipStream_t s) {
    constexpr int R = KC <= 2 ? 8 : 4;
    const int grid = (a.out + R - 1) / R;
    hipLaunchKernelGGL((gemv_kernel<KC, R, PRO, EPI>), dim3(grid), dim3(kBlock), 0, s, a);
    return hipGetLastError();
}

template <int PRO, int EPI>
hipError_t launch_pe(const GemvArgs &a, hipStream_t s) {
    const int kc = (a.in + kChunk - 1) / kChunk;
    switch (kc) {
        case 1: return launch_kc<1, PRO, EPI>(a, s);
        case 2: return launch_kc<2, PRO, EPI>(a, s);
        case 3: return launch_kc<3, PRO, EPI>(a, s);
        case 4: return launch_kc<4, PRO, EPI>(a, s);
        case 5: return launch_kc<5, PRO, EPI>(a, s);
        case 6: return launch_kc<6, PRO, EPI>(a, s);
        case 8:
        case 7: return launch_kc<8, PRO, EPI>(a, s);
        default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------------------
// Attention (reference: decode src/model.rs:434-459; prefill attention_batch
// src/tensor.rs:1099-1139; softmax src/tensor.rs:1055-1060).
//
// Grid (nsplit, nkv, T).  A workgroup owns one KV head and one slice of the
// positions of one query row, and serves all `GROUP` query heads of that KV
// head from each K/V load.  Positions are processed in LDS chunks of 256 with
// a running (max, sum) rescale.  A row covered by one split is written out
// directly; otherwise every split writes (o, max, sum) partials that are merged
// after the kernel boundary, which also publishes them across the XCDs' L2s
// without any in-kernel fence.
// ---------------------------------------------------------------------------

template <int HD, int GROUP>
__global__ __launch_bounds__(kBlock) void attn_kernel(const AttnArgs a) {
    constexpr int TS = HD / 4;            // lanes per position, float4 each
    constexpr int NTEAM = kBlock / TS;    // positions in flight per block
    constexpr int CH = 256;               // positions per LDS chunk
    __shared__ float s_p[GROUP][CH];
    __shared__ float s_red[NTEAM][GROUP][HD];
    __shared__ float scratch[4 * GROUP];

    const int split = blockIdx.x, g = blockIdx.y, ti = blockIdx.z;
    const int t = threadIdx.x, lt = t % TS, team = t / TS;
    const int qpos = (a.pos_dev ? *a.pos_dev : a.start) + ti;
    const int n_ctx = qpos + 1;
    const int active = active_splits(n_ctx, a.nsplit, a.min_chunk);
    if (split >= active) return;
    const int chunk = (n_ctx + active - 1) / active;
    const int t0 = split * chunk, t1 = min(n_ctx, t0 + chunk);
    const int kvd = a.nkv * HD;
    const int qd = a.nq * HD;
    const float *kbase = a.k_cache + g * HD + lt * 4;
    const float *vbase = a.v_cache + g * HD + lt * 4;

    float4 qv[GROUP];
    const float *qrow = a.q + (size_t)ti * qd;
#pragma unroll
    for (int h = 0; h < GROUP; h++) qv[h] = *reinterpret_cast<const float4 *>(qrow + (g * GROUP + h) * HD + lt * 4);

    float m_run[GROUP], l_run[GROUP];
    float4 o_acc[GROUP];
#pragma unroll
    for (int h = 0; h < GROUP; h++) {
        m_run[h] = -INFINITY;
        l_run[h] = 0.0f;
        o_acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
    }

    for (int c0 = t0; c0 < t1; c0 += CH) {
        const int n = min(CH, t1 - c0);
        // scores s = (q . k) * scale
        for (int i = team; i < n; i += NTEAM) {
            const float4 k = *reinterpret_cast<const float4 *>(kbase + (size_t)(c0 + i) * kvd);
#pragma unroll
            for (int h = 0; h < GROUP; h++) {
                float d = qv[h].x * k.x;
                d = fmaf(qv[h].y, k.y, d);
                d = fmaf(qv[h].z, k.z, d);
                d = fmaf(qv[h].w, k.w, d);
                d = group_sum<TS>(d);
                if (lt == 0) s_p[h][i] = d * a.scale;
            }
        }
        __syncthreads();
        float mx[GROUP];
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            mx[h] = -INFINITY;
            for (int i = t; i < n; i += kBlock) mx[h] = fmaxf(mx[h], s_p[h][i]);
        }
        block_max_n<GROUP>(mx, scratch);
        float sm[GROUP], corr[GROUP];
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            const float m_new = fmaxf(m_run[h], mx[h]);
            corr[h] = (m_run[h] == -INFINITY) ? 0.0f : expf(m_run[h] - m_new);
            m_run[h] = m_new;
            sm[h] = 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < GROUP; h++)
            for (int i = t; i < n; i += kBlock) {
                const float p = expf(s_p[h][i] - m_run[h]);
                s_p[h][i] = p;
                sm[h] += p;
            }
        block_sum_n<GROUP>(sm, scratch);
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            l_run[h] = l_run[h] * corr[h] + sm[h];
            o_acc[h].x *= corr[h];
            o_acc[h].y *= corr[h];
            o_acc[h].z *= corr[h];
            o_acc[h].w *= corr[h];
        }
        // o += p * v
        for (int i = team; i < n; i += NTEAM) {
            const float4 v = *reinterpret_cast<const float4 *>(vbase + (size_t)(c0 + i) * kvd);
#pragma unroll
            for (int h = 0; h < GROUP; h++) {
                const float p = s_p[h][i];
                o_acc[h].x = fmaf(p, v.x, o_acc[h].x);
                o_acc[h].y = fmaf(p, v.y, o_acc[h].y);
                o_acc[h].z = fmaf(p, v.z, o_acc[h].z);
                o_acc[h].w = fmaf(p, v.w, o_acc[h].w);
            }
        }
        __syncthreads();
    }

    // reduce the per-team partial outputs
#pragma unroll
    for (int h = 0; h < GROUP; h++) *reinterpret_cast<float4 *>(&s_red[team][h][lt * 4]) = o_acc[h];
    __syncthreads();
    float o_fin[(GROUP * HD + kBlock - 1) / kBlock];
#pragma unroll
    for (int e = 0; e < (GROUP * HD + kBlock - 1) / kBlock; e++) {
        const int idx = t + e * kBlock;
        float s = 0.0f;
        if (idx < GROUP * HD) {
            const int h = idx / HD, d = idx % HD;
            for (int tm = 0; tm < NTEAM; tm++) s += s_red[tm][h][d];
        }
        o_fin[e] = s;
    }

    const size_t row_hd = (size_t)ti * qd + g * GROUP * HD;
    if (active == 1 && (a.out_f32 || a.out_hi)) {
#pragma unroll
        for (int e = 0; e < (GROUP * HD + kBlock - 1) / kBlock; e++) {
            const int idx = t + e * kBlock;
            if (idx < GROUP * HD) {
                const float o = o_fin[e] / l_run[idx / HD];
                if (a.out_f32) a.out_f32[row_hd + idx] = o;
                if (a.out_hi) split_bf16(o, a.out_hi + row_hd + idx, a.out_lo + row_hd + idx);
            }
        }
        return;
    }

    // publish this split's partial; the merge runs after the kernel boundary
    // (fused into the o_proj GEMV prologue, or attn_combine_kernel)
    const size_t pbase = (((size_t)ti * a.nkv + g) * a.nsplit + split) * GROUP;
#pragma unroll
    for (int e = 0; e < (GROUP * HD + kBlock - 1) / kBlock; e++) {
        const int idx = t + e * kBlock;
        if (idx < GROUP * HD) a.part[pbase * HD + idx] = o_fin[e];
    }
    if (t < GROUP) {
        a.part_ml[(pbase + t) * 2 + 0] = m_run[t];
        a.part_ml[(pbase + t) * 2 + 1] = l_run[t];
    }
}

// One thread per (query head, dim) of decode row 0.
__global__ __launch_bounds__(kBlock) void attn_combine_kernel(const AttnArgs a) {
    const int idx = blockIdx.x * kBlock + threadIdx.x;
    if (idx >= a.nq * a.hd) return;
    const int group = a.nq / a.nkv;
    const int h = idx / a.hd, d = idx - h * a.hd;
    const int g = h / group, hq = h - g * group;
    const int n_ctx = *a.pos_dev + 1;
    const int active = active_splits(n_ctx, a.nsplit, a.min_chunk);
    const size_t base = (size_t)g * a.nsplit * group + hq;
    float M = -INFINITY;
    for (int sp = 0; sp < active; sp++) M = fmaxf(M, a.part_ml[(base + (size_t)sp * group) * 2]);
    float L = 0.0f, O = 0.0f;
    for (int sp = 0; sp < active; sp++) {
        const size_t pi = base + (size_t)sp * group;
        const float m = a.part_ml[pi * 2];
        const float w = (m == -INFINITY) ? 0.0f : expf(m - M);
        L = fmaf(a.part_ml[pi * 2 + 1], w, L);
        O = fmaf(a.part[pi * a.hd + d], w, O);
    }
    a.out_f32[idx] = O / L;
}

template <int HD>
hipError_t launch_attn_hd(const AttnArgs &a, hipStream_t s) {
    const dim3 grid(a.nsplit, a.nkv, a.T);
    switch (a.nq / a.nkv) {
        case 1: hipLaunchKernelGGL((attn_kernel<HD, 1>), grid, dim3(kBlock), 0, s, a); break;
        case 2: hipLaunchKernelGGL((attn_kernel<HD, 2>), grid, dim3(kBlock), 0, s, a); break;
        case 4: hipLaunchKernelGGL((attn_kernel<HD, 4>), grid, dim3(kBlock), 0, s, a); break;
        case 8: hipLaunchKernelGGL((attn_kernel<HD, 8>), grid, dim3(kBlock), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Step finalizer: the argmax of the step's logits becomes the next input
// token (generate's `next = argmax(logits)`, src/model.rs:636-637), is
// appended to the history, and the cache position advances.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(1024) void finalize_kernel(const FinalizeArgs a) {
    __shared__ unsigned long long red[16];
    unsigned long long best = kArgmaxInit;
    for (int i = threadIdx.x; i < a.nparts; i += blockDim.x) {
        const unsigned long long k = a.argmax_part[i];
        best = k > best ? k : best;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = shfl_xor_u64(best, off);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) best = red[w] > best ? red[w] : best;
    DevState *st = a.st;
    const unsigned long long key = best;
    int tok = (int)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull));
    if (tok < 0 || tok >= a.V) tok = 0;
    st->cur_token = tok;
    a.history[st->step] = tok;
    st->step = st->step + 1;
    if (a.advance_pos) st->pos = st->pos + 1;
    st->argmax_key = kArgmaxInit;
}

}  // namespace

hipError_t launch_gemv(int pro, int epi, const GemvArgs &a, hipStream_t s) {
#define TMG_PE(P, E) \
    if (pro == P && epi == E) return launch_pe<P, E>(a, s);
    TMG_PE(PRO_PLAIN, EPI_STORE)
    TMG_PE(PRO_PLAIN, EPI_RESID)
    TMG_PE(PRO_ATTN_COMBINE, EPI_RESID)
    TMG_PE(PRO_NORM, EPI_SWIGLU)
    TMG_PE(PRO_NORM, EPI_QKV)
    TMG_PE(PRO_EMBED_NORM, EPI_QKV)
    TMG_PE(PRO_NORM, EPI_LOGITS)
    TMG_PE(PRO_NORM_BATCH, EPI_LOGITS)
#undef TMG_PE
    return hipErrorInvalidValue;
}

hipError_t launch_attn(const AttnArgs &a, hipStream_t s) {
    switch (a.hd) {
        case 16: return launch_attn_hd<16>(a, s);
        case 32: return launch_attn_hd<32>(a, s);
        case 64: return launch_attn_hd<64>(a, s);
        case 128: return launch_attn_hd<128>(a, s);
        case 256: return launch_attn_hd<256>(a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_attn_combine(const AttnArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(attn_combine_kernel, dim3((a.nq * a.hd + kBlock - 1) / kBlock), dim3(kBlock), 0, s, a);
    return hipGetLastError();
}

int gemv_blocks(int out, int in) {
    const int kc = (in + kChunk - 1) / kChunk;
    const int R = kc <= 2 ? 8 : 4;
    return (out + R - 1) / R;
}

hipError_t launch_finalize(const FinalizeArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(finalize_kernel, dim3(1), dim3(1024), 0, s, a);
    return hipGetLastError();
}

}  // namespace tmg
