// Prefill kernels for gfx950 (reference Model::forward_seq,
// src/model.rs:503-590).
//
// The batched projections Y[T,out] = X[T,in] W^T (reference
// matmul_batch_w_into -> gemm_tile_avx2, src/tensor.rs:573-858) run on bf16
// MFMA.  The reference multiplies f32 activations by BF16 weights, so the
// activations are carried as split-bf16 pairs x = hi + lo (|x-hi-lo| <=
// 2^-18|x|) and each tile issues one MFMA per half; the weights are exact
// BF16 and accumulation is f32.  Epilogues fuse RoPE + KV append, the
// residual add and SwiGLU; the next GEMM's split operands are written
// directly.
#include "coh.cuh"
#include "common.cuh"
#include "kernels.hpp"

namespace tmg {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__global__ __launch_bounds__(kBlock) void embed_gather_kernel(const int *tokens, int H, const uint16_t *eb,
                                                             const float *ef, float *x) {
    const int row = blockIdx.x;
    const int tok = tokens[row];
    for (int i = threadIdx.x; i < H; i += kBlock)
        x[(size_t)row * H + i] = eb ? bf16_to_f32(eb[(size_t)tok * H + i]) : ef[(size_t)tok * H + i];
}

// v*(inv*w) (rms_norm_batch, src/tensor.rs:951) or (v*inv)*w (rms_norm_into,
// src/tensor.rs:975).
__device__ __forceinline__ float norm_scale(float v, float inv, float w, int decode_assoc) {
    return decode_assoc ? (v * inv) * w : v * (inv * w);
}

// rms_norm_batch (src/tensor.rs:946-954): inv = 1/sqrt(ss/n + eps), v*(inv*w).
// One wavefront per row (four rows per workgroup), sum of squares reduced in
// registers + DPP.  Rows of up to 4096 floats in 256-float blocks are held in
// registers with the norm weights (every load issued up front); other widths
// take a strided loop.
__global__ __launch_bounds__(kBlock) void rmsnorm_split_kernel(const float *x, const float *w, float eps, int H, int T,
                                                              uint16_t *hi, uint16_t *lo, int decode_assoc) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= T) return;
    const float *xr = x + (size_t)row * H;
    uint16_t *hr = hi + (size_t)row * H, *lr = lo + (size_t)row * H;
    if (H % 256 == 0 && H <= 4096) {
        const int nb = H / 256;
        float4 v[16], wv[16];
#pragma unroll
        for (int b = 0; b < 16; b++)
            if (b < nb) {
                v[b] = *reinterpret_cast<const float4 *>(xr + b * 256 + lane * 4);
                wv[b] = *reinterpret_cast<const float4 *>(w + b * 256 + lane * 4);
            }
        float ss = 0.0f;
#pragma unroll
        for (int b = 0; b < 16; b++)
            if (b < nb) ss += v[b].x * v[b].x + v[b].y * v[b].y + v[b].z * v[b].z + v[b].w * v[b].w;
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)H + eps);
#pragma unroll
        for (int b = 0; b < 16; b++) {
            if (b < nb) {
                const int i = b * 256 + lane * 4;
                const float e[4] = {norm_scale(v[b].x, inv, wv[b].x, decode_assoc),
                                    norm_scale(v[b].y, inv, wv[b].y, decode_assoc),
                                    norm_scale(v[b].z, inv, wv[b].z, decode_assoc),
                                    norm_scale(v[b].w, inv, wv[b].w, decode_assoc)};
                uint16_t h[4], l[4];
#pragma unroll
                for (int c = 0; c < 4; c++) split_bf16(e[c], &h[c], &l[c]);
                *reinterpret_cast<uint2 *>(hr + i) = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
                *reinterpret_cast<uint2 *>(lr + i) = make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
            }
        }
        return;
    }
    float ss = 0.0f;
    for (int i = lane; i < H; i += 64) ss += xr[i] * xr[i];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)H + eps);
    for (int i = lane; i < H; i += 64) split_bf16(norm_scale(xr[i], inv, w[i], decode_assoc), hr + i, lr + i);
}

// Epilogue of one MFMA output fragment: rows mb .. mb+3 (mb a multiple of 4)
// of token column n.  Pair epilogues use rows (mb, mb+1) and (mb+2, mb+3).
template <int EPI>
__device__ __forceinline__ void gemm_store(const GemmArgs &a, int mb, int n, const f32x4 &acc) {
    if (n >= a.N) return;
    f32x4 v = acc;
    if (a.wscale) {
        // int8 weights: the row scale at write-back, y = acc * scale[o]
        // (src/tensor.rs:839-840), rounded before the residual add
#pragma clang fp contract(off)
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (mb + i < a.M) v[i] = v[i] * a.wscale[mb + i];
    }
    if constexpr (EPI == GEPI_STORE || EPI == GEPI_RESID) {
        float *yr = a.y + (size_t)n * a.M;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = mb + i;
            if (m < a.M) {
                if constexpr (EPI == GEPI_RESID)
                    yr[m] += v[i];
                else
                    yr[m] = v[i];
            }
        }
    } else {
#pragma unroll
        for (int pr = 0; pr < 2; pr++) {
            const int m = mb + 2 * pr;
            if (m + 1 >= a.M) continue;
            const int P = m >> 1;
            const float va = v[2 * pr], vb = v[2 * pr + 1];
            if constexpr (EPI == GEPI_SWIGLU) {
                const size_t o = (size_t)n * (a.M >> 1) + P;
                split_bf16(swiglu(va, vb), a.h_hi + o, a.h_lo + o);
            } else {  // GEPI_QKV
                const int half = a.hd >> 1;
                const int head = P / half, j = P - head * half;
                const int pos = a.pos_seq ? a.pos_seq[n] : a.start + n;
                const int kvd = a.nkv * a.hd;
                float *const kcache = a.k_seq ? a.k_seq[n] + a.kv_layer_off : a.k_cache;
                float *const vcache = a.v_seq ? a.v_seq[n] + a.kv_layer_off : a.v_cache;
                if (head < a.nq + a.nkv) {
                    float oa, ob;
                    rope_pair(va, vb, a.rope_cos[(size_t)pos * half + j], a.rope_sin[(size_t)pos * half + j], &oa,
                              &ob);
                    if (head < a.nq) {
                        float *qr = a.q_out + (size_t)n * a.nq * a.hd + head * a.hd;
                        qr[j] = oa;
                        qr[j + half] = ob;
                    } else {
                        float *kr = kcache + (size_t)pos * kvd + (head - a.nq) * a.hd;
                        kr[j] = oa;
                        kr[j + half] = ob;
                    }
                } else {
                    float *vr = vcache + (size_t)pos * kvd + (head - a.nq - a.nkv) * a.hd;
                    vr[j] = va;
                    vr[j + half] = vb;
                }
            }
        }
    }
}

// The vector epilogue of rows mb .. mb+3 (mb a multiple of 4) of token column
// n, in two phases so that a batch of tokens issues all its loads before any
// of its stores (the compiler cannot reorder a token's loads above another
// token's stores, so a one-phase epilogue pays one memory round trip per
// token).  Used where the rows are inside M, M is a multiple of 4 and (QKV)
// head_dim is a multiple of 4; gemm_store covers the rest element by element.
struct Epi4Tok {
    f32x4 y;      // RESID: the residual rows before the add
    float2 c, s;  // QKV: RoPE cos / sin of the rotation pairs j, j+1
    int pos;      // QKV: the token's position
};

template <int EPI>
__device__ __forceinline__ void epi4_load(const GemmArgs &a, int mb, int n, Epi4Tok &t) {
    if constexpr (EPI == GEPI_RESID) t.y = *reinterpret_cast<const f32x4 *>(a.y + (size_t)n * a.M + mb);
    if constexpr (EPI == GEPI_QKV) {
        const int half = a.hd >> 1;
        const int P = mb >> 1;
        const int head = P / half, j = P - head * half;
        t.pos = a.pos_seq ? a.pos_seq[n] : a.start + n;
        if (head < a.nq + a.nkv) {
            t.c = *reinterpret_cast<const float2 *>(a.rope_cos + (size_t)t.pos * half + j);
            t.s = *reinterpret_cast<const float2 *>(a.rope_sin + (size_t)t.pos * half + j);
        }
    }
}

// Phase two: v already carries the norm scale and the int8 row scale.
// Returns, for RESID with a norm hand-off (a.nrm_w; nw = nrm_w[mb .. mb+3]),
// the sum of squares of the four new residual values, after writing them
// times nrm_w as split-bf16 to nx_hi / nx_lo; 0 otherwise.
template <int EPI>
__device__ __forceinline__ float epi4_finish(const GemmArgs &a, int mb, int n, const f32x4 &v, const Epi4Tok &t,
                                             const f32x4 &nw) {
    if constexpr (EPI == GEPI_STORE) {
        *reinterpret_cast<f32x4 *>(a.y + (size_t)n * a.M + mb) = v;
    } else if constexpr (EPI == GEPI_RESID) {
        f32x4 y = t.y;
#pragma unroll
        for (int i = 0; i < 4; i++) y[i] = y[i] + v[i];
        const size_t o = (size_t)n * a.M + mb;
        *reinterpret_cast<f32x4 *>(a.y + o) = y;
        if (a.nrm_w) {
            uint32_t hi[2], lo[2];
#pragma unroll
            for (int pr = 0; pr < 2; pr++) {
                uint16_t h0, l0, h1, l1;
                split_bf16(y[2 * pr] * nw[2 * pr], &h0, &l0);
                split_bf16(y[2 * pr + 1] * nw[2 * pr + 1], &h1, &l1);
                hi[pr] = (uint32_t)h0 | ((uint32_t)h1 << 16);
                lo[pr] = (uint32_t)l0 | ((uint32_t)l1 << 16);
            }
            *reinterpret_cast<u32x2 *>(a.nx_hi + o) = u32x2{hi[0], hi[1]};
            *reinterpret_cast<u32x2 *>(a.nx_lo + o) = u32x2{lo[0], lo[1]};
            return (y[0] * y[0] + y[1] * y[1]) + (y[2] * y[2] + y[3] * y[3]);
        }
    } else if constexpr (EPI == GEPI_SWIGLU) {
        // pairs (mb, mb+1) and (mb+2, mb+3) -> h[P], h[P+1], P = mb / 2
        uint32_t hi = 0, lo = 0;
#pragma unroll
        for (int pr = 0; pr < 2; pr++) {
            uint16_t h, l;
            split_bf16(swiglu(v[2 * pr], v[2 * pr + 1]), &h, &l);
            hi |= (uint32_t)h << (16 * pr);
            lo |= (uint32_t)l << (16 * pr);
        }
        const size_t o = (size_t)n * (a.M >> 1) + (mb >> 1);
        *reinterpret_cast<uint32_t *>(a.h_hi + o) = hi;
        *reinterpret_cast<uint32_t *>(a.h_lo + o) = lo;
    } else {  // GEPI_QKV: pairs P, P+1 are rotation pairs j, j+1 of one head
        const int half = a.hd >> 1;
        const int P = mb >> 1;
        const int head = P / half, j = P - head * half;
        const int kvd = a.nkv * a.hd;
        float *dst;
        float2 o0, o1;  // values at j, j+1 and at j+half, j+half+1
        if (head < a.nq + a.nkv) {
            rope_pair(v[0], v[1], t.c.x, t.s.x, &o0.x, &o1.x);
            rope_pair(v[2], v[3], t.c.y, t.s.y, &o0.y, &o1.y);
            if (head < a.nq) {
                dst = a.q_out + (size_t)n * a.nq * a.hd + head * a.hd;
            } else {
                float *const kcache = a.k_seq ? a.k_seq[n] + a.kv_layer_off : a.k_cache;
                dst = kcache + (size_t)t.pos * kvd + (head - a.nq) * a.hd;
            }
        } else {
            o0 = make_float2(v[0], v[2]);
            o1 = make_float2(v[1], v[3]);
            float *const vcache = a.v_seq ? a.v_seq[n] + a.kv_layer_off : a.v_cache;
            dst = vcache + (size_t)t.pos * kvd + (head - a.nq - a.nkv) * a.hd;
        }
        *reinterpret_cast<float2 *>(dst + j) = o0;
        *reinterpret_cast<float2 *>(dst + j + half) = o1;
    }
    return 0.0f;
}

// The inputs of a one-pass, one-batch epilogue (FI = 4, FJ = 1, NB = 4: the
// split-K kernel) that do not depend on the tile's values: the tokens' norm
// partials (consumer side of the hand-off), the rows' scales and next norm
// weights, the residual rows or RoPE tables.  The split-K kernel loads them
// before its partial exchange, so that they arrive during the exchange's
// round trips instead of after them.
template <int EPI, int NB>
struct EpiPre {
    f32x4 nss[kMaxNormGroups / 4];
    f32x4 sc, nrw;
    Epi4Tok tk[NB];
};

template <int EPI, int NB>
__device__ __forceinline__ void epi_prefetch(const GemmArgs &a, int mw, int nw, EpiPre<EPI, NB> &p) {
    const int lane = threadIdx.x & 63, r = lane & 15, nsub = lane >> 4;
    if (a.nss_in) {
        const int n = min(nw + r, a.N - 1);
        const f32x4 *src = reinterpret_cast<const f32x4 *>(a.nss_in + (size_t)n * a.ngroups);
#pragma unroll
        for (int i = 0; i < kMaxNormGroups / 4; i++)
            if (4 * i < a.ngroups) p.nss[i] = src[i];
    }
    const int mb = mw + r * 4;
    const bool rows_vec = mb + 3 < a.M && !(a.M & 3) && !(EPI == GEPI_QKV && (a.hd & 3));
    p.sc = f32x4{1.f, 1.f, 1.f, 1.f};
    p.nrw = f32x4{0.f, 0.f, 0.f, 0.f};
    if (rows_vec && a.wscale) p.sc = *reinterpret_cast<const f32x4 *>(a.wscale + mb);
    if constexpr (EPI == GEPI_RESID)
        if (rows_vec && a.nrm_w) p.nrw = *reinterpret_cast<const f32x4 *>(a.nrm_w + mb);
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int nl = b * 4 + nsub;
        if (rows_vec && nw + nl < a.N) epi4_load<EPI>(a, mb, nw + nl, p.tk[b]);
    }
}

// 1 / rms of a token from its norm partials, added in group order
__device__ __forceinline__ float nss_inv_rms(const GemmArgs &a, const f32x4 (&p)[kMaxNormGroups / 4]) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxNormGroups / 4; i++)
        if (4 * i < a.ngroups) ss = ((ss + p[i][0]) + p[i][1]) + (p[i][2] + p[i][3]);
    return 1.0f / sqrtf(ss / (float)a.K + a.nrm_eps);
}

// The output of one wavefront's FI x FJ MFMA fragments (fragment (i, j): rows
// mw + 16 i + 4 (lane >> 4) .. +3 of token nw + 16 j + (lane & 15)) through
// the wavefront's own LDS region `buf` (FJ 16 token rows of 64 floats), 64
// rows at a time: written as [token][row], read back as four consecutive rows
// per lane, so that 16 lanes cover 64 consecutive rows of one token.  The
// 16-byte chunk c of token t sits at chunk c ^ (t & 15): both the fragment
// writes and the row reads are then free of bank conflicts (measured; a
// padded 68-float pitch conflicts on the reads).  LDS accesses of one
// wavefront execute in order, so no barrier separates the writes from the
// reads.  Tokens go through the epilogue in batches of NB, each batch's loads
// (residual rows, RoPE tables) issued before its stores: the split-K
// kernel's last-arriving wave, whose epilogue ends the GEMM, takes NB = 4
// (64-token prefill 1.72 -> 1.70 ms); the tiled kernels, whose epilogues
// overlap other workgroups' main loops, measured faster with NB = 1.
constexpr int kStagePitch = 64;  // floats per staged token row

template <int EPI, int FI, int FJ, int NB, bool PRE = false>
__device__ __forceinline__ void stage_epilogue(const GemmArgs &a, float *buf, int mw, int nw,
                                               const f32x4 (&acc)[FI][FJ], const EpiPre<EPI, NB> *pre = nullptr) {
    static_assert(FI % 4 == 0, "64-row passes");
    static_assert(FJ * 16 <= 64, "one token per lane for the norm scales");
    constexpr int NR = FJ * 4;  // token rows per lane per pass
    static_assert(NR % NB == 0, "whole batches");
    static_assert(!PRE || (FI == 4 && FJ == 1 && NR == NB), "prefetched inputs cover one pass of one batch");
    const int lane = threadIdx.x & 63, r = lane & 15, q4 = lane >> 4;
    const int nsub = lane >> 4;
    // norm hand-off, consumer side: lane l holds the scale of token
    // nw + l % (16 FJ); the token's partial sums are contiguous and all of
    // them are loaded at once (one memory round trip), then added in order
    float inv_l = 1.0f;
    if (a.nss_in) {
        if constexpr (PRE) {
            inv_l = nss_inv_rms(a, pre->nss);
        } else {
            const int n = min(nw + (lane & (FJ * 16 - 1)), a.N - 1);
            const f32x4 *src = reinterpret_cast<const f32x4 *>(a.nss_in + (size_t)n * a.ngroups);
            f32x4 p[kMaxNormGroups / 4];
#pragma unroll
            for (int i = 0; i < kMaxNormGroups / 4; i++)
                if (4 * i < a.ngroups) p[i] = src[i];
            inv_l = nss_inv_rms(a, p);
        }
    }
#pragma unroll
    for (int h = 0; h < FI / 4; h++) {
#pragma unroll
        for (int ii = 0; ii < 4; ii++)
#pragma unroll
            for (int j = 0; j < FJ; j++)
                *reinterpret_cast<f32x4 *>(buf + (j * 16 + r) * kStagePitch + (((ii * 4 + q4) ^ r) * 4)) =
                    acc[4 * h + ii][j];
        const int mb = mw + h * 64 + r * 4;
        const bool rows_vec = mb + 3 < a.M && !(a.M & 3) && !(EPI == GEPI_QKV && (a.hd & 3));
        // per-row inputs, the same for every token of the pass
        f32x4 sc = {1.f, 1.f, 1.f, 1.f}, nrw = {0.f, 0.f, 0.f, 0.f};
        if constexpr (PRE) {
            sc = pre->sc;
            nrw = pre->nrw;
        } else {
            if (rows_vec && a.wscale) sc = *reinterpret_cast<const f32x4 *>(a.wscale + mb);
            if constexpr (EPI == GEPI_RESID)
                if (rows_vec && a.nrm_w) nrw = *reinterpret_cast<const f32x4 *>(a.nrm_w + mb);
        }
#pragma unroll
        for (int r0 = 0; r0 < NR; r0 += NB) {
            f32x4 v[NB];
            Epi4Tok tk[NB];
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const int nl = (r0 + b) * 4 + nsub;
                v[b] = *reinterpret_cast<const f32x4 *>(buf + nl * kStagePitch + ((r ^ (nl & 15)) * 4));
                if (a.nss_in) {
                    const float inv = __shfl(inv_l, nl);
#pragma unroll
                    for (int i = 0; i < 4; i++) v[b][i] = v[b][i] * inv;
                }
                if constexpr (PRE)
                    tk[b] = pre->tk[b];
                else if (rows_vec && nw + nl < a.N)
                    epi4_load<EPI>(a, mb, nw + nl, tk[b]);
            }
#pragma unroll
            for (int b = 0; b < NB; b++) {
                const int nl = (r0 + b) * 4 + nsub, n = nw + nl;
                float sq = 0.0f;
                if (n < a.N) {
                    if (rows_vec) {
                        f32x4 vv = v[b];
                        if (a.wscale) {
#pragma clang fp contract(off)
#pragma unroll
                            for (int i = 0; i < 4; i++) vv[i] = vv[i] * sc[i];
                        }
                        sq = epi4_finish<EPI>(a, mb, n, vv, tk[b], nrw);
                    } else {
                        gemm_store<EPI>(a, mb, n, v[b]);
                    }
                }
                if constexpr (EPI == GEPI_RESID) {
                    // norm hand-off, producer side: the 16 lanes of token nl
                    // hold its 64 rows of this pass (the hand-off is set up
                    // only for M a multiple of 64, so rows_vec holds there)
                    if (a.nrm_w) {
                        const float tot = group_sum<16>(sq);
                        const int m64 = mw + h * 64;
                        if (r == 0 && n < a.N && m64 < a.M) a.nss[(size_t)n * (a.M >> 6) + (m64 >> 6)] = tot;
                    }
                }
            }
        }
    }
}

// MFMA GEMM D[m][n] = sum_k W[m][k] * (Bhi[n][k] + Blo[n][k]).
//
// Workgroup tile: 16 weight rows x 64 tokens; the four wavefronts split K in
// interleaved 32-wide steps and are summed through LDS.  MFMA
// v_mfma_f32_16x16x32_bf16 operand layout: lane l supplies A row (l & 15),
// k = 8*(l >> 4) .. +7, and B column (l & 15), the same k; it receives D rows
// 4*(l >> 4) .. +3 of column (l & 15).  So every lane owns two adjacent
// weight-row pairs of one token, which is what the pair epilogues need.
template <int EPI>
__global__ __launch_bounds__(kBlock) void gemm_kernel(const GemmArgs a) {
    constexpr int NB = 4;  // 16-token column blocks per workgroup
    __shared__ f32x4 s_acc[4][NB][64];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int m0 = blockIdx.x * 16, n0 = blockIdx.y * 16 * NB;
    const int K = a.K;
    const int r = lane & 15, kq = (lane >> 4) * 8;
    const uint16_t *Ap = a.W + (size_t)min(m0 + r, a.M - 1) * K + kq;
    const uint16_t *Bh[NB], *Bl[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        const int n = min(n0 + nb * 16 + r, a.N - 1);
        Bh[nb] = a.Bhi + (size_t)n * K + kq;
        Bl[nb] = a.Blo + (size_t)n * K + kq;
    }
    f32x4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k = wave * 32; k < K; k += 128) {
        const u32x4 av = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(Ap + k));
        u32x4 bh[NB], bl[NB];
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            bh[nb] = *reinterpret_cast<const u32x4 *>(Bh[nb] + k);
            bl[nb] = *reinterpret_cast<const u32x4 *>(Bl[nb] + k);
        }
        const bf16x8 A = __builtin_bit_cast(bf16x8, av);
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(bf16x8, bh[nb]), acc[nb], 0, 0, 0);
            acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(bf16x8, bl[nb]), acc[nb], 0, 0, 0);
        }
    }
#pragma unroll
    for (int nb = 0; nb < NB; nb++) s_acc[wave][nb][lane] = acc[nb];
    __syncthreads();
    // wave w finishes column block nb = w
    const int nb = wave;
    const f32x4 v = (s_acc[0][nb][lane] + s_acc[1][nb][lane]) + (s_acc[2][nb][lane] + s_acc[3][nb][lane]);
    const int n = n0 + nb * 16 + (lane & 15);
    const int mb = m0 + (lane >> 4) * 4;  // rows mb .. mb+3
    gemm_store<EPI>(a, mb, n, v);
}

// The same product over f32 weights (WMat::F32; matmul_batch_w_into's F32
// arm, src/tensor.rs:573-760) on the fp32 MFMA v_mfma_f32_16x16x4_f32, whose
// output layout is the bf16 one's: lane l supplies A row (l & 15) and B
// column (l & 15) at k = l >> 4 and receives D rows 4 (l >> 4) .. +3 of
// column (l & 15).  The activation is hi + lo, exact in f32.  Each lane
// loads 4 consecutive k of its weight row and of its token (16 and 2 x 8
// bytes), which serve 4 MFMAs: MFMA j takes the j-th of them from every lane,
// the same k set on both operands.  Workgroup tile 16 rows x 64 tokens, the
// four wavefronts on interleaved 16-wide K blocks, summed through LDS.
template <int EPI>
__global__ __launch_bounds__(kBlock) void gemm_f32w_kernel(const GemmArgs a) {
    constexpr int NB = 4;  // 16-token column blocks per workgroup
    __shared__ f32x4 s_acc[4][NB][64];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int m0 = blockIdx.x * 16, n0 = blockIdx.y * 16 * NB;
    const int K = a.K;
    const int r = lane & 15, kq = (lane >> 4) * 4;
    const float *Ap = a.Wf + (size_t)min(m0 + r, a.M - 1) * K + kq;
    const uint16_t *Bh[NB], *Bl[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
        const int n = min(n0 + nb * 16 + r, a.N - 1);
        Bh[nb] = a.Bhi + (size_t)n * K + kq;
        Bl[nb] = a.Blo + (size_t)n * K + kq;
    }
    f32x4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k = wave * 16; k < K; k += 64) {
        const f32x4 av = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(Ap + k));
        u32x2 bh[NB], bl[NB];
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            bh[nb] = *reinterpret_cast<const u32x2 *>(Bh[nb] + k);
            bl[nb] = *reinterpret_cast<const u32x2 *>(Bl[nb] + k);
        }
#pragma unroll
        for (int nb = 0; nb < NB; nb++) {
            const float x[4] = {bf16_lo(bh[nb].x) + bf16_lo(bl[nb].x), bf16_hi(bh[nb].x) + bf16_hi(bl[nb].x),
                                bf16_lo(bh[nb].y) + bf16_lo(bl[nb].y), bf16_hi(bh[nb].y) + bf16_hi(bl[nb].y)};
#pragma unroll
            for (int j = 0; j < 4; j++) acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j], x[j], acc[nb], 0, 0, 0);
        }
    }
#pragma unroll
    for (int nb = 0; nb < NB; nb++) s_acc[wave][nb][lane] = acc[nb];
    __syncthreads();
    const int nb = wave;
    const f32x4 v = (s_acc[0][nb][lane] + s_acc[1][nb][lane]) + (s_acc[2][nb][lane] + s_acc[3][nb][lane]);
    const int n = n0 + nb * 16 + (lane & 15);
    const int mb = m0 + (lane >> 4) * 4;  // rows mb .. mb+3
    gemm_store<EPI>(a, mb, n, v);
}

// Tiled MFMA GEMM for prompts of at least kTiledMinTokens tokens: workgroup
// tile 128 weight rows x 128 tokens, K in steps of 64; each of the four
// wavefronts owns a 64 x 64 quarter (4 x 4 MFMA fragments).
constexpr int kTM = 128, kTN = 128, kTK = 64;

// The W / Bhi / Blo tiles go global -> LDS directly (global_load_lds_dwordx4,
// no register staging) through a 3-stage ring, so step s + 2 is in flight
// while step s is multiplied and each step needs one barrier.  LDS rows are unpadded 128 B with the 16-byte chunks
// XOR-swizzled by (row & 7) against bank conflicts: a DMA wave-instruction
// fills 1 KB = 8 rows contiguously, so each lane fetches the global chunk that
// belongs at its LDS slot.
constexpr int kGStages = 3;
constexpr int kGTile = kTM * kTK * 2;  // bytes of one 128 x 64 bf16 tile

// NW = 8 wavefronts (two per SIMD, so one's MFMAs overlap the other's LDS
// reads): wave w owns rows 64 (w & 1) .. +63 and tokens 32 (w >> 1) .. +31
// (4 x 2 MFMA fragments) and issues two of each tile's 16 DMA instructions.
constexpr int kGWaves = 8;

template <int EPI>
__global__ __launch_bounds__(kGWaves * 64) void gemm_dma_kernel(const GemmArgs a) {
    constexpr int DPW = 16 / kGWaves;  // DMA instructions per wave per tile
    constexpr int NJ = kTN / 16 / (kGWaves / 2);  // token fragments per wave
    static_assert(3 * DPW <= 15, "vmcnt immediate");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[kGStages * 3 * kGTile];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int wm = wave & 1, wn = wave >> 1;
    const int m0 = blockIdx.x * kTM, n0 = blockIdx.y * kTN;
    const int K = a.K;
    const int nsteps = K / kTK;
    // DMA: wave w's instruction i fills rows (DPW w + i) * 8 .. +7 of a tile;
    // lane l writes row (DPW w + i) * 8 + (l >> 3), physical chunk l & 7, which
    // holds logical chunk (l & 7) ^ (row & 7)
    uint32_t off[3][DPW];
#pragma unroll
    for (int i = 0; i < DPW; i++) {
        const int row = (wave * DPW + i) * 8 + (lane >> 3);
        const int lc = (lane & 7) ^ (row & 7);
        off[0][i] = (uint32_t)min(m0 + row, a.M - 1) * (uint32_t)K + lc * 8;
        off[1][i] = (uint32_t)min(n0 + row, a.N - 1) * (uint32_t)K + lc * 8;
        off[2][i] = off[1][i];
    }
    auto issue = [&](int stage, int k0) {
#pragma unroll
        for (int x = 0; x < 3; x++) {
            const uint16_t *base = x == 0 ? a.W : (x == 1 ? a.Bhi : a.Blo);
#pragma unroll
            for (int i = 0; i < DPW; i++)
                __builtin_amdgcn_global_load_lds(base + off[x][i] + k0,
                                                 smem + (stage * 3 + x) * kGTile + (wave * DPW + i) * 1024, 16, 0, 0);
        }
    };
    issue(0, 0);
    if (nsteps > 1) issue(1, kTK);
    f32x4 acc[4][NJ];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int r = lane & 15, q4 = lane >> 4;
    for (int st = 0; st < nsteps; st++) {
        // this step's 3 DPW DMAs are complete once at most the next step's are
        // outstanding (vector memory counts complete in issue order)
        if (st + 1 < nsteps)
            __builtin_amdgcn_s_waitcnt(0xF70 | (3 * DPW));  // vmcnt(3 DPW)
        else
            __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0)
        __builtin_amdgcn_s_barrier();  // every wave's DMAs for this step landed; step - 1's reads are done
        if (st + 2 < nsteps) issue((st + 2) % kGStages, (st + 2) * kTK);
        const unsigned char *sa = smem + ((st % kGStages) * 3 + 0) * kGTile;
        const unsigned char *sh = sa + kGTile, *sl = sa + 2 * kGTile;
#pragma unroll
        for (int kk = 0; kk < kTK; kk += 32) {
            const int lc = kk / 8 + q4;
            bf16x8 fa[4], fh[NJ], fl[NJ];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int ra = wm * 64 + i * 16 + r;
                fa[i] = *reinterpret_cast<const bf16x8 *>(sa + ra * 128 + ((lc ^ (ra & 7)) * 16));
            }
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                const int rb = wn * NJ * 16 + j * 16 + r;
                fh[j] = *reinterpret_cast<const bf16x8 *>(sh + rb * 128 + ((lc ^ (rb & 7)) * 16));
                fl[j] = *reinterpret_cast<const bf16x8 *>(sl + rb * 128 + ((lc ^ (rb & 7)) * 16));
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fh[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fl[j], acc[i][j], 0, 0, 0);
        }
    }
    // the ring is free once every wave is past its last fragment reads
    __builtin_amdgcn_s_barrier();
    stage_epilogue<EPI, 4, NJ, 1>(a, reinterpret_cast<float *>(smem) + wave * NJ * 16 * kStagePitch, m0 + wm * 64,
                               n0 + wn * NJ * 16, acc);
}

// Large-tile MFMA GEMM for long prompts: workgroup tile 256 weight rows x
// 256 tokens, K in steps of 32.  The global -> LDS DMA path carries about
// 45 GB/s per CU (measured), and a step's W, Bhi and Blo tiles are 48 KB
// either way; the 256 x 256 tile does twice the MFMA work of the 128 x 128
// one for them.  Three-stage ring of 48 KB stages, up to three steps in
// flight, one barrier per step; LDS rows are 64 B (32 bf16) with the four
// 16-byte chunks XOR-swizzled by (row >> 1) & 3: by rocprofv3's
// SQ_LDS_BANK_CONFLICT, a fragment read (16 rows x 4 chunks) is then
// conflict-free, where (row >> 2) & 3 or row & 3 cost a second cycle per read;
// a DMA wave-instruction fills 16 rows (1 KB).  Wave w owns rows 128 (w & 1) .. +127 and tokens 64 (w >> 1) .. +63
// (8 x 4 MFMA fragments); its fragment reads for the next step overlap the
// current step's MFMAs.  The output leaves through LDS (stage_epilogue).
constexpr int kBM = 256, kBN = 256, kBK = 32;
constexpr int kBStages = 3;
constexpr int kBTile = kBM * kBK * 2;  // bytes of one 256 x 32 bf16 tile (kBN == kBM)
static_assert(kBM == kBN, "W and B tiles share the staging layout");

template <int EPI>
__global__ __launch_bounds__(kGWaves * 64) void gemm_big_kernel(const GemmArgs a) {
    constexpr int DPW = kBTile / 1024 / kGWaves;  // DMA instructions per wave per tile
    constexpr int FI = 8, FJ = 4;                 // row / token fragments per wave
    static_assert(6 * DPW <= 15, "vmcnt immediate");
    __shared__ __attribute__((aligned(1024))) unsigned char smem[kBStages * 3 * kBTile];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int wm = wave & 1, wn = wave >> 1;
    // A grid of at most one workgroup per CU runs in one round: each XCD (one
    // L2; workgroups go to XCDs round robin) then takes an eighth of the
    // token tiles against every row tile, so it fetches its activation rows
    // once and the weights (the smaller operand at these shapes) once per XCD,
    // instead of every activation row once per XCD (6-9% faster at 2048
    // weight rows x 8192 tokens; no gain or a loss for larger grids).
    int mt = blockIdx.x, nt = blockIdx.y;
    if ((gridDim.y & 7) == 0 && gridDim.x * gridDim.y <= 256) {
        const int L = blockIdx.x + gridDim.x * blockIdx.y;
        const int sl = L >> 3;
        mt = sl % gridDim.x;
        nt = (L & 7) * (gridDim.y >> 3) + sl / gridDim.x;
    }
    const int m0 = mt * kBM, n0 = nt * kBN;
    const int K = a.K;
    const int nsteps = K / kBK;
    uint32_t off[2][DPW];
#pragma unroll
    for (int i = 0; i < DPW; i++) {
        const int row = (wave * DPW + i) * 16 + (lane >> 2);
        const int lc = (lane & 3) ^ ((row >> 1) & 3);
        off[0][i] = (uint32_t)min(m0 + row, a.M - 1) * (uint32_t)K + lc * 8;
        off[1][i] = (uint32_t)min(n0 + row, a.N - 1) * (uint32_t)K + lc * 8;
    }
    auto issue = [&](int stage, int k0) {
#pragma unroll
        for (int x = 0; x < 3; x++) {
            const uint16_t *base = x == 0 ? a.W : (x == 1 ? a.Bhi : a.Blo);
#pragma unroll
            for (int i = 0; i < DPW; i++)
                __builtin_amdgcn_global_load_lds(base + off[x == 0 ? 0 : 1][i] + k0,
                                                 smem + (stage * 3 + x) * kBTile + (wave * DPW + i) * 1024, 16, 0, 0);
        }
    };
    const int r = lane & 15, q4 = lane >> 4;
    uint32_t ao[FI], bo[FJ];
#pragma unroll
    for (int i = 0; i < FI; i++) {
        const int ra = wm * 128 + i * 16 + r;
        ao[i] = ra * 64 + ((q4 ^ ((ra >> 1) & 3)) * 16);
    }
#pragma unroll
    for (int j = 0; j < FJ; j++) {
        const int rb = wn * 64 + j * 16 + r;
        bo[j] = kBTile + rb * 64 + ((q4 ^ ((rb >> 1) & 3)) * 16);
    }
    auto rd = [&](int stage, uint32_t o) {
        return *reinterpret_cast<const bf16x8 *>(smem + stage * 3 * kBTile + o);
    };
    // three steps in flight; wait for step 0 (the later groups may remain:
    // only DMAs are outstanding, and they complete in issue order)
    issue(0, 0);
    if (nsteps > 1) issue(1, kBK);
    if (nsteps > 2) issue(2, 2 * kBK);
    if (nsteps > 2)
        __builtin_amdgcn_s_waitcnt(0xF70 | (6 * DPW));
    else if (nsteps > 1)
        __builtin_amdgcn_s_waitcnt(0xF70 | (3 * DPW));
    else
        __builtin_amdgcn_s_waitcnt(0xF70);
    __builtin_amdgcn_s_barrier();
    f32x4 acc[FI][FJ];
#pragma unroll
    for (int i = 0; i < FI; i++)
#pragma unroll
        for (int j = 0; j < FJ; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x8 fa[FI], fh[FJ], fl[FJ];
#pragma unroll
    for (int i = 0; i < FI; i++) fa[i] = rd(0, ao[i]);
#pragma unroll
    for (int j = 0; j < FJ; j++) fh[j] = rd(0, bo[j]);
    // Step st: the hi pass (W x Bhi) from registers, reading step st's Blo
    // fragments after its first row group (their registers are free once the
    // previous lo pass is done); then, with every wave's reads of stage st
    // done and step st + 1's DMAs landed, one barrier, step st + 3's DMAs
    // into the freed stage, and the lo pass (W x Blo) with step st + 1's W and
    // Bhi fragment reads interleaved, each into registers the pass no longer
    // needs.  The scheduling barriers keep each read where it is placed.
    auto hi_pass = [&](int stage) {
#pragma unroll
        for (int i = 0; i < FI; i++) {
#pragma unroll
            for (int j = 0; j < FJ; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fh[j], acc[i][j], 0, 0, 0);
            if (i == 0) {
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < FJ; j++) fl[j] = rd(stage, bo[j] + kBTile);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    for (int st = 0; st + 1 < nsteps; st++) {
        const int ns = (st + 1) % kBStages;
        hi_pass(st % kBStages);
        // this wave's reads of stage st are done (lgkmcnt 0) and step st + 1's
        // DMAs have landed: only step st + 2's group may remain outstanding
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        if (st + 2 < nsteps)
            __builtin_amdgcn_s_waitcnt(0xF70 | (3 * DPW));  // vmcnt(3 DPW)
        else
            __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0)
        __builtin_amdgcn_s_barrier();
        if (st + 3 < nsteps) issue(st % kBStages, (st + 3) * kBK);
#pragma unroll
        for (int j = 0; j < FJ; j++) fh[j] = rd(ns, bo[j]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < FI; i++) {
#pragma unroll
            for (int j = 0; j < FJ; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fl[j], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            fa[i] = rd(ns, ao[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    hi_pass((nsteps - 1) % kBStages);
#pragma unroll
    for (int i = 0; i < FI; i++)
#pragma unroll
        for (int j = 0; j < FJ; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fl[j], acc[i][j], 0, 0, 0);
    // the ring is free once every wave is past its last fragment reads
    __builtin_amdgcn_s_barrier();
    stage_epilogue<EPI, FI, FJ, 1>(a, reinterpret_cast<float *>(smem) + wave * FJ * 16 * kStagePitch, m0 + wm * 128,
                                n0 + wn * 64, acc);
}

// Split-K MFMA GEMM for short prompts (fewer than kTiledMinTokens tokens).
//
// Workgroup tile: 64 weight rows x 64 tokens over one contiguous range of K
// (split ks of nsplit).  Each 64-wide K step's W, Bhi and Blo tiles go
// global -> LDS by DMA (XOR-swizzled 128-byte rows, as in gemm_dma_kernel)
// through a kSkStages-deep ring, so the next steps are in flight while one
// is multiplied and each step needs one barrier.  Wavefront w owns tokens
// 16 w .. 16 w + 15 against all 64 rows (4 MFMA row blocks).  The ring is
// 72 KB, so two workgroups share a CU and one's MFMAs overlap the other's
// LDS reads.
//
// With nsplit > 1 every wavefront stores its partial quarter tile, and the
// last of the quarter's nsplit wavefronts to arrive (device-scope counter)
// adds the partials in split order and runs the epilogue, so the result does
// not depend on arrival order.  Token tiles of one (row tile, split) pair are
// placed 8 blocks apart, i.e. on one XCD, so the W stream they share is read
// from HBM once.
constexpr int kSkStages = 3;
constexpr int kSkTile = 64 * 128;  // bytes of one 64 x 64 bf16 tile
constexpr int kSkOps = 6;          // DMA instructions per wave per step
constexpr int kSkMaxSplit = 8;

// PAIR: eight wavefronts, waves 4-7 taking the odd K steps (their partials
// added to waves 0-3's through LDS), with a ring of step pairs (144 KB, one
// workgroup per CU).  Used where the grid is at most one workgroup per CU
// and K is not split (the gate/up shape at 64 tokens: 18.2 -> 17.1 us):
// two wavefronts per SIMD then hide each other's LDS and barrier waits.
template <int EPI, bool PAIR>
__global__ __launch_bounds__(PAIR ? 2 * kBlock : kBlock, PAIR ? 1 : 2) void gemm_skinny_kernel(const GemmArgs a,
                                                                                                  int nsplit,
                                                                                                  int n_tiles) {
    constexpr int NPAR = PAIR ? 2 : 1;  // K steps per ring stage
    __shared__ __attribute__((aligned(1024))) unsigned char smem[kSkStages * NPAR * 3 * kSkTile];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int wq = wave & 3, par = PAIR ? wave >> 2 : 0;  // token quarter, step parity
    const int r = lane & 15, q = lane >> 4;
    const int m_tiles = (a.M + 63) >> 6;
    const int rest = blockIdx.x >> 3;
    const int nt = rest % n_tiles;
    const int g = (rest / n_tiles) * 8 + (blockIdx.x & 7);
    if (g >= m_tiles * nsplit) return;  // padding blocks of the XCD grouping
    const int mt = g % m_tiles, ks = g / m_tiles;
    const int K = a.K, nk = K >> 6;
    const int s0 = ks * nk / nsplit, ns = (ks + 1) * nk / nsplit - s0;
    const int m0 = mt * 64, n0 = nt * 64;
    // DMA: wave w fills row groups 2 wq, 2 wq + 1 (8 rows of 128 B) of each
    // tile of its steps; lane l writes physical chunk l & 7 of row (l >> 3),
    // i.e. logical chunk (l & 7) ^ (row & 7)
    const uint16_t *src[3][2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int row = (2 * wq + i) * 8 + (lane >> 3);
        const int lc = (lane & 7) ^ (row & 7);
        const size_t kofs = (size_t)s0 * 64 + lc * 8;
        src[0][i] = a.W + (size_t)min(m0 + row, a.M - 1) * K + kofs;
        src[1][i] = a.Bhi + (size_t)min(n0 + row, a.N - 1) * K + kofs;
        src[2][i] = a.Blo + (size_t)min(n0 + row, a.N - 1) * K + kofs;
    }
    // stage p % kSkStages holds steps NPAR p .. NPAR p + NPAR - 1; this wave
    // loads and multiplies step NPAR p + par
    auto has = [&](int p) { return NPAR * p + par < ns; };
    auto stage = [&](int p) { return smem + ((p % kSkStages) * NPAR + par) * 3 * kSkTile; };
    auto issue = [&](int p) {
        const int j = NPAR * p + par;
        unsigned char *dst = stage(p);
#pragma unroll
        for (int x = 0; x < 3; x++)
#pragma unroll
            for (int i = 0; i < 2; i++)
                __builtin_amdgcn_global_load_lds(src[x][i] + j * 64, dst + x * kSkTile + (2 * wq + i) * 1024, 16, 0, 0);
    };
    static_assert(kSkStages == 3, "wait counts assume one stage in flight behind the current one");
    const int np = (ns + NPAR - 1) / NPAR;
    if (has(0)) issue(0);
    if (has(1)) issue(1);
    f32x4 acc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int rb = wq * 16 + r;
    for (int p = 0; p < np; p++) {
        // stage p's DMAs of this wave are complete once at most stage p + 1's
        // are outstanding (only DMAs are outstanding: they complete in issue
        // order)
        if (has(p + 1))
            __builtin_amdgcn_s_waitcnt(0x0F70 | kSkOps);  // vmcnt(kSkOps)
        else
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __builtin_amdgcn_s_barrier();  // every wave's DMAs of stage p landed; stage p-1's reads are done
        if (has(p + 2)) issue(p + 2);
        if (!has(p)) continue;
        const unsigned char *sa = stage(p);
        const unsigned char *sh = sa + kSkTile, *sl = sa + 2 * kSkTile;
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            const int lc = kk * 4 + q;
            bf16x8 fa[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int ra = i * 16 + r;
                fa[i] = *reinterpret_cast<const bf16x8 *>(sa + ra * 128 + ((lc ^ (ra & 7)) * 16));
            }
            const bf16x8 fh = *reinterpret_cast<const bf16x8 *>(sh + rb * 128 + ((lc ^ (rb & 7)) * 16));
            const bf16x8 fl = *reinterpret_cast<const bf16x8 *>(sl + rb * 128 + ((lc ^ (rb & 7)) * 16));
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fh, acc[i], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fl, acc[i], 0, 0, 0);
        }
    }
    // the ring is free for the output staging once every wave is past its reads
    __builtin_amdgcn_s_barrier();
    if constexpr (PAIR) {
        // the odd steps' partials to the even-step waves of the same tokens,
        // through the LDS region that is the receiving wave's own staging
        // buffer below (its LDS accesses complete in order)
        f32x4 *hand =reinterpret_cast<f32x4 *>(smem) + (wq * 64 + lane) * 4;
        if (par) {
#pragma unroll
            for (int i = 0; i < 4; i++) hand[i] = acc[i];
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        if (par) return;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const f32x4 o = hand[i];
#pragma unroll
            for (int e = 0; e < 4; e++) acc[i][e] += o[e];
        }
    }
    // the epilogue's other inputs are loaded now (by every wave: the last to
    // arrive is not known yet), so they arrive during the exchange
    EpiPre<EPI, 4> pre;
    epi_prefetch<EPI, 4>(a, m0, n0 + wq * 16, pre);
    if (nsplit > 1) {
        // wave w's quarter of the tile (its 16 tokens) is reduced by the last
        // of the tile's nsplit waves w to arrive.  Partials move through
        // device-scope (sc1) stores and loads, which bypass the per-XCD L2s,
        // and each wave's stores are complete before its counter increment,
        // so no cache write-back or invalidation is needed; a per-wave
        // counter needs no workgroup barrier.
        const int slot = (nt * m_tiles + mt) * 4 + wq;
        float *part = a.part + ((size_t)slot * nsplit + ks) * 1024 + lane;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) st_dev(part + (i * 4 + e) * 64, acc[i][e]);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        unsigned old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(&a.cnt[slot], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old != (unsigned)(nsplit - 1)) return;
        // all partials are loaded before any is added (one memory round trip)
        const float *p0 = a.part + (size_t)slot * nsplit * 1024 + lane;
        float pv[kSkMaxSplit][16];
#pragma unroll
        for (int sp = 0; sp < kSkMaxSplit; sp++)
            if (sp < nsplit)
#pragma unroll
                for (int e = 0; e < 16; e++) pv[sp][e] = ld_dev(p0 + (size_t)sp * 1024 + e * 64);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[i][e] = pv[0][i * 4 + e];
#pragma unroll
        for (int sp = 1; sp < kSkMaxSplit; sp++)
            if (sp < nsplit)
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[i][e] += pv[sp][i * 4 + e];
        if (lane == 0) __hip_atomic_store(&a.cnt[slot], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const f32x4 out[4][1] = {{acc[0]}, {acc[1]}, {acc[2]}, {acc[3]}};
    stage_epilogue<EPI, 4, 1, 4, true>(a, reinterpret_cast<float *>(smem) + wq * 16 * kStagePitch, m0, n0 + wq * 16,
                                       out, &pre);
}

// The split-K short-prompt GEMM over 128-row tiles: eight wavefronts, waves
// 4-7 taking rows 64-127 of the tile against the same 64 tokens.  The
// activation tiles (hi and lo, 4 bytes per element against the weights' 2)
// are staged once per 128 weight rows instead of once per 64, a third less
// DMA per weight byte; each wave's MFMAs, split-K exchange and epilogue are
// those of gemm_skinny_kernel for its own 64 rows.  One workgroup per CU
// (a 96 KB ring).
constexpr int kSk2Ops = 4;  // DMA instructions per wave per step
template <int EPI>
__global__ __launch_bounds__(2 * kBlock, 1) void gemm_skinny_wide_kernel(const GemmArgs a, int nsplit, int n_tiles) {
    // stage: W rows 0-63, W rows 64-127, X hi, X lo
    __shared__ __attribute__((aligned(1024))) unsigned char smem[kSkStages * 4 * kSkTile];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int wq = wave & 3, half = wave >> 2;
    const int r = lane & 15, q = lane >> 4;
    const int m_tiles = (a.M + 127) >> 7;
    const int rest = blockIdx.x >> 3;
    const int nt = rest % n_tiles;
    const int g = (rest / n_tiles) * 8 + (blockIdx.x & 7);
    if (g >= m_tiles * nsplit) return;  // padding blocks of the XCD grouping
    const int mt = g % m_tiles, ks = g / m_tiles;
    const int K = a.K, nk = K >> 6;
    const int s0 = ks * nk / nsplit, ns = (ks + 1) * nk / nsplit - s0;
    const int m0 = mt * 128 + half * 64, n0 = nt * 64;
    // DMA: wave w fills row groups 2 wq, 2 wq + 1 of its half's W tile and of
    // X hi (waves 0-3) or X lo (waves 4-7)
    const uint16_t *src[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int row = (2 * wq + i) * 8 + (lane >> 3);
        const int lc = (lane & 7) ^ (row & 7);
        const size_t kofs = (size_t)s0 * 64 + lc * 8;
        src[0][i] = a.W + (size_t)min(m0 + row, a.M - 1) * K + kofs;
        src[1][i] = (half ? a.Blo : a.Bhi) + (size_t)min(n0 + row, a.N - 1) * K + kofs;
    }
    auto stage = [&](int p) { return smem + (p % kSkStages) * 4 * kSkTile; };
    auto issue = [&](int p) {
        unsigned char *dst = stage(p);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            __builtin_amdgcn_global_load_lds(src[0][i] + p * 64, dst + half * kSkTile + (2 * wq + i) * 1024, 16, 0, 0);
            __builtin_amdgcn_global_load_lds(src[1][i] + p * 64, dst + (2 + half) * kSkTile + (2 * wq + i) * 1024, 16, 0, 0);
        }
    };
    static_assert(kSkStages == 3, "wait counts assume one stage in flight behind the current one");
    if (0 < ns) issue(0);
    if (1 < ns) issue(1);
    f32x4 acc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int rb = wq * 16 + r;
    for (int p = 0; p < ns; p++) {
        // stage p's DMAs of this wave are complete once at most stage p + 1's
        // are outstanding (only DMAs are outstanding: they complete in order)
        if (p + 1 < ns)
            __builtin_amdgcn_s_waitcnt(0x0F70 | kSk2Ops);  // vmcnt(kSk2Ops)
        else
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __builtin_amdgcn_s_barrier();  // every wave's DMAs of stage p landed; stage p-1's reads are done
        if (p + 2 < ns) issue(p + 2);
        const unsigned char *st = stage(p);
        const unsigned char *sa = st + half * kSkTile, *sh = st + 2 * kSkTile, *sl = st + 3 * kSkTile;
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            const int lc = kk * 4 + q;
            bf16x8 fa[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int ra = i * 16 + r;
                fa[i] = *reinterpret_cast<const bf16x8 *>(sa + ra * 128 + ((lc ^ (ra & 7)) * 16));
            }
            const bf16x8 fh = *reinterpret_cast<const bf16x8 *>(sh + rb * 128 + ((lc ^ (rb & 7)) * 16));
            const bf16x8 fl = *reinterpret_cast<const bf16x8 *>(sl + rb * 128 + ((lc ^ (rb & 7)) * 16));
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fh, acc[i], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fl, acc[i], 0, 0, 0);
        }
    }
    // the ring is free for the output staging once every wave is past its reads
    __builtin_amdgcn_s_barrier();
    if (m0 >= a.M) return;  // the second half of the last row tile lies past the rows
    EpiPre<EPI, 4> pre;
    epi_prefetch<EPI, 4>(a, m0, n0 + wq * 16, pre);
    if (nsplit > 1) {
        // as in gemm_skinny_kernel, per 64-row half: device-scope partials,
        // a per-quarter counter, the last wave to arrive adds the partials
        // in split order
        const int m64 = (a.M + 63) >> 6;  // 64-row tiles: the counters and partials are laid out per 64 rows
        const int slot = (nt * m64 + mt * 2 + half) * 4 + wq;
        float *part = a.part + ((size_t)slot * nsplit + ks) * 1024 + lane;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) st_dev(part + (i * 4 + e) * 64, acc[i][e]);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        unsigned old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(&a.cnt[slot], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old != (unsigned)(nsplit - 1)) return;
        const float *p0 = a.part + (size_t)slot * nsplit * 1024 + lane;
        float pv[kSkMaxSplit][16];
#pragma unroll
        for (int sp = 0; sp < kSkMaxSplit; sp++)
            if (sp < nsplit)
#pragma unroll
                for (int e = 0; e < 16; e++) pv[sp][e] = ld_dev(p0 + (size_t)sp * 1024 + e * 64);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) acc[i][e] = pv[0][i * 4 + e];
#pragma unroll
        for (int sp = 1; sp < kSkMaxSplit; sp++)
            if (sp < nsplit)
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[i][e] += pv[sp][i * 4 + e];
        if (lane == 0) __hip_atomic_store(&a.cnt[slot], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const f32x4 out[4][1] = {{acc[0]}, {acc[1]}, {acc[2]}, {acc[3]}};
    stage_epilogue<EPI, 4, 1, 4, true>(a, reinterpret_cast<float *>(smem) + wave * 16 * kStagePitch, m0, n0 + wq * 16,
                                       out, &pre);
}

hipError_t launch_skinny(int epi, const GemmArgs &a, hipStream_t s) {
    // split K while the grid stays within one workgroup per CU, or while
    // splits keep at least 20 K steps within three workgroups per CU; at most
    // kSkMaxSplit ways, at least 2 steps per split
    const int m_tiles = (a.M + 63) / 64, n_tiles = (a.N + 63) / 64, nk = a.K / 64;
    int nsplit = 1;
    if (a.part && a.cnt) {
        for (;;) {
            const int wg2 = m_tiles * n_tiles * nsplit * 2, ns2 = nk / (nsplit * 2);
            if (nsplit * 2 > kSkMaxSplit || ns2 < 2) break;
            if (wg2 <= 256 || (ns2 >= 20 && wg2 <= 768))
                nsplit *= 2;
            else
                break;
        }
    }
    if (nsplit > 1 && (size_t)m_tiles * n_tiles * nsplit * 4096 > kSkinnyPartFloats) return hipErrorInvalidValue;
    const dim3 grid((m_tiles * nsplit + 7) / 8 * n_tiles * 8);
    // eight wavefronts per workgroup (step pairs) where K is not split and the
    // grid is at most one workgroup per CU
    if (nsplit == 1 && m_tiles * n_tiles <= 256) {
        switch (epi) {
            case GEPI_STORE: hipLaunchKernelGGL((gemm_skinny_kernel<GEPI_STORE, true>), grid, dim3(2 * kBlock), 0, s, a, nsplit, n_tiles); break;
            case GEPI_RESID: hipLaunchKernelGGL((gemm_skinny_kernel<GEPI_RESID, true>), grid, dim3(2 * kBlock), 0, s, a, nsplit, n_tiles); break;
            case GEPI_SWIGLU: hipLaunchKernelGGL((gemm_skinny_kernel<GEPI_SWIGLU, true>), grid, dim3(2 * kBlock), 0, s, a, nsplit, n_tiles); break;
            case GEPI_QKV: hipLaunchKernelGGL((gemm_skinny_kernel<GEPI_QKV, true>), grid, dim3(2 * kBlock), 0, s, a, nsplit, n_tiles); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    // one token tile: 64-row tiles of four waves (128-row tiles measured
    // slower there: 1B 64-token prefill 1.62 -> 1.81 ms)
    if (n_tiles == 1) {
        switch (epi) {
            case GEPI_STORE: hipLaunchKernelGGL((gemm_skinny_kernel<GEPI_STORE, false>), grid, dim3(kBlock), 0, s, a, nsplit, n_tiles); break;
            case GEPI_RESID: hipLaunchKernelGGL((gemm_skinny_kernel<GEPI_RESID, false>), grid, dim3(kBlock), 0, s, a, nsplit, n_tiles); break;
            case GEPI_SWIGLU: hipLaunchKernelGGL((gemm_skinny_kernel<GEPI_SWIGLU, false>), grid, dim3(kBlock), 0, s, a, nsplit, n_tiles); break;
            case GEPI_QKV: hipLaunchKernelGGL((gemm_skinny_kernel<GEPI_QKV, false>), grid, dim3(kBlock), 0, s, a, nsplit, n_tiles); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    // two or more token tiles: 128-row tiles (the activation tiles staged
    // once per 128 weight rows; 4B 128-token prefill 5.83 -> 5.58 ms), K
    // split while the grid stays within one workgroup (eight waves, a 96 KB
    // ring) per CU
    const int m2 = (a.M + 127) / 128;
    int ns2 = 1;
    if (a.part && a.cnt)
        while (ns2 * 2 <= kSkMaxSplit && nk / (ns2 * 2) >= 2 && m2 * n_tiles * ns2 * 2 <= 256) ns2 *= 2;
    if (ns2 > 1 && (size_t)m_tiles * n_tiles * ns2 * 4096 > kSkinnyPartFloats) return hipErrorInvalidValue;
    const dim3 grid2((m2 * ns2 + 7) / 8 * n_tiles * 8);
    switch (epi) {
        case GEPI_STORE: hipLaunchKernelGGL((gemm_skinny_wide_kernel<GEPI_STORE>), grid2, dim3(2 * kBlock), 0, s, a, ns2, n_tiles); break;
        case GEPI_RESID: hipLaunchKernelGGL((gemm_skinny_wide_kernel<GEPI_RESID>), grid2, dim3(2 * kBlock), 0, s, a, ns2, n_tiles); break;
        case GEPI_SWIGLU: hipLaunchKernelGGL((gemm_skinny_wide_kernel<GEPI_SWIGLU>), grid2, dim3(2 * kBlock), 0, s, a, ns2, n_tiles); break;
        case GEPI_QKV: hipLaunchKernelGGL((gemm_skinny_wide_kernel<GEPI_QKV>), grid2, dim3(2 * kBlock), 0, s, a, ns2, n_tiles); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

__global__ void copy_row_kernel(const float *x, int row, int H, float *dst) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < H; i += gridDim.x * blockDim.x)
        dst[i] = x[(size_t)row * H + i];
}

}  // namespace

hipError_t launch_embed_gather(const int *tokens, int T, int H, const uint16_t *eb, const float *ef, float *x,
                               hipStream_t s) {
    hipLaunchKernelGGL(embed_gather_kernel, dim3(T), dim3(kBlock), 0, s, tokens, H, eb, ef, x);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_split(const float *x, const float *w, float eps, int T, int H, uint16_t *hi, uint16_t *lo,
                                hipStream_t s, bool decode_assoc) {
    hipLaunchKernelGGL(rmsnorm_split_kernel, dim3((T + 3) / 4), dim3(kBlock), 0, s, x, w, eps, H, T, hi, lo,
                       decode_assoc ? 1 : 0);
    return hipGetLastError();
}

bool gemm_stages_output(int M, int N, int K) {
    if (K % 32 != 0 || M <= 0 || N <= 0) return false;
    if (N >= kTiledMinTokens && ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN) >= 240) return true;
    return K % 64 == 0;  // the 128 x 128 tiled or the split-K kernel
}

hipError_t launch_gemm(int epi, const GemmArgs &a, hipStream_t s) {
    if (a.K % 32 != 0 || a.M <= 0 || a.N <= 0) return hipErrorInvalidValue;
    if (a.Wf) {
        // f32 weights: the per-element epilogue only (no norm hand-off, no row scales)
        if (a.nrm_w || a.nss_in || a.wscale) return hipErrorInvalidValue;
        const dim3 grid((a.M + 15) / 16, (a.N + 63) / 64);
        switch (epi) {
            case GEPI_STORE: hipLaunchKernelGGL(gemm_f32w_kernel<GEPI_STORE>, grid, dim3(kBlock), 0, s, a); break;
            case GEPI_RESID: hipLaunchKernelGGL(gemm_f32w_kernel<GEPI_RESID>, grid, dim3(kBlock), 0, s, a); break;
            case GEPI_SWIGLU: hipLaunchKernelGGL(gemm_f32w_kernel<GEPI_SWIGLU>, grid, dim3(kBlock), 0, s, a); break;
            case GEPI_QKV: hipLaunchKernelGGL(gemm_f32w_kernel<GEPI_QKV>, grid, dim3(kBlock), 0, s, a); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    if ((a.nrm_w || a.nss_in) && !gemm_stages_output(a.M, a.N, a.K)) return hipErrorInvalidValue;
    if (a.nrm_w && (epi != GEPI_RESID || a.M % 64 != 0 || !a.nss || !a.nx_hi || !a.nx_lo)) return hipErrorInvalidValue;
    if (a.nss_in && (a.ngroups <= 0 || a.ngroups > kMaxNormGroups || a.ngroups % 4)) return hipErrorInvalidValue;
    // the 256 x 256 tile once its grid is about a workgroup per CU
    if (a.N >= kTiledMinTokens && a.K % kBK == 0 && ((a.M + kBM - 1) / kBM) * ((a.N + kBN - 1) / kBN) >= 240) {
        const dim3 grid((a.M + kBM - 1) / kBM, (a.N + kBN - 1) / kBN);
        switch (epi) {
            case GEPI_STORE: hipLaunchKernelGGL(gemm_big_kernel<GEPI_STORE>, grid, dim3(kGWaves * 64), 0, s, a); break;
            case GEPI_RESID: hipLaunchKernelGGL(gemm_big_kernel<GEPI_RESID>, grid, dim3(kGWaves * 64), 0, s, a); break;
            case GEPI_SWIGLU: hipLaunchKernelGGL(gemm_big_kernel<GEPI_SWIGLU>, grid, dim3(kGWaves * 64), 0, s, a); break;
            case GEPI_QKV: hipLaunchKernelGGL(gemm_big_kernel<GEPI_QKV>, grid, dim3(kGWaves * 64), 0, s, a); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    if (a.N >= kTiledMinTokens && a.K % kTK == 0) {
        const dim3 grid((a.M + kTM - 1) / kTM, (a.N + kTN - 1) / kTN);
        switch (epi) {
            case GEPI_STORE: hipLaunchKernelGGL(gemm_dma_kernel<GEPI_STORE>, grid, dim3(kGWaves * 64), 0, s, a); break;
            case GEPI_RESID: hipLaunchKernelGGL(gemm_dma_kernel<GEPI_RESID>, grid, dim3(kGWaves * 64), 0, s, a); break;
            case GEPI_SWIGLU: hipLaunchKernelGGL(gemm_dma_kernel<GEPI_SWIGLU>, grid, dim3(kGWaves * 64), 0, s, a); break;
            case GEPI_QKV: hipLaunchKernelGGL(gemm_dma_kernel<GEPI_QKV>, grid, dim3(kGWaves * 64), 0, s, a); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    if (a.K % 64 == 0) return launch_skinny(epi, a, s);
    const dim3 grid((a.M + 15) / 16, (a.N + 63) / 64);
    switch (epi) {
        case GEPI_STORE: hipLaunchKernelGGL(gemm_kernel<GEPI_STORE>, grid, dim3(kBlock), 0, s, a); break;
        case GEPI_RESID: hipLaunchKernelGGL(gemm_kernel<GEPI_RESID>, grid, dim3(kBlock), 0, s, a); break;
        case GEPI_SWIGLU: hipLaunchKernelGGL(gemm_kernel<GEPI_SWIGLU>, grid, dim3(kBlock), 0, s, a); break;
        case GEPI_QKV: hipLaunchKernelGGL(gemm_kernel<GEPI_QKV>, grid, dim3(kBlock), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_copy_row(const float *x, int row, int H, float *dst, hipStream_t s) {
    hipLaunchKernelGGL(copy_row_kernel, dim3((H + 255) / 256), dim3(256), 0, s, x, row, H, dst);
    return hipGetLastError();
}

}  // namespace tmg
