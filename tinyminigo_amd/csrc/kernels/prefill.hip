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
#include "common.cuh"
#include "kernels.hpp"

namespace tmg {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kBlock) void embed_gather_kernel(const int *tokens, int H, const uint16_t *eb,
                                                             const float *ef, float *x) {
    const int row = blockIdx.x;
    const int tok = tokens[row];
    for (int i = threadIdx.x; i < H; i += kBlock)
        x[(size_t)row * H + i] = eb ? bf16_to_f32(eb[(size_t)tok * H + i]) : ef[(size_t)tok * H + i];
}

// rms_norm_batch (src/tensor.rs:946-954): inv = 1/sqrt(ss/n + eps), v*(inv*w).
__global__ __launch_bounds__(kBlock) void rmsnorm_split_kernel(const float *x, const float *w, float eps, int H,
                                                              uint16_t *hi, uint16_t *lo) {
    __shared__ float scratch[4];
    const int row = blockIdx.x;
    const float *xr = x + (size_t)row * H;
    float ss[1] = {0.0f};
    for (int i = threadIdx.x; i < H; i += kBlock) ss[0] += xr[i] * xr[i];
    block_sum_n<1>(ss, scratch);
    const float inv = 1.0f / sqrtf(ss[0] / (float)H + eps);
    for (int i = threadIdx.x; i < H; i += kBlock) {
        const float v = __fmul_rn(xr[i], __fmul_rn(inv, w[i]));
        split_bf16(v, hi + (size_t)row * H + i, lo + (size_t)row * H + i);
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
    if (n >= a.N) return;
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
                const int pos = a.start + n;
                const int kvd = a.nkv * a.hd;
                if (head < a.nq + a.nkv) {
                    float oa, ob;
                    rope_pair(va, vb, a.rope_cos[(size_t)pos * half + j], a.rope_sin[(size_t)pos * half + j], &oa,
                              &ob);
                    if (head < a.nq) {
                        float *qr = a.q_out + (size_t)n * a.nq * a.hd + head * a.hd;
                        qr[j] = oa;
                        qr[j + half] = ob;
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
                                hipStream_t s) {
    hipLaunchKernelGGL(rmsnorm_split_kernel, dim3(T), dim3(kBlock), 0, s, x, w, eps, H, hi, lo);
    return hipGetLastError();
}

hipError_t launch_gemm(int epi, const GemmArgs &a, hipStream_t s) {
    if (a.K % 32 != 0 || a.M <= 0 || a.N <= 0) return hipErrorInvalidValue;
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
