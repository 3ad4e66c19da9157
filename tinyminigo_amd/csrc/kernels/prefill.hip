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

// Epilogue of one MFMA output fragment: rows mb .. mb+3 (mb a multiple of 4)
// of token column n.  Pair epilogues use rows (mb, mb+1) and (mb+2, mb+3).
template <int EPI>
__device__ __forceinline__ void gemm_store(const GemmArgs &a, int mb, int n, const f32x4 &v) {
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

// Tiled MFMA GEMM for long prompts: workgroup tile 128 weight rows x 128
// tokens, K in steps of 64 staged through LDS (W, Bhi, Blo; rows padded to
// 72 bf16 against bank conflicts).  The four wavefronts each own a 64 x 64
// quarter (4 x 4 MFMA fragments).  The next K step's global loads are held
// in registers while the current one is multiplied.
constexpr int kTM = 128, kTN = 128, kTK = 64, kTKP = kTK + 8;

template <int EPI>
__global__ __launch_bounds__(kBlock) void gemm_tiled_kernel(const GemmArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t sA[kTM][kTKP];
    __shared__ __attribute__((aligned(16))) uint16_t sH[kTN][kTKP];
    __shared__ __attribute__((aligned(16))) uint16_t sL[kTN][kTKP];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int wm = wave & 1, wn = wave >> 1;
    const int m0 = blockIdx.x * kTM, n0 = blockIdx.y * kTN;
    const int K = a.K;
    // global -> register staging: chunk c = t + 256 i (i < 4) is row c >> 3,
    // 16-byte column c & 7 of each 128 x 64 tile
    const uint16_t *gA[4], *gH[4], *gL[4];
    int srow[4], scol[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = t + kBlock * i;
        srow[i] = c >> 3;
        scol[i] = (c & 7) * 8;
        const int m = min(m0 + srow[i], a.M - 1), n = min(n0 + srow[i], a.N - 1);
        gA[i] = a.W + (size_t)m * K + scol[i];
        gH[i] = a.Bhi + (size_t)n * K + scol[i];
        gL[i] = a.Blo + (size_t)n * K + scol[i];
    }
    u32x4 rA[4], rH[4], rL[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        rA[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(gA[i]));
        rH[i] = *reinterpret_cast<const u32x4 *>(gH[i]);
        rL[i] = *reinterpret_cast<const u32x4 *>(gL[i]);
    }
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int r = lane & 15, kq = (lane >> 4) * 8;
    for (int k0 = 0; k0 < K; k0 += kTK) {
        __syncthreads();  // the previous step's fragments are read
#pragma unroll
        for (int i = 0; i < 4; i++) {
            *reinterpret_cast<u32x4 *>(&sA[srow[i]][scol[i]]) = rA[i];
            *reinterpret_cast<u32x4 *>(&sH[srow[i]][scol[i]]) = rH[i];
            *reinterpret_cast<u32x4 *>(&sL[srow[i]][scol[i]]) = rL[i];
        }
        __syncthreads();
        if (k0 + kTK < K) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                rA[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(gA[i] + k0 + kTK));
                rH[i] = *reinterpret_cast<const u32x4 *>(gH[i] + k0 + kTK);
                rL[i] = *reinterpret_cast<const u32x4 *>(gL[i] + k0 + kTK);
            }
        }
#pragma unroll
        for (int kk = 0; kk < kTK; kk += 32) {
            bf16x8 fa[4], fh[4], fl[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                fa[i] = *reinterpret_cast<const bf16x8 *>(&sA[wm * 64 + i * 16 + r][kk + kq]);
                fh[i] = *reinterpret_cast<const bf16x8 *>(&sH[wn * 64 + i * 16 + r][kk + kq]);
                fl[i] = *reinterpret_cast<const bf16x8 *>(&sL[wn * 64 + i * 16 + r][kk + kq]);
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fh[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fl[j], acc[i][j], 0, 0, 0);
                }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            gemm_store<EPI>(a, m0 + wm * 64 + i * 16 + (lane >> 4) * 4, n0 + wn * 64 + j * 16 + r, acc[i][j]);
}

// Tiled MFMA GEMM, LDS-DMA version: the same 128 x 128 workgroup tile and
// 64 x 64 wavefront quarters, but the W / Bhi / Blo tiles go global -> LDS
// directly (global_load_lds_dwordx4, no register staging) through a 3-stage
// ring, so step s + 2 is in flight while step s is multiplied and each step
// needs one barrier.  LDS rows are unpadded 128 B with the 16-byte chunks
// XOR-swizzled by (row & 7) against bank conflicts: a DMA wave-instruction
// fills 1 KB = 8 rows contiguously, so each lane fetches the global chunk that
// belongs at its LDS slot.
constexpr int kGStages = 3;
constexpr int kGTile = kTM * kTK * 2;  // bytes of one 128 x 64 bf16 tile

template <int EPI>
__global__ __launch_bounds__(kBlock) void gemm_dma_kernel(const GemmArgs a) {
    __shared__ __attribute__((aligned(1024))) unsigned char smem[kGStages * 3 * kGTile];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int wm = wave & 1, wn = wave >> 1;
    const int m0 = blockIdx.x * kTM, n0 = blockIdx.y * kTN;
    const int K = a.K;
    const int nsteps = K / kTK;
    // DMA: wave w's instruction i fills rows (4 w + i) * 8 .. +7 of a tile;
    // lane l writes row (4 w + i) * 8 + (l >> 3), physical chunk l & 7, which
    // holds logical chunk (l & 7) ^ (row & 7)
    uint32_t off[3][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = (wave * 4 + i) * 8 + (lane >> 3);
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
            for (int i = 0; i < 4; i++)
                __builtin_amdgcn_global_load_lds(base + off[x][i] + k0,
                                                 smem + (stage * 3 + x) * kGTile + (wave * 4 + i) * 1024, 16, 0, 0);
        }
    };
    issue(0, 0);
    if (nsteps > 1) issue(1, kTK);
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int r = lane & 15, q4 = lane >> 4;
    for (int st = 0; st < nsteps; st++) {
        // this step's 12 DMAs are complete once at most the next step's 12
        // are outstanding (vector memory counts complete in issue order)
        if (st + 1 < nsteps)
            __builtin_amdgcn_s_waitcnt(0xF7C);  // vmcnt(12)
        else
            __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0)
        __builtin_amdgcn_s_barrier();  // every wave's DMAs for this step landed; step - 1's reads are done
        if (st + 2 < nsteps) issue((st + 2) % kGStages, (st + 2) * kTK);
        const unsigned char *sa = smem + ((st % kGStages) * 3 + 0) * kGTile;
        const unsigned char *sh = sa + kGTile, *sl = sa + 2 * kGTile;
#pragma unroll
        for (int kk = 0; kk < kTK; kk += 32) {
            const int lc = kk / 8 + q4;
            bf16x8 fa[4], fh[4], fl[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int ra = wm * 64 + i * 16 + r, rb = wn * 64 + i * 16 + r;
                fa[i] = *reinterpret_cast<const bf16x8 *>(sa + ra * 128 + ((lc ^ (ra & 7)) * 16));
                fh[i] = *reinterpret_cast<const bf16x8 *>(sh + rb * 128 + ((lc ^ (rb & 7)) * 16));
                fl[i] = *reinterpret_cast<const bf16x8 *>(sl + rb * 128 + ((lc ^ (rb & 7)) * 16));
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fh[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[i], fl[j], acc[i][j], 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            gemm_store<EPI>(a, m0 + wm * 64 + i * 16 + q4 * 4, n0 + wn * 64 + j * 16 + r, acc[i][j]);
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
    if (a.N >= kTiledMinTokens && a.K % kTK == 0) {
        const dim3 grid((a.M + kTM - 1) / kTM, (a.N + kTN - 1) / kTN);
        switch (epi) {
            case GEPI_STORE: hipLaunchKernelGGL(gemm_dma_kernel<GEPI_STORE>, grid, dim3(kBlock), 0, s, a); break;
            case GEPI_RESID: hipLaunchKernelGGL(gemm_dma_kernel<GEPI_RESID>, grid, dim3(kBlock), 0, s, a); break;
            case GEPI_SWIGLU: hipLaunchKernelGGL(gemm_dma_kernel<GEPI_SWIGLU>, grid, dim3(kBlock), 0, s, a); break;
            case GEPI_QKV: hipLaunchKernelGGL(gemm_dma_kernel<GEPI_QKV>, grid, dim3(kBlock), 0, s, a); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
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
