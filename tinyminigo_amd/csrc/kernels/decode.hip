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
#include "attn.cuh"
#include "common.cuh"
#include "gemv.cuh"
#include "kernels.hpp"

namespace tmg {
namespace {

// NT threads per workgroup (kBlock, or kWideBlock for rows of 2560 -- and
// multiples -- that 2048-element chunks would leave a partial chunk of).
template <int KC, int R, int PRO, int EPI, int NT = kBlock>
__global__ __launch_bounds__(NT) void gemv_kernel(const GemvArgs a) {
    constexpr int NW = NT / 64;
    __shared__ float red[NW][R];
    __shared__ float scratch[NW];
    WeightRegs<KC, R> W;
    float xv[KC][8];
    if constexpr (PRO == PRO_EMBED_NORM) {
        // the gathered row depends on the token id: weights first
        gemv_load<KC, R, NT>(a, blockIdx.x, W);
        const int pos = EPI == EPI_QKV ? *a.pos : 0;
        gemv_embed_prologue<KC, NT>(a, *a.token, xv, scratch, blockIdx.x == 0);
        gemv_finish<KC, R, EPI, false, NT>(a, blockIdx.x, pos, W, xv, red);
    } else {
        // activation-side loads, then the weights (see gemv.cuh)
        ActIn<KC, PRO> in;
        act_issue<KC, PRO, NT>(a, in);
        EpiIn pre{};
        if constexpr (EPI == EPI_RESID) epi_issue_resid<R>(a, blockIdx.x, pre);
        gemv_load<KC, R, NT>(a, blockIdx.x, W);
        // keep the scalar loads below after the weight loads: a wait for them
        // would otherwise hold back the remaining weight loads
        __builtin_amdgcn_sched_barrier(0);
        const int pos = (EPI == EPI_QKV || PRO == PRO_ATTN_COMBINE) ? *a.pos : 0;
        if constexpr (EPI == EPI_QKV) epi_load_rope<R>(a, blockIdx.x, pos, pre);
        act_finish<KC, PRO, NT>(a, pos, in, xv, scratch);
        gemv_finish<KC, R, EPI, true, NT>(a, blockIdx.x, pos, W, xv, red, pre);
    }
}

// The same GEMV over int8 rows (GemvArgs::W8): the activation prologue and
// the epilogues are shared with gemv_kernel; between them the activation is
// quantized (quantize_act) and the rows are dotted in int32 (gemv_dot8).
template <int KC, int R, int PRO, int EPI>
__global__ __launch_bounds__(kBlock) void gemv_i8_kernel(const GemvArgs a) {
    __shared__ float red[4][R];
    __shared__ float scratch[4];
    WeightRegs8<KC, R> W;
    float xv[KC][8];
    EpiIn pre{};
    int pos = 0;
    if constexpr (PRO == PRO_EMBED_NORM) {
        gemv_load8<KC, R>(a, blockIdx.x, W);
        epi_issue_scale<R, EPI>(a, blockIdx.x, pre);
        if constexpr (EPI == EPI_QKV) pos = *a.pos;
        gemv_embed_prologue<KC>(a, *a.token, xv, scratch, blockIdx.x == 0);
        if constexpr (EPI == EPI_QKV) epi_load_rope<R>(a, blockIdx.x, pos, pre);
    } else {
        ActIn<KC, PRO> in;
        act_issue<KC, PRO>(a, in);
        if constexpr (EPI == EPI_RESID) epi_issue_resid<R>(a, blockIdx.x, pre);
        epi_issue_scale<R, EPI>(a, blockIdx.x, pre);
        gemv_load8<KC, R>(a, blockIdx.x, W);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (EPI == EPI_QKV || PRO == PRO_ATTN_COMBINE) pos = *a.pos;
        if constexpr (EPI == EPI_QKV) epi_load_rope<R>(a, blockIdx.x, pos, pre);
        act_finish<KC, PRO>(a, pos, in, xv, scratch);
    }
    int xq[KC][2];
    const float xs = quantize_act<KC>(xv, xq, scratch);
    gemv_dot8<KC, R>(W, xq, red);
    __syncthreads();
    gemv_epilogue<R, EPI, true, true>(a, blockIdx.x, pos, red, pre, xs);
}

// The same GEMV over f32 rows (GemvArgs::Wf): prologues and epilogues
// shared with gemv_kernel, two 16-byte weight loads per chunk and row.
template <int KC, int R, int PRO, int EPI>
__global__ __launch_bounds__(kBlock) void gemv_f32_kernel(const GemvArgs a) {
    __shared__ float red[4][R];
    __shared__ float scratch[4];
    WeightRegsF<KC, R> W;
    float xv[KC][8];
    EpiIn pre{};
    int pos = 0;
    if constexpr (PRO == PRO_EMBED_NORM) {
        gemv_loadf<KC, R>(a, blockIdx.x, W);
        if constexpr (EPI == EPI_QKV) pos = *a.pos;
        gemv_embed_prologue<KC>(a, *a.token, xv, scratch, blockIdx.x == 0);
    } else {
        ActIn<KC, PRO> in;
        act_issue<KC, PRO>(a, in);
        if constexpr (EPI == EPI_RESID) epi_issue_resid<R>(a, blockIdx.x, pre);
        gemv_loadf<KC, R>(a, blockIdx.x, W);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (EPI == EPI_QKV || PRO == PRO_ATTN_COMBINE) pos = *a.pos;
        if constexpr (EPI == EPI_QKV) epi_load_rope<R>(a, blockIdx.x, pos, pre);
        act_finish<KC, PRO>(a, pos, in, xv, scratch);
    }
    gemv_dotf<KC, R>(a, W, xv, red);
    __syncthreads();
    gemv_epilogue<R, EPI, PRO != PRO_EMBED_NORM, false>(a, blockIdx.x, pos, red, pre, 0.0f);
}

template <int KC, int PRO, int EPI>
hipError_t launch_kc(const GemvArgs &a, hipStream_t s) {
    // the split-merge prologue re-reads every split's partials per
    // workgroup; over a 2048-wide attention output 16 rows per workgroup
    // instead of 8 were slower (1B o_proj 4.37 -> 4.77 us, the step 0.7414
    // -> 0.7528 ms).  The one-chunk gate/up and QKV GEMVs take 16 rows (half
    // the workgroups, each with the RMSNorm prologue): 1B gate/up 9.70 ->
    // 9.46 us, the step 0.747 -> 0.745 ms; QKV 5.11 -> 4.98 us, the step
    // 0.7414 -> 0.7403 ms.  The plain GEMV (tmg_gemv_bf16) over one chunk
    // takes 4 rows (16 KB per workgroup): HBM-cold 2048 x 2048 3.44 -> 3.35
    // us, 73448 x 2048 45.9 -> 45.1 us; over three chunks 4 rows were slower
    // (2048 x 6144 5.95 -> 6.14 us)
    constexpr int R = ((EPI == EPI_SWIGLU || (EPI == EPI_QKV && PRO == PRO_NORM)) && KC == 1) ? 16
                      : (PRO == PRO_PLAIN && EPI == EPI_STORE && KC == 1)                     ? 4
                                                                                               : gemv_rows<KC>();
    const int grid = (a.out + R - 1) / R;
    if (!a.W8 && a.Wf) {
        // (the split-merge prologue is fused only over attention outputs of
        // at most 4096, i.e. two chunks)
        if constexpr (PRO == PRO_ATTN_COMBINE && KC > 2) {
            return hipErrorInvalidValue;
        } else {
            constexpr int RF = gemv_rows_f32<KC>();
            hipLaunchKernelGGL((gemv_f32_kernel<KC, RF, PRO, EPI>), dim3((a.out + RF - 1) / RF), dim3(kBlock), 0, s,
                               a);
        }
    } else if (a.W8) {
        if constexpr (EPI == EPI_LOGITS || PRO == PRO_NORM_BATCH) {
            return hipErrorInvalidValue;  // lm_head keeps BF16 rows
        } else {
            constexpr int R8 = gemv_rows8<KC, PRO>();
            hipLaunchKernelGGL((gemv_i8_kernel<KC, R8, PRO, EPI>), dim3((a.out + R8 - 1) / R8), dim3(kBlock), 0, s,
                               a);
        }
    } else if constexpr (PRO == PRO_ATTN_COMBINE && KC > 1) {
        return hipErrorInvalidValue;  // BF16 rows of 2049-4096: launch_merge_wide
    } else {
        hipLaunchKernelGGL((gemv_kernel<KC, R, PRO, EPI>), dim3(grid), dim3(kBlock), 0, s, a);
    }
    return hipGetLastError();
}

// Rows of 2560 elements (the 4B-class hidden size) in 2048-element chunks
// leave a second chunk three quarters empty: its clamped loads repeat the
// row's last 16 bytes and its registers halve the waves per SIMD.  Such
// rows (and multiples of 2560 that are not multiples of 2048) take
// kWideBlock threads and whole chunks of 2560.
constexpr int kWideBlock = 320;
constexpr int kWideChunk = kWideBlock * 8;

template <int KC, int PRO, int EPI>
hipError_t launch_wide(const GemvArgs &a, hipStream_t s) {
    constexpr int R = (EPI == EPI_SWIGLU && KC == 1) ? 16 : gemv_rows<KC>();
    static_assert(EPI != EPI_LOGITS || gemv_rows<KC>() == 8, "the argmax partials are counted with 8 rows per workgroup");
    hipLaunchKernelGGL((gemv_kernel<KC, R, PRO, EPI, kWideBlock>), dim3((a.out + R - 1) / R), dim3(kWideBlock), 0, s,
                       a);
    return hipGetLastError();
}

// The split merge over an attention output of 2049-4096 elements (the
// 4B-class o_proj): 512 threads with one 4096-element chunk each, so a
// wavefront issues half the loads of two chunks at 256 threads (24 partial
// and 16 weight loads, within the 63 that vmcnt counts) and holds 156
// VGPRs instead of 256 plus 46 spilled to AGPRs: 4B o_proj 8.25 -> 7.21 us,
// the sampled 4B step 1.920 -> 1.883 ms.  16 rows per workgroup (each
// workgroup re-reads all the split partials, so fewer rows re-read them
// more often: 8 rows took 9.4 us).
constexpr int kMergeBlock = 512;

template <int PRO, int EPI>
hipError_t launch_merge_wide(const GemvArgs &a, hipStream_t s) {
    constexpr int R = 16;
    hipLaunchKernelGGL((gemv_kernel<1, R, PRO, EPI, kMergeBlock>), dim3((a.out + R - 1) / R), dim3(kMergeBlock), 0, s,
                       a);
    return hipGetLastError();
}

// The residual GEMV over the down projection's long rows, 4 rows per
// workgroup, in wider workgroups with fewer chunks per thread than 2048-
// element chunks at 256 threads:
// - rows of 10240 (4B-class): 640 threads, two 5120-element chunks (12 loads
//   per wavefront instead of 30, 58 VGPRs instead of 128): 11.13 -> 10.91 us
//   per launch (8 rows: 12.4);
// - rows of 6144 (1B-class): 768 threads, one 6144-element chunk (6 loads
//   per wavefront instead of 30): 5.98 -> 6.05 us replayed alone, but the
//   step 0.7461 -> 0.7424 ms (8 rows: 0.7433).
template <int KC, int NT, int PRO, int EPI>
hipError_t launch_down_wide(const GemvArgs &a, hipStream_t s) {
    constexpr int R = 4;
    hipLaunchKernelGGL((gemv_kernel<KC, R, PRO, EPI, NT>), dim3((a.out + R - 1) / R), dim3(NT), 0, s, a);
    return hipGetLastError();
}

template <int PRO, int EPI>
hipError_t launch_pe(const GemvArgs &a, hipStream_t s) {
    if constexpr (PRO == PRO_PLAIN && EPI == EPI_RESID) {
        if (!a.W8 && !a.Wf && a.in == 2 * 640 * 8) return launch_down_wide<2, 640, PRO, EPI>(a, s);
        if (!a.W8 && !a.Wf && a.in == 768 * 8) return launch_down_wide<1, 768, PRO, EPI>(a, s);
    }
    if constexpr (PRO == PRO_ATTN_COMBINE) {
        if (!a.W8 && !a.Wf && a.in > kChunk && a.in <= kMergeBlock * 8) return launch_merge_wide<PRO, EPI>(a, s);
    } else {
        if (!a.W8 && !a.Wf && a.in % kChunk != 0 && a.in % kWideChunk == 0) {
            switch (a.in / kWideChunk) {
                case 1: return launch_wide<1, PRO, EPI>(a, s);
                case 2: return launch_wide<2, PRO, EPI>(a, s);
                default: break;  // wider rows: 2048-element chunks
            }
        }
    }
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

// The GEMV over several activation rows (batched decode, gemv.cuh): the
// first group's activation loads, then the block's weight rows, then the
// groups one after another against the weights held in registers.
template <int KC, int R, int TG, int PRO, int EPI>
__global__ __launch_bounds__(kBlock) void gemv_mt_kernel(const GemvArgs a) {
    __shared__ float red[4][R * TG];
    __shared__ float scratch[4 * TG];
    float wv[KC][8];
    if constexpr (PRO == PRO_NORM) {
        load_norm_w<KC>(a, wv);
    } else {
#pragma unroll
        for (int c = 0; c < KC; c++)
#pragma unroll
            for (int j = 0; j < 8; j++) wv[c][j] = 0.0f;
    }
    float xv[TG][KC][8];
    mt_issue<KC, TG>(a, 0, xv);
    WeightRegs<KC, R> W;
    gemv_load<KC, R>(a, blockIdx.x, W);
    __builtin_amdgcn_sched_barrier(0);
    for (int b0 = 0; b0 < a.nb; b0 += TG) {
        if (b0 > 0) mt_issue<KC, TG>(a, b0, xv);
        mt_norm<KC, TG, PRO>(a, wv, xv, scratch);
        mt_dot<KC, R, TG>(a, W, xv, red);
        __syncthreads();
        mt_epilogue<R, TG, EPI>(a, blockIdx.x, b0, red);
        __syncthreads();  // red and scratch are reused by the next group
    }
}

template <int KC, int TG, int PRO, int EPI>
hipError_t launch_mt_kt(const GemvArgs &a, hipStream_t s) {
    constexpr int R = gemv_mt_rows(KC, TG);
    hipLaunchKernelGGL((gemv_mt_kernel<KC, R, TG, PRO, EPI>), dim3((a.out + R - 1) / R), dim3(kBlock), 0, s, a);
    return hipGetLastError();
}

template <int KC, int PRO, int EPI>
hipError_t launch_mt_kc(const GemvArgs &a, hipStream_t s) {
    if constexpr (KC <= 3) {
        if constexpr (KC == 1)
            if (gemv_mt_group(KC, a.nb) == 8) return launch_mt_kt<KC, 8, PRO, EPI>(a, s);
        if (gemv_mt_group(KC, a.nb) == 4) return launch_mt_kt<KC, 4, PRO, EPI>(a, s);
    }
    return launch_mt_kt<KC, 2, PRO, EPI>(a, s);
}

template <int PRO, int EPI>
hipError_t launch_mt_pe(const GemvArgs &a, hipStream_t s) {
    switch ((a.in + kChunk - 1) / kChunk) {
        case 1: return launch_mt_kc<1, PRO, EPI>(a, s);
        case 2: return launch_mt_kc<2, PRO, EPI>(a, s);
        case 3: return launch_mt_kc<3, PRO, EPI>(a, s);
        case 4: return launch_mt_kc<4, PRO, EPI>(a, s);
        case 5: return launch_mt_kc<5, PRO, EPI>(a, s);
        case 6: return launch_mt_kc<6, PRO, EPI>(a, s);
        case 8:
        case 7: return launch_mt_kc<8, PRO, EPI>(a, s);
        default: return hipErrorInvalidValue;
    }
}

// WMat::quantize_i8 (src/tensor.rs:275-293) of BF16 rows, one workgroup per
// row: the row's max |w| (block reduction), scale = max/127 or 1 for a zero
// row, q = round(w / scale) with halves away from zero, clamped to +-127.
__global__ __launch_bounds__(kBlock) void quantize_i8_kernel(uint16_t *w, int in, int8_t *q8, float *scale,
                                                             int rewrite) {
    __shared__ float scratch[4];
    const int row = blockIdx.x;
    uint16_t *wr = w + (size_t)row * in;
    int8_t *qr = q8 + (size_t)row * in;
    float m[1] = {0.0f};
    for (int k = threadIdx.x * 8; k < in; k += kBlock * 8) {
        const uint4 u = *reinterpret_cast<const uint4 *>(wr + k);
        const uint32_t p[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; j++) m[0] = fmaxf(fabsf(bf16_hi(p[j])), fmaxf(fabsf(bf16_lo(p[j])), m[0]));
    }
    block_max_n<1>(m, scratch);
    const float sc = m[0] > 0.0f ? __fdiv_rn(m[0], 127.0f) : 1.0f;
    for (int k = threadIdx.x * 8; k < in; k += kBlock * 8) {
        const uint4 u = *reinterpret_cast<const uint4 *>(wr + k);
        const uint32_t p[4] = {u.x, u.y, u.z, u.w};
        uint32_t packed[2] = {0u, 0u}, codes[4];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float v = (j & 1) ? bf16_hi(p[j >> 1]) : bf16_lo(p[j >> 1]);
            const float r = roundf(__fdiv_rn(v, sc));
            const int q = r == r ? (int)fminf(fmaxf(r, -127.0f), 127.0f) : 0;
            packed[j >> 2] |= ((uint32_t)q & 0xffu) << (8 * (j & 3));
            const uint32_t b = f32_to_bf16_rne((float)q);  // exact: |q| <= 127
            if (j & 1)
                codes[j >> 1] |= b << 16;
            else
                codes[j >> 1] = b;
        }
        *reinterpret_cast<uint2 *>(qr + k) = make_uint2(packed[0], packed[1]);
        if (rewrite) *reinterpret_cast<uint4 *>(wr + k) = make_uint4(codes[0], codes[1], codes[2], codes[3]);
    }
    if (threadIdx.x == 0) scale[row] = sc;
}

// quantize_i8 of f32 rows, one workgroup per row: the same steps as
// quantize_i8_kernel on the row's f32 values; the codes also go to `codes`
// as BF16 (exact, |q| <= 127).
__global__ __launch_bounds__(kBlock) void quantize_i8_f32_kernel(const float *w, int in, int8_t *q8, float *scale,
                                                                 uint16_t *codes) {
    __shared__ float scratch[4];
    const int row = blockIdx.x;
    const float *wr = w + (size_t)row * in;
    int8_t *qr = q8 + (size_t)row * in;
    uint16_t *cr = codes + (size_t)row * in;
    float m[1] = {0.0f};
    for (int k = threadIdx.x * 8; k < in; k += kBlock * 8) {
        const float4 a = *reinterpret_cast<const float4 *>(wr + k), b = *reinterpret_cast<const float4 *>(wr + k + 4);
        m[0] = fmaxf(m[0], fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
        m[0] = fmaxf(m[0], fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
    }
    block_max_n<1>(m, scratch);
    const float sc = m[0] > 0.0f ? __fdiv_rn(m[0], 127.0f) : 1.0f;
    for (int k = threadIdx.x * 8; k < in; k += kBlock * 8) {
        const float4 a = *reinterpret_cast<const float4 *>(wr + k), b = *reinterpret_cast<const float4 *>(wr + k + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t packed[2] = {0u, 0u}, cw[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float r = roundf(__fdiv_rn(v[j], sc));
            const int q = r == r ? (int)fminf(fmaxf(r, -127.0f), 127.0f) : 0;
            packed[j >> 2] |= ((uint32_t)q & 0xffu) << (8 * (j & 3));
            cw[j >> 1] |= (uint32_t)f32_to_bf16_rne((float)q) << (16 * (j & 1));
        }
        *reinterpret_cast<uint2 *>(qr + k) = make_uint2(packed[0], packed[1]);
        *reinterpret_cast<uint4 *>(cr + k) = make_uint4(cw[0], cw[1], cw[2], cw[3]);
    }
    if (threadIdx.x == 0) scale[row] = sc;
}

// ---------------------------------------------------------------------------
// Attention: grid (nsplit, nkv, T), one attn_item per workgroup.  A row
// covered by one split is written out directly; otherwise every split writes
// (o, max, sum) partials that are merged after the kernel boundary (fused
// into the o_proj GEMV prologue, or attn_combine_kernel), which also publishes
// them across the XCDs' L2s without any in-kernel fence.
// ---------------------------------------------------------------------------

// SPEC (decode): splits below a.spec_splits (default kSpecSplits) load their
// first chunk before the position is read (see attn_item).
template <int HD, int GROUP, bool SPEC, int NT = kBlock, int CHW = kAttnBlockLong>
__global__ __launch_bounds__(NT) void attn_kernel(const AttnArgs a) {
    __shared__ AttnShared<HD, GROUP, NT> sm;
    const int split = blockIdx.x, g = blockIdx.y, ti = blockIdx.z;
    if constexpr (SPEC) {
        if (split < (a.spec_splits > 0 ? a.spec_splits : kSpecSplits)) {
            attn_item<HD, GROUP, true, NT, CHW>(a, split, g, ti, 0, 0, sm);
            return;
        }
    }
    const int qpos = a.pos_seq ? a.pos_seq[ti] : (a.pos_dev ? *a.pos_dev : a.start) + ti;
    const int active = active_splits(qpos + 1, a.nsplit, AttnGeom<HD, GROUP, NT, CHW>::CH);
    if (split >= active) return;
    attn_item<HD, GROUP, false, NT, CHW>(a, split, g, ti, qpos, active, sm);
}

// Merge of the split-K partials of a decode launch, one workgroup per
// (query head, row): the split statistics (max m_s, sum l_s) are reduced
// once per workgroup, then 256 threads = (256 / hd) split lanes x hd dims
// accumulate sum_s e^(m_s - M) o_s[d] with all their partial loads in
// flight, and the split lanes are summed through LDS.  out = that /
// sum_s e^(m_s - M) l_s.  Row ti's position is pos_seq[ti] (batched decode)
// or the cache position + ti.
__global__ __launch_bounds__(kBlock) void attn_combine_kernel(const AttnArgs a) {
    __shared__ float s_w[kBlock];
    __shared__ float s_o[kBlock];
    __shared__ float scratch[4];
    const int h = blockIdx.x, ti = blockIdx.y, t = threadIdx.x;
    const int group = a.nq / a.nkv;
    const int g = h / group, hq = h - g * group;
    const int qpos = a.pos_seq ? a.pos_seq[ti] : (a.pos_dev ? *a.pos_dev : a.start) + ti;
    const int active = active_splits(qpos + 1, a.nsplit, a.block ? a.block : kAttnBlockLong);
    const size_t base = ((size_t)ti * a.nkv + g) * a.nsplit * group + hq;
    float m = -INFINITY, l = 0.0f;
    if (t < active) {
        const float2 ml = *reinterpret_cast<const float2 *>(a.part_ml + (base + (size_t)t * group) * 2);
        m = ml.x;
        l = ml.y;
    }
    float M[1] = {m};
    block_max_n<1>(M, scratch);
    const float w = (m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - M[0]);
    float L[1] = {w * l};
    block_sum_n<1>(L, scratch);
    s_w[t] = w;
    __syncthreads();
    const int d = t % a.hd, j0 = t / a.hd, step = kBlock / a.hd;
    float acc = 0.0f;
#pragma unroll 8
    for (int sp = j0; sp < active; sp += step) acc = fmaf(a.part[(base + (size_t)sp * group) * a.hd + d], s_w[sp], acc);
    s_o[t] = acc;
    __syncthreads();
    if (t < a.hd) {
        float o = s_o[t];
        for (int j = 1; j < step; j++) o += s_o[j * a.hd + t];
        a.out_f32[(size_t)ti * a.nq * a.hd + h * a.hd + t] = o / L[0];
    }
}

constexpr int kWideAttnSplits = 32;
static_assert(kAttnThreads == kBlock, "the host sizes the attention partition for kBlock threads");

// The instantiation whose chunk (= partition block) is a.block positions:
// the short-context width (decode of short caches, prefill rows at four or
// more query heads per KV head) or kAttnBlockLong.
template <int HD, int GROUP, bool SPEC>
hipError_t launch_attn_group(const AttnArgs &a, dim3 grid, hipStream_t s) {
    const int blk = a.block ? a.block : kAttnBlockLong;
    if (blk == attn_chunk(HD, GROUP, kBlock, kAttnBlockLong)) {
        hipLaunchKernelGGL((attn_kernel<HD, GROUP, SPEC, kBlock, kAttnBlockLong>), grid, dim3(kBlock), 0, s, a);
    } else if (blk == attn_chunk(HD, GROUP, kBlock, kAttnBlockShort)) {
        hipLaunchKernelGGL((attn_kernel<HD, GROUP, SPEC, kBlock, kAttnBlockShort>), grid, dim3(kBlock), 0, s, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int HD, bool SPEC>
hipError_t launch_attn_hd(const AttnArgs &a, hipStream_t s) {
    const dim3 grid(a.nsplit, a.nkv, a.T);
    // Long contexts (all 32 splits in use; one workgroup per CU with 8 KV
    // heads): 512 threads, two positions per team per chunk, two waves per
    // SIMD -- 15.6 against 16.0 us per layer at 8K positions; at short
    // contexts 256 threads are faster (4.5 against 4.7 us).
    if constexpr (HD == 128 && SPEC) {
        if (a.nsplit >= kWideAttnSplits && a.nq / a.nkv == 2 && (a.block ? a.block : kAttnBlockLong) == kAttnBlockLong) {
            hipLaunchKernelGGL((attn_kernel<HD, 2, SPEC, 512>), grid, dim3(512), 0, s, a);
            return hipGetLastError();
        }
    }
    // Short caches with four query heads per KV head (one float4 per lane,
    // 32-lane teams): 512 threads form 16 teams, one position each per
    // 16-position block instead of two at 256 threads, the same blocks and
    // splits.  4B decode attention 4.57 -> 4.31 us, the step 1.875 -> 1.865
    // ms; the per-row prefill attention (not SPEC) was slower with it.
    if constexpr (HD == 128 && SPEC) {
        if (a.nq / a.nkv == 4 && a.block == attn_chunk(HD, 4, kBlock, kAttnBlockShort) &&
            a.block == attn_chunk(HD, 4, 512, kAttnBlockShort)) {
            hipLaunchKernelGGL((attn_kernel<HD, 4, SPEC, 512, kAttnBlockShort>), grid, dim3(512), 0, s, a);
            return hipGetLastError();
        }
    }
    switch (a.nq / a.nkv) {
        case 1: return launch_attn_group<HD, 1, SPEC>(a, grid, s);
        case 2: return launch_attn_group<HD, 2, SPEC>(a, grid, s);
        case 4: return launch_attn_group<HD, 4, SPEC>(a, grid, s);
        case 8: return launch_attn_group<HD, 8, SPEC>(a, grid, s);
        default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------------------
// Step finalizer: the argmax of the step's logits becomes the next input
// token (generate's `next = argmax(logits)`, src/model.rs:636-637), is
// appended to the history, and the cache position advances.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(1024) void finalize_kernel(const FinalizeArgs a) {
    __shared__ unsigned long long red[16];
    unsigned long long best = kArgmaxInit;
    for (int i0 = threadIdx.x; i0 < a.nparts; i0 += 8 * blockDim.x) {
        unsigned long long k[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int i = i0 + u * blockDim.x;
            k[u] = i < a.nparts ? a.argmax_part[i] : 0ull;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) best = k[u] > best ? k[u] : best;
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
    const int stp = st->step;
    if (stp >= 0 && stp < a.hist_cap) a.history[stp] = tok;
    st->step = stp + 1;
    if (a.advance_pos) st->pos = st->pos + 1;
    st->argmax_key = kArgmaxInit;
}

// ---------------------------------------------------------------------------
// Batched greedy decode: the per-sequence argmax of a [B][V] logit block
// (generate's `next = argmax(logits)`, src/model.rs:636-637, for every
// sequence), one workgroup per sequence, same packed-key tie rule as the
// single-sequence path (largest value, lowest id; all -inf/NaN -> id 0).
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(1024) void batch_select_kernel(const BatchSelectArgs a) {
    __shared__ unsigned long long red[16];
    const int b = blockIdx.x;
    const float *row = a.logits + (size_t)b * a.V;
    unsigned long long best = kArgmaxInit;
    for (int i = threadIdx.x; i < a.V; i += blockDim.x) {
        const float v = row[i];
        if (v == v) {
            const unsigned long long k = argmax_key(v, (uint32_t)i);
            best = k > best ? k : best;
        }
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
    int tok = (int)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
    if (tok < 0 || tok >= a.V) tok = 0;
    a.tokens[b] = tok;
    const int p = a.pos[b];
    const int i = p - a.plen[b] + 1;  // index of the id chosen from position p's logits
    if (i >= 0 && i < a.out_stride) a.out[(size_t)b * a.out_stride + i] = tok;
    a.pos[b] = p + 1;
}

// Same selection from per-workgroup keys [B][nparts] of the multi-row
// lm_head GEMV.
__global__ __launch_bounds__(1024) void batch_select_parts_kernel(const unsigned long long *parts, int nparts,
                                                                  const BatchSelectArgs a) {
    __shared__ unsigned long long red[16];
    const int b = blockIdx.x;
    unsigned long long best = kArgmaxInit;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) {
        const unsigned long long k = parts[(size_t)b * nparts + i];
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
    int tok = (int)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
    if (tok < 0 || tok >= a.V) tok = 0;
    a.tokens[b] = tok;
    const int p = a.pos[b];
    const int i = p - a.plen[b] + 1;
    if (i >= 0 && i < a.out_stride) a.out[(size_t)b * a.out_stride + i] = tok;
    a.pos[b] = p + 1;
}

__global__ __launch_bounds__(1024) void batch_first_kernel(const unsigned long long *part, int nparts, int V, int b,
                                                           int *tokens, int *out, int out_stride) {
    __shared__ unsigned long long red[16];
    unsigned long long best = kArgmaxInit;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) best = part[i] > best ? part[i] : best;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = shfl_xor_u64(best, off);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) best = red[w] > best ? red[w] : best;
    int tok = (int)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
    if (tok < 0 || tok >= V) tok = 0;
    tokens[b] = tok;
    out[(size_t)b * out_stride] = tok;
}

}  // namespace

hipError_t launch_batch_select(const BatchSelectArgs &a, hipStream_t s) {
    if (a.B <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(batch_select_kernel, dim3(a.B), dim3(1024), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_gemv_mt(int pro, int epi, const GemvArgs &a, hipStream_t s) {
    if (a.nb < 1 || a.nb > kMtMaxSeq || a.W8) return hipErrorInvalidValue;
    if (pro == PRO_NORM && epi == EPI_QKV) return launch_mt_pe<PRO_NORM, EPI_QKV>(a, s);
    if (pro == PRO_PLAIN && epi == EPI_RESID) return launch_mt_pe<PRO_PLAIN, EPI_RESID>(a, s);
    if (pro == PRO_NORM && epi == EPI_SWIGLU) return launch_mt_pe<PRO_NORM, EPI_SWIGLU>(a, s);
    if (pro == PRO_NORM && epi == EPI_LOGITS) return launch_mt_pe<PRO_NORM, EPI_LOGITS>(a, s);
    return hipErrorInvalidValue;
}

int gemv_mt_blocks(int out, int in, int nb) {
    const int kc = (in + kChunk - 1) / kChunk;
    const int R = gemv_mt_rows(kc, gemv_mt_group(kc, nb));
    return (out + R - 1) / R;
}

hipError_t launch_batch_select_parts(const unsigned long long *parts, int nparts, const BatchSelectArgs &a,
                                     hipStream_t s) {
    if (a.B <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(batch_select_parts_kernel, dim3(a.B), dim3(1024), 0, s, parts, nparts, a);
    return hipGetLastError();
}

hipError_t launch_batch_first(const unsigned long long *argmax_part, int nparts, int V, int b, int *tokens, int *out,
                              int out_stride, hipStream_t s) {
    hipLaunchKernelGGL(batch_first_kernel, dim3(1), dim3(1024), 0, s, argmax_part, nparts, V, b, tokens, out,
                       out_stride);
    return hipGetLastError();
}

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

hipError_t launch_quantize_i8(uint16_t *w, int rows, int in, int8_t *q8, float *scale, bool rewrite,
                              hipStream_t s) {
    if (rows <= 0 || in <= 0 || in % 8) return hipErrorInvalidValue;
    hipLaunchKernelGGL(quantize_i8_kernel, dim3(rows), dim3(kBlock), 0, s, w, in, q8, scale, rewrite ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_quantize_i8_f32(const float *w, int rows, int in, int8_t *q8, float *scale, uint16_t *codes,
                                  hipStream_t s) {
    if (rows <= 0 || in <= 0 || in % 8) return hipErrorInvalidValue;
    hipLaunchKernelGGL(quantize_i8_f32_kernel, dim3(rows), dim3(kBlock), 0, s, w, in, q8, scale, codes);
    return hipGetLastError();
}

hipError_t launch_attn(const AttnArgs &a, hipStream_t s) {
    const bool spec = a.pos_dev && a.cap > 0 && a.T == 1;
    switch (a.hd) {
        case 16: return spec ? launch_attn_hd<16, true>(a, s) : launch_attn_hd<16, false>(a, s);
        case 32: return spec ? launch_attn_hd<32, true>(a, s) : launch_attn_hd<32, false>(a, s);
        case 64: return spec ? launch_attn_hd<64, true>(a, s) : launch_attn_hd<64, false>(a, s);
        case 128: return spec ? launch_attn_hd<128, true>(a, s) : launch_attn_hd<128, false>(a, s);
        case 256: return spec ? launch_attn_hd<256, true>(a, s) : launch_attn_hd<256, false>(a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_attn_combine(const AttnArgs &a, hipStream_t s) {
    if (a.nsplit > kBlock || a.hd > kBlock || kBlock % a.hd != 0 || a.T < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(a.nq, a.T), dim3(kBlock), 0, s, a);
    return hipGetLastError();
}

int gemv_blocks(int out, int in, bool f32) {
    const int kc = (in + kChunk - 1) / kChunk;
    const int R = f32 ? (kc <= 1 ? 8 : kc <= 3 ? 4 : 2)  // gemv_rows_f32<KC>()
                      : (kc <= 3 ? 8 : 4);                // gemv_rows<KC>()
    return (out + R - 1) / R;
}

hipError_t launch_finalize(const FinalizeArgs &a, hipStream_t s) {
    hipLaunchKernelGGL(finalize_kernel, dim3(1), dim3(1024), 0, s, a);
    return hipGetLastError();
}

}  // namespace tmg
