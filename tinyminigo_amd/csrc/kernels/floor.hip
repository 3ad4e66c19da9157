// The decode step's floor, measured on the device (no counterpart in the
// reference; measurement only): a streaming phase is what one kernel of the
// step would cost if it only streamed its bytes.  Workgroup b of a phase
// reads `nchunk` chunks of NB 4-KiB blocks of its own weights (one 16-byte
// nontemporal load per thread per block, all NB loads of a chunk in flight),
// dots them as BF16 pairs with 8 floats of the previous phase's output
// (act[t*8 .. t*8+7]: a dependent load, as every phase of the step has one),
// reduces across the workgroup and writes out[b].  Phases launched in the
// step's order, each with the grid and bytes of the kernel it stands for,
// form a chain with the step's launches and weight stream and none of its
// other work (norm prologues, epilogues, split merges).
#include <hip/hip_runtime.h>

#include "common.cuh"
#include "kernels.hpp"

namespace tmg {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int NB>
__global__ __launch_bounds__(kBlock) void stream_phase_kernel(const u32x4 *w, int nchunk, const float *act,
                                                              float *out) {
    __shared__ float red[kBlock / 64];
    const int t = threadIdx.x;
    const u32x4 *p = w + (size_t)blockIdx.x * nchunk * NB * 256 + t;
    const float4 a0 = *reinterpret_cast<const float4 *>(act + t * 8);
    const float4 a1 = *reinterpret_cast<const float4 *>(act + t * 8 + 4);
    float s = 0.0f;
    for (int c = 0; c < nchunk; c++, p += NB * 256) {
        u32x4 r[NB];
#pragma unroll
        for (int i = 0; i < NB; i++) r[i] = __builtin_nontemporal_load(p + i * 256);
#pragma unroll
        for (int i = 0; i < NB; i++)
            s += a0.x * bf16_lo(r[i].x) + a0.y * bf16_hi(r[i].x) + a0.z * bf16_lo(r[i].y) + a0.w * bf16_hi(r[i].y) +
                 a1.x * bf16_lo(r[i].z) + a1.y * bf16_hi(r[i].z) + a1.z * bf16_lo(r[i].w) + a1.w * bf16_hi(r[i].w);
    }
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if ((t & 63) == 0) red[t >> 6] = s;
    __syncthreads();
    if (t == 0) out[blockIdx.x] = (red[0] + red[1] + red[2] + red[3]) * (1.0f / 4096.0f) + 0.25f;
}

__global__ __launch_bounds__(kBlock) void empty_kernel() {}

}  // namespace

hipError_t launch_stream_phase(const void *w, int nwg, int nb, int nchunk, const float *act, float *out,
                               hipStream_t s) {
    if (nwg < 1 || nchunk < 1) return hipErrorInvalidValue;
    const u32x4 *wv = static_cast<const u32x4 *>(w);
    switch (nb) {
#define TMG_PHASE(N) \
    case N: stream_phase_kernel<N><<<nwg, kBlock, 0, s>>>(wv, nchunk, act, out); break;
        TMG_PHASE(1) TMG_PHASE(2) TMG_PHASE(3) TMG_PHASE(4) TMG_PHASE(5) TMG_PHASE(6) TMG_PHASE(7) TMG_PHASE(8)
        TMG_PHASE(9) TMG_PHASE(10) TMG_PHASE(11) TMG_PHASE(12) TMG_PHASE(13) TMG_PHASE(14) TMG_PHASE(15)
        TMG_PHASE(16) TMG_PHASE(17) TMG_PHASE(18) TMG_PHASE(19) TMG_PHASE(20) TMG_PHASE(21) TMG_PHASE(22)
        TMG_PHASE(23) TMG_PHASE(24) TMG_PHASE(25) TMG_PHASE(26) TMG_PHASE(27) TMG_PHASE(28) TMG_PHASE(29)
        TMG_PHASE(30) TMG_PHASE(31) TMG_PHASE(32)
#undef TMG_PHASE
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_empty(int nwg, hipStream_t s) {
    empty_kernel<<<nwg, kBlock, 0, s>>>();
    return hipGetLastError();
}

}  // namespace tmg
