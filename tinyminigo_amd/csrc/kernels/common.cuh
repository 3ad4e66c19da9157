// Device helpers shared by the gfx950 kernels: BF16 unpacking, 64-lane
// wavefront reductions and 256-thread block reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tmg {

constexpr int kBlock = 256;  // 4 wavefronts of 64 lanes

// Two BF16 values packed in one u32 widen exactly by shifting into the high
// half of an f32 (the reference's `bits << 16`, src/tensor.rs:85-88).
__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// x = hi + lo with hi = bf16(x), lo = bf16(x - hi): |x - hi - lo| <= 2^-18 |x|.
__device__ __forceinline__ void split_bf16(float x, uint16_t *hi, uint16_t *lo) {
    uint16_t h = f32_to_bf16_rne(x);
    *hi = h;
    *lo = f32_to_bf16_rne(x - bf16_to_f32(h));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Sum within aligned groups of W lanes (W a power of two <= 64).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Reduce R values per lane across the 64-lane wavefront with a transposed
// butterfly (log2(R) exchange steps that halve the live values, then a plain
// butterfly): 10 shuffles for R = 8 instead of 48.  On return every lane
// holds the wave sum of value (lane >> (6 - log2 R)).
template <int R>
__device__ __forceinline__ float multi_wave_sum(float (&v)[R], int lane) {
    static_assert(R == 1 || R == 2 || R == 4 || R == 8, "R must be 1, 2, 4 or 8");
    constexpr int LR = R == 8 ? 3 : R == 4 ? 2 : R == 2 ? 1 : 0;
    float cur[R];
#pragma unroll
    for (int i = 0; i < R; i++) cur[i] = v[i];
#pragma unroll
    for (int s = 0; s < LR; s++) {
        const int off = 32 >> s;
        const bool up = (lane & off) != 0;
        const int n = R >> (s + 1);
#pragma unroll
        for (int i = 0; i < n; i++) {
            float send = up ? cur[i] : cur[i + n];
            float keep = up ? cur[i + n] : cur[i];
            cur[i] = keep + __shfl_xor(send, off, 64);
        }
    }
    float x = cur[0];
#pragma unroll
    for (int off = 32 >> LR; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
    return x;
}

// Block (256-thread) reductions of N values at once; every thread receives
// the results.  `scratch` must hold 4*N floats.
template <int N>
__device__ __forceinline__ void block_sum_n(float (&v)[N], float *scratch) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = wave_sum(v[i]);
    if (l == 0)
#pragma unroll
        for (int i = 0; i < N; i++) scratch[w * N + i] = v[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = (scratch[i] + scratch[N + i]) + (scratch[2 * N + i] + scratch[3 * N + i]);
    __syncthreads();
}

template <int N>
__device__ __forceinline__ void block_max_n(float (&v)[N], float *scratch) {
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = wave_max(v[i]);
    if (l == 0)
#pragma unroll
        for (int i = 0; i < N; i++) scratch[w * N + i] = v[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; i++)
        v[i] = fmaxf(fmaxf(scratch[i], scratch[N + i]), fmaxf(scratch[2 * N + i], scratch[3 * N + i]));
    __syncthreads();
}

// Orderable key of an f32 for unsigned comparison (NaN excluded by callers).
__device__ __forceinline__ uint32_t f32_order(float v) {
    uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    return ((unsigned long long)f32_order(v) << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int off) {
    uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
    lo = __shfl_xor(lo, off, 64);
    hi = __shfl_xor(hi, off, 64);
    return ((unsigned long long)hi << 32) | lo;
}

// SiLU(g) * u in the reference's order: (g / (1 + exp(-g))) * u
// (src/model.rs:473-475).
__device__ __forceinline__ float swiglu(float g, float u) { return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), u); }

// rotate_half RoPE of the pair (a, b) = (v[i], v[i+hd/2]) without FMA
// contraction, as the reference computes it (src/tensor.rs:1031-1036).
__device__ __forceinline__ void rope_pair(float a, float b, float c, float s, float *oa, float *ob) {
    *oa = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s));
    *ob = __fadd_rn(__fmul_rn(a, s), __fmul_rn(b, c));
}

}  // namespace tmg
