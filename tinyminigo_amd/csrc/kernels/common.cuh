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

// Round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// x = hi + lo with hi = bf16(x), lo = bf16(x - hi): |x - hi - lo| <= 2^-18 |x|.
__device__ __forceinline__ void split_bf16(float x, uint16_t *hi, uint16_t *lo) {
    uint16_t h = f32_to_bf16_rne(x);
    *hi = h;
    *lo = f32_to_bf16_rne(x - bf16_to_f32(h));
}

// Cross-lane moves without LDS: DPP within rows of 16 lanes and the gfx950
// permlane swaps across rows.  For lane l:
//   xor1 / xor2      -> value of lane l^1 / l^2       (DPP quad_perm)
//   half_mirror      -> value of lane (l & ~7) | (7 - (l & 7))
//   ror8             -> value of lane l^8             (DPP row_ror:8)
//   permlane16_swap(a, b) -> {[a0-15, b0-15, a32-47, b32-47],
//                             [a16-31, b16-31, a48-63, b48-63]}
//   permlane32_swap(a, b) -> {[a0-31, b0-31], [a32-63, b32-63]}
template <class T>
__device__ __forceinline__ uint32_t as_u32(T v) {
    static_assert(sizeof(T) == 4, "32-bit lanes only");
    return __builtin_bit_cast(uint32_t, v);
}
template <class T>
__device__ __forceinline__ T from_u32(uint32_t u) {
    return __builtin_bit_cast(T, u);
}

template <int CTRL, class T>
__device__ __forceinline__ T dpp_mov(T v) {
    return from_u32<T>((uint32_t)__builtin_amdgcn_update_dpp(0, (int)as_u32(v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppRor8 = 0x128;       // row_ror:8

// x + (x of lane l^16), and x + (x of lane l^32)
template <class T>
__device__ __forceinline__ T add_xor16(T x) {
    const auto r = __builtin_amdgcn_permlane16_swap(as_u32(x), as_u32(x), false, false);
    return from_u32<T>(r[0]) + from_u32<T>(r[1]);
}
template <class T>
__device__ __forceinline__ T add_xor32(T x) {
    const auto r = __builtin_amdgcn_permlane32_swap(as_u32(x), as_u32(x), false, false);
    return from_u32<T>(r[0]) + from_u32<T>(r[1]);
}

// Sum within aligned groups of W lanes (W a power of two <= 64); every lane
// of a group receives the group's sum.  T is float or a 32-bit integer.
template <int W, class T>
__device__ __forceinline__ T group_sum(T v) {
    static_assert(W == 1 || W == 2 || W == 4 || W == 8 || W == 16 || W == 32 || W == 64, "W must be a power of two");
    if constexpr (W >= 2) v += dpp_mov<kDppXor1>(v);
    if constexpr (W >= 4) v += dpp_mov<kDppXor2>(v);
    if constexpr (W >= 8) v += dpp_mov<kDppHalfMirror>(v);  // quads hold equal values
    if constexpr (W >= 16) v += dpp_mov<kDppRor8>(v);
    if constexpr (W >= 32) v = add_xor16(v);
    if constexpr (W >= 64) v = add_xor32(v);
    return v;
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_mov<kDppXor1>(v));
    v = fmaxf(v, dpp_mov<kDppXor2>(v));
    v = fmaxf(v, dpp_mov<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_mov<kDppRor8>(v));
    {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    return v;
}

// log2 of a power-of-two count of values per lane, at most 64 (one per lane).
template <int R>
__host__ __device__ constexpr int log2_pow2() {
    static_assert(R == 1 || R == 2 || R == 4 || R == 8 || R == 16 || R == 32 || R == 64, "R must be 2^k <= 64");
    return R == 64 ? 6 : R == 32 ? 5 : R == 16 ? 4 : R == 8 ? 3 : R == 4 ? 2 : R == 2 ? 1 : 0;
}

// Reduce R values per lane across the 64-lane wavefront with a transposed
// butterfly: log2(R) exchange steps (lane halves 32 and 16 by permlane swaps,
// 8 by DPP) that halve the live values, then a plain butterfly within the
// remaining lane group.  On return every lane holds the wave sum of value
// (lane >> (6 - log2 R)).
template <int R, class T>
__device__ __forceinline__ T multi_wave_sum(T (&v)[R], int lane) {
    constexpr int LR = log2_pow2<R>();
    T cur[R];
#pragma unroll
    for (int i = 0; i < R; i++) cur[i] = v[i];
    if constexpr (LR >= 1) {  // lanes 32-63 keep values [R/2, R)
#pragma unroll
        for (int i = 0; i < R / 2; i++) {
            const auto r = __builtin_amdgcn_permlane32_swap(as_u32(cur[i]), as_u32(cur[i + R / 2]), false, false);
            cur[i] = from_u32<T>(r[0]) + from_u32<T>(r[1]);
        }
    }
    if constexpr (LR >= 2) {  // lanes with bit 4 set keep the upper half
#pragma unroll
        for (int i = 0; i < R / 4; i++) {
            const auto r = __builtin_amdgcn_permlane16_swap(as_u32(cur[i]), as_u32(cur[i + R / 4]), false, false);
            cur[i] = from_u32<T>(r[0]) + from_u32<T>(r[1]);
        }
    }
    if constexpr (LR >= 3) {  // lanes with bit 3 set keep the upper half
#pragma unroll
        for (int i = 0; i < R / 8; i++) {
            const bool up = (lane & 8) != 0;
            const T send = up ? cur[i] : cur[i + R / 8];
            const T keep = up ? cur[i + R / 8] : cur[i];
            cur[i] = keep + dpp_mov<kDppRor8>(send);
        }
    }
    if constexpr (LR >= 4) {  // lanes with bit 2 set keep the upper half; the
        // partner across the half-row mirror (7 - l within 8 lanes) has bit 2
        // clear and the same higher bits, so it holds the same values
#pragma unroll
        for (int i = 0; i < R / 16; i++) {
            const bool up = (lane & 4) != 0;
            const T send = up ? cur[i] : cur[i + R / 16];
            const T keep = up ? cur[i + R / 16] : cur[i];
            cur[i] = keep + dpp_mov<kDppHalfMirror>(send);
        }
    }
    if constexpr (LR >= 5) {  // bit 1, partner l ^ 2
#pragma unroll
        for (int i = 0; i < R / 32; i++) {
            const bool up = (lane & 2) != 0;
            const T send = up ? cur[i] : cur[i + R / 32];
            const T keep = up ? cur[i + R / 32] : cur[i];
            cur[i] = keep + dpp_mov<kDppXor2>(send);
        }
    }
    if constexpr (LR >= 6) {  // bit 0, partner l ^ 1
        const bool up = (lane & 1) != 0;
        const T send = up ? cur[0] : cur[1];
        const T keep = up ? cur[1] : cur[0];
        cur[0] = keep + dpp_mov<kDppXor1>(send);
    }
    return group_sum<(64 >> LR)>(cur[0]);
}

// Block reductions of N values at once over NW wavefronts (256 threads by
// default); every thread receives the results.  `scratch` must hold NW*N
// floats.  The wave sums are added as ((w0 + w1) + (w2 + w3)) + w4 + ...
template <int N, int NW = kBlock / 64>
__device__ __forceinline__ void block_sum_n(float (&v)[N], float *scratch) {
    static_assert(NW >= 4, "at least four wavefronts");
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = wave_sum(v[i]);
    if (l == 0)
#pragma unroll
        for (int i = 0; i < N; i++) scratch[w * N + i] = v[i];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; i++) {
        float s = (scratch[i] + scratch[N + i]) + (scratch[2 * N + i] + scratch[3 * N + i]);
#pragma unroll
        for (int k = 4; k < NW; k++) s += scratch[k * N + i];
        v[i] = s;
    }
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

// Argmax key of a non-NaN value: -0.0 and +0.0 share one key, since the
// reference's `v > best` treats them as equal (the first one wins).
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx) {
    const uint32_t o = v == 0.0f ? 0x80000000u : f32_order(v);
    return ((unsigned long long)o << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
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
// (HIP's __fmul_rn / __fsub_rn are plain operators compiled where
// contraction is on; the operators written under the pragma are not fused.)
__device__ __forceinline__ void rope_pair(float a, float b, float c, float s, float *oa, float *ob) {
#pragma clang fp contract(off)
    *oa = a * c - b * s;
    *ob = a * s + b * c;
}

}  // namespace tmg
