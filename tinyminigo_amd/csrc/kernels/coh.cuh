// Loads and stores of data exchanged between workgroups of one persistent
// launch.  MI355X has one L2 per XCD and they are not coherent with each
// other, so such data is accessed with device-scope (sc1) operations -- the
// code the compiler emits for agent-scope relaxed atomics -- instead of
// cached ones.  With COH = false they are ordinary accesses, for kernels whose
// producers ran in an earlier launch.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tmg {

template <bool COH>
__device__ __forceinline__ float ldf(const float *p) {
    if constexpr (COH)
        return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        return *p;
}

template <bool COH>
__device__ __forceinline__ void stf(float *p, float v) {
    if constexpr (COH)
        __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *p = v;
}

template <bool COH>
__device__ __forceinline__ float4 ldf4(const float *p) {
    if constexpr (COH)
        return make_float4(ldf<true>(p), ldf<true>(p + 1), ldf<true>(p + 2), ldf<true>(p + 3));
    else
        return *reinterpret_cast<const float4 *>(p);
}

template <bool COH>
__device__ __forceinline__ void stf4(float *p, float4 v) {
    if constexpr (COH) {
        stf<true>(p, v.x);
        stf<true>(p + 1, v.y);
        stf<true>(p + 2, v.z);
        stf<true>(p + 3, v.w);
    } else {
        *reinterpret_cast<float4 *>(p) = v;
    }
}

template <bool COH>
__device__ __forceinline__ unsigned long long ldu64(const unsigned long long *p) {
    if constexpr (COH)
        return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        return *p;
}

template <bool COH>
__device__ __forceinline__ void stu64(unsigned long long *p, unsigned long long v) {
    if constexpr (COH)
        __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        *p = v;
}

}  // namespace tmg
