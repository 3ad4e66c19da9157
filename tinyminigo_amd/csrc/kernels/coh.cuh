// Device-scope loads and stores for data exchanged between workgroups of one
// launch (the split-K partials of the short-prompt prefill GEMM).  MI355X
// has one L2 per XCD and they are not coherent with each other, so such data
// is accessed with device-scope (sc1) operations -- the code the compiler
// emits for agent-scope relaxed atomics -- instead of cached ones.  Data
// produced by an earlier launch needs none of this: the kernel boundary
// writes back and invalidates the caches.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tmg {

__device__ __forceinline__ float ld_dev(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void st_dev(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace tmg
