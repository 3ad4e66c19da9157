// argmax over a device vector (reference tensor::argmax, src/tensor.rs:1063-1073):
// the index of the first maximum.  `v > best` skips NaN, keeps the first of
// equal values (-0.0 and +0.0 are equal) and leaves index 0 when every value
// is -inf or NaN (or the vector is empty).
//
// Two passes: argmax_partial_kernel reduces each 4096-element chunk to one
// packed key (orderable value bits << 32 | 0xFFFFFFFF - index, so the larger
// key is the larger value and, among equal values, the lower index) in a
// scratch array; argmax_final_kernel reduces the chunk keys and writes the
// index.  The decode step's lm_head epilogue and finalize_kernel use the same
// key (common.cuh).
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "../host/common.hpp"
#include "common.cuh"
#include "kernels.hpp"

namespace tmg {
namespace {

constexpr int kArgmaxPerThread = 16;
constexpr int kArgmaxChunk = kBlock * kArgmaxPerThread;  // elements per partial key

__device__ __forceinline__ unsigned long long block_max_key(unsigned long long best, unsigned long long *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = shfl_xor_u64(best, off);
        best = o > best ? o : best;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    best = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) best = red[w] > best ? red[w] : best;
    return best;
}

__global__ __launch_bounds__(kBlock) void argmax_partial_kernel(const float *x, uint32_t n, unsigned long long *part) {
    __shared__ unsigned long long red[kBlock / 64];
    const size_t base = (size_t)blockIdx.x * kArgmaxChunk;
    float v[kArgmaxPerThread];
#pragma unroll
    for (int j = 0; j < kArgmaxPerThread; j++) {
        const size_t i = base + (size_t)j * kBlock + threadIdx.x;
        v[j] = i < n ? x[i] : __builtin_nanf("");
    }
    unsigned long long best = 0ull;  // below every real key
#pragma unroll
    for (int j = 0; j < kArgmaxPerThread; j++) {
        if (v[j] == v[j]) {
            const unsigned long long k = argmax_key(v[j], (uint32_t)(base + (size_t)j * kBlock + threadIdx.x));
            best = k > best ? k : best;
        }
    }
    best = block_max_key(best, red);
    if (threadIdx.x == 0) part[blockIdx.x] = best;
}

__global__ __launch_bounds__(kBlock) void argmax_final_kernel(const unsigned long long *part, uint32_t nparts,
                                                             uint32_t *out) {
    __shared__ unsigned long long red[kBlock / 64];
    unsigned long long best = kArgmaxInit;  // (-inf, index 0)
    for (uint32_t i = threadIdx.x; i < nparts; i += kBlock) best = part[i] > best ? part[i] : best;
    best = block_max_key(best, red);
    if (threadIdx.x == 0) *out = 0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull);
}

}  // namespace

// Chunk keys of tmg_argmax_f32_noalloc: one array per GPU, held until the
// process ends (32 KiB: 4096 keys cover n <= 4096 * 4096 = 16,777,216).
constexpr uint32_t kNoAllocParts = 4096;
static __device__ __align__(256) unsigned long long scratch[kNoAllocParts];

uint32_t argmax_parts(uint32_t n) { return (uint32_t)(((uint64_t)n + kArgmaxChunk - 1) / kArgmaxChunk); }

hipError_t launch_argmax(const float *x, uint32_t n, uint32_t *out, unsigned long long *part, hipStream_t s) {
    const uint32_t np = argmax_parts(n);
    if (np) hipLaunchKernelGGL(argmax_partial_kernel, dim3(np), dim3(kBlock), 0, s, x, n, part);
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kBlock), 0, s, (const unsigned long long *)part, np, out);
    return hipGetLastError();
}

}  // namespace tmg

using namespace tmg;

// Kernel level argmax; the chunk keys live in a buffer allocated on `stream`
// for the call (stream-ordered allocation, freed after the final pass).
extern "C" int tmg_argmax_f32(const float *x_dev, uint32_t n, uint32_t *out_dev, void *stream) {
    clear_error();
    if (!out_dev || (n && !x_dev)) return set_error(TMG_E_INVALID, "null argument to tmg_argmax_f32");
    hipStream_t s = (hipStream_t)stream;
    const uint32_t np = argmax_parts(n);
    void *part = nullptr;
    if (np) {
        hipError_t e = hipMallocAsync(&part, (size_t)np * sizeof(unsigned long long), s);
        if (e != hipSuccess)
            return set_error(TMG_E_NOMEM, std::string("hipMallocAsync of the argmax chunk keys failed: ") +
                                              hipGetErrorString(e));
    }
    hipError_t e = launch_argmax(x_dev, n, out_dev, (unsigned long long *)part, s);
    if (part) {
        const hipError_t f = hipFreeAsync(part, s);
        if (e == hipSuccess) e = f;
    }
    if (e != hipSuccess) return set_error(TMG_E_DEVICE, std::string("tmg_argmax_f32: ") + hipGetErrorString(e));
    return TMG_OK;
}

// tmg_argmax_f32 without any allocation: the chunk keys go to this GPU's
// `scratch` array.  Its device address is looked up once per device, with
// that device current, on the first call there (host code never passes the
// array's name itself: on the host it is only a stand-in symbol).
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned long long *g_scratch[kMaxDevices] = {};

int noalloc_scratch(unsigned long long **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(TMG_E_DEVICE, std::string("hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return set_error(TMG_E_DEVICE, "device index beyond the no-alloc table");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(TMG_E_DEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        g_scratch[dev] = (unsigned long long *)p;
    }
    *out = g_scratch[dev];
    return TMG_OK;
}
}  // namespace

extern "C" int tmg_argmax_f32_noalloc(const float *x_dev, uint32_t n, uint32_t *out_dev, void *stream) {
    clear_error();
    if (!out_dev || (n && !x_dev)) return set_error(TMG_E_INVALID, "null argument to tmg_argmax_f32_noalloc");
    if (argmax_parts(n) > kNoAllocParts)
        return set_error(TMG_E_INVALID, "tmg_argmax_f32_noalloc: n = " + std::to_string(n) + " exceeds its maximum of " +
                                            std::to_string((uint64_t)kNoAllocParts * kArgmaxChunk) + " elements");
    unsigned long long *part = nullptr;
    int rc = noalloc_scratch(&part);
    if (rc) return rc;
    // every key the final pass reads is written by this call's first pass,
    // so the array needs no clearing between calls
    const hipError_t e = launch_argmax(x_dev, n, out_dev, part, (hipStream_t)stream);
    if (e != hipSuccess) return set_error(TMG_E_DEVICE, std::string("tmg_argmax_f32_noalloc: ") + hipGetErrorString(e));
    return TMG_OK;
}
