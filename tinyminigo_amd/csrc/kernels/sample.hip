// On-device token selection for gfx950 (reference generate,
// src/model.rs:631-646; apply_repetition_penalty, src/tensor.rs:1142-1154;
// sample, src/tensor.rs:1157-1213).
//
// Top-k path (0 < k <= kSampleMaxK, or greedy with a repetition penalty):
//   pass 1, one workgroup per 2048-id slice: penalty, temperature, and a
//   bitonic sort of packed (value, id) keys in LDS; the slice's best k keys
//   are written out.
//   pass 2, one workgroup: bitonic sort of all slice winners, then one lane
//   runs the reference's sequential tail over the k candidates in order:
//   softmax (max, exp, sequential sum, divide), nucleus cut at the first
//   cumulative sum > top_p, renormalization, and the inverse-CDF walk.
// Full-vocabulary path (no top-k, top_p >= 1): one workgroup computes the
// softmax and finds the draw with a block prefix sum in id order.
//
// Keys order by value descending, then id ascending, which is the reference
// argmax tie rule; the reference's sort_unstable_by leaves equal-value order
// unspecified, so any order among exact ties is as faithful as another.
#include "common.cuh"
#include "kernels.hpp"

namespace tmg {
namespace {

constexpr unsigned long long kGamma = 0x9E3779B97F4A7C15ull;

__device__ __forceinline__ unsigned long long mix64(unsigned long long z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Uniform f32 in [0, 1) with 24 random bits, draw `i` of stream `key`.
__device__ __forceinline__ float uniform_f32(unsigned long long key, unsigned long long i) {
    return (float)(mix64(key + (i + 1) * kGamma) >> 40) * 0x1.0p-24f;
}

__device__ __forceinline__ float key_value(unsigned long long key) {
    uint32_t o = (uint32_t)(key >> 32);
    uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
    return __uint_as_float(u);
}
__device__ __forceinline__ int key_index(unsigned long long key) { return (int)(0xFFFFFFFFu - (uint32_t)key); }

// Penalized (and, when sampling, temperature-scaled) logit of id i.
__device__ __forceinline__ float adjusted(const float *logits, const unsigned *seen, const DevState &st, int i,
                                          bool greedy) {
    float v = logits[i];
    if (st.penalty != 1.0f && seen && ((seen[i >> 5] >> (i & 31)) & 1u))
        v = v > 0.0f ? __fdiv_rn(v, st.penalty) : __fmul_rn(v, st.penalty);
    if (!greedy) v = __fdiv_rn(v, st.temperature);
    return v;
}

// Bitonic sort of n (power of two) keys in LDS, descending.
__device__ void bitonic_desc(unsigned long long *k, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int i = threadIdx.x; i < n / 2; i += blockDim.x) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool desc = ((lo & size) == 0);
                const unsigned long long a = k[lo], b = k[hi];
                if (desc ? (a < b) : (a > b)) {
                    k[lo] = b;
                    k[hi] = a;
                }
            }
        }
    }
    __syncthreads();
}

__global__ __launch_bounds__(kBlock) void sample_partial_kernel(const SampleArgs a) {
    __shared__ unsigned long long keys[kSampleSlice];
    const DevState st = *a.st;
    const bool greedy = a.greedy != 0;
    const int K = greedy ? 1 : st.top_k;
    const int base = blockIdx.x * kSampleSlice;
    for (int j = threadIdx.x; j < kSampleSlice; j += kBlock) {
        const int i = base + j;
        unsigned long long key = 0ull;
        if (i < a.V) {
            const float v = adjusted(a.logits, a.seen, st, i, greedy);
            if (v == v) key = argmax_key(v, (uint32_t)i);
        }
        keys[j] = key;
    }
    bitonic_desc(keys, kSampleSlice);
    for (int j = threadIdx.x; j < K; j += kBlock) a.cand[(size_t)blockIdx.x * kSampleMaxK + j] = keys[j];
}

__device__ void emit_token(const SampleArgs &a, int tok) {
    if (tok < 0 || tok >= a.V) tok = 0;  // only reachable when every logit is NaN
    DevState *st = a.st;
    st->cur_token = tok;
    const int stp = st->step;
    if (stp >= 0 && stp < a.hist_cap) a.history[stp] = tok;
    st->step = stp + 1;
    if (a.advance_pos) st->pos = st->pos + 1;
    st->argmax_key = kArgmaxInit;
    a.seen_rw[tok >> 5] |= 1u << (tok & 31);
}

__global__ __launch_bounds__(1024) void sample_select_kernel(const SampleArgs a, int nslices, int npad) {
    extern __shared__ unsigned long long cand[];
    __shared__ float probs[kSampleMaxK];
    const DevState st = *a.st;
    const bool greedy = a.greedy != 0;
    const int K = greedy ? 1 : st.top_k;
    for (int i = threadIdx.x; i < npad; i += blockDim.x) {
        const int sl = i / K, j = i - sl * K;
        cand[i] = (sl < nslices) ? a.cand[(size_t)sl * kSampleMaxK + j] : 0ull;
    }
    bitonic_desc(cand, npad);
    if (threadIdx.x != 0) return;
    if (greedy) {
        // all -inf/NaN logits leave key 0 on top: the reference returns 0
        const unsigned long long top = cand[0];
        emit_token(a, top ? key_index(top) : 0);
        return;
    }
    // softmax over the k candidates in candidate order (src/tensor.rs:1177-1179)
    const float mx = key_value(cand[0]);
    float sum = 0.0f;
    for (int i = 0; i < K; i++) {
        probs[i] = expf(key_value(cand[i]) - mx);
        sum += probs[i];
    }
    for (int i = 0; i < K; i++) probs[i] = probs[i] / sum;
    // nucleus (src/tensor.rs:1182-1201): candidates are already in descending
    // probability order
    if (st.top_p < 1.0f) {
        float cum = 0.0f;
        int cutoff = K;
        for (int r = 0; r < K; r++) {
            cum += probs[r];
            if (cum > st.top_p) {
                cutoff = r + 1;
                break;
            }
        }
        float s2 = 0.0f;
        for (int r = 0; r < cutoff; r++) s2 += probs[r];
        for (int r = 0; r < K; r++) probs[r] = r < cutoff ? probs[r] / s2 : 0.0f;
    }
    // inverse-CDF walk in candidate order (src/tensor.rs:1203-1212)
    const float r = uniform_f32(st.seed, (unsigned long long)st.step);
    float cum = 0.0f;
    int pick = -1;
    for (int i = 0; i < K; i++) {
        cum += probs[i];
        if (r < cum) {
            pick = i;
            break;
        }
    }
    if (pick < 0) {
        pick = 0;
        for (int i = 0; i < K; i++)
            if (probs[i] > 0.0f) {
                pick = i;
                break;
            }
    }
    emit_token(a, key_index(cand[pick]));
}

// No top-k: candidates are all ids in id order (src/tensor.rs:1169-1179).
__global__ __launch_bounds__(1024) void sample_full_kernel(const SampleArgs a) {
    __shared__ float red[32];
    __shared__ float pre[1024];
    const DevState st = *a.st;
    const int nt = blockDim.x, t = threadIdx.x;
    const int per = (a.V + nt - 1) / nt;
    const int b = min(a.V, t * per), e = min(a.V, b + per);
    float mx = -INFINITY;
    for (int i = b; i < e; i++) mx = fmaxf(mx, adjusted(a.logits, a.seen, st, i, false));
    // block max
    mx = wave_max(mx);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    if (t < 64) {
        float v = t < (nt >> 6) ? red[t] : -INFINITY;
        v = wave_max(v);
        if (t == 0) red[16] = v;
    }
    __syncthreads();
    const float M = red[16];
    __syncthreads();
    float s = 0.0f;
    for (int i = b; i < e; i++) s += expf(adjusted(a.logits, a.seen, st, i, false) - M);
    float ws = wave_sum(s);
    if ((t & 63) == 0) red[t >> 6] = ws;
    __syncthreads();
    if (t < 64) {
        float v = t < (nt >> 6) ? red[t] : 0.0f;
        v = wave_sum(v);
        if (t == 0) red[17] = v;
    }
    __syncthreads();
    const float S = red[17];
    // per-thread sums of probabilities, then an exclusive prefix in id order
    float c = 0.0f;
    for (int i = b; i < e; i++) c += expf(adjusted(a.logits, a.seen, st, i, false) - M) / S;
    pre[t] = c;
    __syncthreads();
    if (t == 0) {
        const float r = uniform_f32(st.seed, (unsigned long long)st.step);
        float cum = 0.0f;
        int pick = -1;
        for (int th = 0; th < nt && pick < 0; th++) {
            if (r < cum + pre[th]) {
                const int bb = min(a.V, th * per), ee = min(a.V, bb + per);
                for (int i = bb; i < ee; i++) {
                    cum += expf(adjusted(a.logits, a.seen, st, i, false) - M) / S;
                    if (r < cum) {
                        pick = i;
                        break;
                    }
                }
            } else {
                cum += pre[th];
            }
        }
        if (pick < 0) {
            pick = 0;
            for (int i = 0; i < a.V; i++)
                if (expf(adjusted(a.logits, a.seen, st, i, false) - M) / S > 0.0f) {
                    pick = i;
                    break;
                }
        }
        emit_token(a, pick);
    }
}

}  // namespace

hipError_t launch_sample(const SampleArgs &a, hipStream_t s) {
    const int nslices = (a.V + kSampleSlice - 1) / kSampleSlice;
    if (a.greedy || a.cand) {
        // top-k (or greedy) path; the host only sets cand when top_k is usable
        hipLaunchKernelGGL(sample_partial_kernel, dim3(nslices), dim3(kBlock), 0, s, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        // npad: power of two covering nslices * kSampleMaxK (worst case k)
        int npad = 1;
        while (npad < nslices * kSampleMaxK) npad <<= 1;
        hipLaunchKernelGGL(sample_select_kernel, dim3(1), dim3(1024), (size_t)npad * 8, s, a, nslices, npad);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(sample_full_kernel, dim3(1), dim3(1024), 0, s, a);
    return hipGetLastError();
}

}  // namespace tmg
