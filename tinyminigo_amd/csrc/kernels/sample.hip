// On-device token selection for gfx950 (reference generate,
// src/model.rs:631-646; apply_repetition_penalty, src/tensor.rs:1142-1154;
// sample, src/tensor.rs:1157-1213).
//
// Top-k path (0 < k <= kSampleMaxK, or greedy with a repetition penalty):
//   pass 1, one workgroup per 2048-id slice: penalty and temperature, then a
//   radix select over the packed (value, id) keys held in registers (8-bit
//   digits from the top, LDS histograms) finds the slice's k-th largest key;
//   the slice's best k keys are written out unordered.
//   pass 2, one workgroup: the same radix select over all slice winners, the
//   k selected keys sorted by one wavefront (register bitonic sort), then one
//   lane runs the reference's sequential tail over the k candidates in
//   order: softmax (max, exp, sequential sum, divide), nucleus cut at the
//   first cumulative sum > top_p, renormalization, and the inverse-CDF walk.
// Full-vocabulary path (no top-k, top_p >= 1): one workgroup computes the
// softmax and finds the draw with a block prefix sum in id order.
//
// Keys order by value descending, then id ascending, which is the reference
// argmax tie rule; the reference's sort_unstable_by leaves equal-value order
// unspecified, so any order among exact ties is as faithful as another.
// Keys are unique (they contain the id), so the top k set is exact.
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

// Radix select state shared by a workgroup.
struct RadixSel {
    unsigned hist[256];
    int digit, above, count, n;
};

// Finds the k-th largest of the KPT keys each thread holds (k >= 1, at most
// the number of keys): on return every thread has (prefix, mask) such that
// the selected keys are exactly those with (key & mask) >= prefix, where mask
// covers the top bits decided.  8-bit digits from the most significant;
// stops as soon as the whole bin holding the k-th key is selected.
template <int KPT>
__device__ void radix_select(const unsigned long long (&key)[KPT], int k, RadixSel &rs, unsigned long long &prefix,
                             unsigned long long &mask) {
    const int t = threadIdx.x, nt = blockDim.x;
    prefix = 0;
    mask = 0;
    int remaining = k;
    for (int shift = 56; shift >= 0; shift -= 8) {
        for (int i = t; i < 256; i += nt) rs.hist[i] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < KPT; j++)
            if ((key[j] & mask) == prefix) atomicAdd(&rs.hist[(key[j] >> shift) & 255], 1u);
        __syncthreads();
        if (t < 64) {
            // lane l holds digits 255 - 4l .. 252 - 4l, high digits first
            unsigned c[4], sum = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                c[j] = rs.hist[255 - 4 * t - j];
                sum += c[j];
            }
            // exclusive prefix over lanes by shuffles
            unsigned incl = sum;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const unsigned o = __shfl_up(incl, off, 64);
                if (t >= off) incl += o;
            }
            unsigned cum = incl - sum;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (cum < (unsigned)remaining && cum + c[j] >= (unsigned)remaining) {
                    rs.digit = 255 - 4 * t - j;
                    rs.above = (int)cum;
                    rs.count = (int)c[j];
                }
                cum += c[j];
            }
        }
        __syncthreads();
        const int d = rs.digit;
        remaining -= rs.above;
        prefix |= (unsigned long long)d << shift;
        mask |= 255ull << shift;
        const bool done = rs.count == remaining;
        __syncthreads();  // rs is rewritten by the next round
        if (done) break;
    }
}

// Writes the selected keys (at most k; extra ties among padding keys are
// dropped) to out[0 ..) in arbitrary order.
template <int KPT>
__device__ void radix_compact(const unsigned long long (&key)[KPT], int k, unsigned long long prefix,
                              unsigned long long mask, RadixSel &rs, unsigned long long *out) {
    if (threadIdx.x == 0) rs.n = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < KPT; j++) {
        if ((key[j] & mask) >= prefix) {
            const int pos = atomicAdd(&rs.n, 1);
            if (pos < k) out[pos] = key[j];
        }
    }
}

__global__ __launch_bounds__(kBlock) void sample_partial_kernel(const SampleArgs a) {
    __shared__ RadixSel rs;
    constexpr int KPT = kSampleSlice / kBlock;
    const DevState st = *a.st;
    const bool greedy = a.greedy != 0;
    const int K = greedy ? 1 : st.top_k;
    const int base = blockIdx.x * kSampleSlice;
    unsigned long long key[KPT];
#pragma unroll
    for (int j = 0; j < KPT; j++) {
        const int i = base + j * kBlock + threadIdx.x;
        key[j] = 0ull;
        if (i < a.V) {
            const float v = adjusted(a.logits, a.seen, st, i, greedy);
            if (v == v) key[j] = argmax_key(v, (uint32_t)i);
        }
    }
    unsigned long long prefix, mask;
    radix_select<KPT>(key, K, rs, prefix, mask);
    radix_compact<KPT>(key, K, prefix, mask, rs, a.cand + (size_t)blockIdx.x * kSampleMaxK);
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

__global__ __launch_bounds__(1024) void sample_select_kernel(const SampleArgs a, int nslices) {
    __shared__ RadixSel rs;
    __shared__ unsigned long long cand[kSampleMaxK];
    __shared__ float probs[kSampleMaxK];
    constexpr int KPT = kSampleSelectKeys / 1024;
    const DevState st = *a.st;
    const bool greedy = a.greedy != 0;
    const int K = greedy ? 1 : st.top_k;
    const int n = nslices * K;
    unsigned long long key[KPT];
#pragma unroll
    for (int j = 0; j < KPT; j++) {
        const int i = j * 1024 + threadIdx.x;
        const int sl = i / K, jj = i - sl * K;
        key[j] = i < n ? a.cand[(size_t)sl * kSampleMaxK + jj] : 0ull;
    }
    unsigned long long prefix, mask;
    radix_select<KPT>(key, K, rs, prefix, mask);
    if (threadIdx.x < kSampleMaxK) cand[threadIdx.x] = 0ull;
    __syncthreads();
    radix_compact<KPT>(key, K, prefix, mask, rs, cand);
    __syncthreads();
    if (threadIdx.x >= 64) return;
    // sort the (at most 64) winners descending: register bitonic sort in one wavefront
    {
        const int lane = threadIdx.x;
        unsigned long long v = cand[lane];
#pragma unroll
        for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                const unsigned long long o = shfl_xor_u64(v, stride);
                const bool lower = (lane & stride) == 0, desc = (lane & size) == 0;
                const unsigned long long hi = v > o ? v : o, lo = v > o ? o : v;
                v = (lower == desc) ? hi : lo;
            }
        }
        cand[lane] = v;
    }
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
        if (nslices * kSampleMaxK > kSampleSelectKeys) return hipErrorInvalidValue;
        hipLaunchKernelGGL(sample_partial_kernel, dim3(nslices), dim3(kBlock), 0, s, a);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(sample_select_kernel, dim3(1), dim3(1024), 0, s, a, nslices);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(sample_full_kernel, dim3(1), dim3(1024), 0, s, a);
    return hipGetLastError();
}

}  // namespace tmg
