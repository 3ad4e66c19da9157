// On-device token selection for gfx950 (reference generate,
// src/model.rs:631-646; apply_repetition_penalty, src/tensor.rs:1142-1154;
// sample, src/tensor.rs:1157-1213).
//
// Top-k path (0 < k <= kSampleMaxK, or greedy with a repetition penalty):
//   pass 1, one workgroup per 2048-id slice: penalty and temperature, then a
//   radix select over the packed (value, id) keys held in registers (8-bit
//   digits from the top, LDS histograms; block_top_k) finds the slice's k-th
//   largest key; the slice's best k keys are written out unordered.
//   pass 2, one workgroup: the same selection over all slice winners, the
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
    unsigned long long kmin;
    unsigned hist[256];
    int digit, above, count, n;
};

// Finds the k-th largest of the valid keys among the KPT each thread holds
// (1 <= k <= number of valid keys): on return every thread has
// (prefix, mask) such that the selected valid keys are exactly those with
// (key & mask) >= prefix, where mask covers the top bits decided.  8-bit
// digits from the most significant; stops as soon as the whole bin holding
// the k-th key is selected.
template <int KPT>
__device__ void radix_select(const unsigned long long (&key)[KPT], const bool (&valid)[KPT], int k, RadixSel &rs,
                             unsigned long long &prefix, unsigned long long &mask) {
    const int t = threadIdx.x, nt = blockDim.x;
    prefix = 0;
    mask = 0;
    int remaining = k;
    for (int shift = 56; shift >= 0; shift -= 8) {
        for (int i = t; i < 256; i += nt) rs.hist[i] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < KPT; j++)
            if (valid[j] && (key[j] & mask) == prefix) atomicAdd(&rs.hist[(key[j] >> shift) & 255], 1u);
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

// Selects the k largest valid keys of the block (all of them when there are
// at most k) and writes them, unordered, to out[0 .. k); missing ones are
// written as 0.  With PREFILTER, a first selection over the per-thread maxima
// gives a lower bound T0 for the k-th largest key (the k largest maxima are k
// distinct keys), and only keys >= T0 enter the exact selection: worth it
// where most threads hold few real keys (the second pass), not where every
// thread holds eight (the slices).
template <int KPT, bool PREFILTER>
__device__ void block_top_k(const unsigned long long (&key)[KPT], const bool (&valid)[KPT], int nvalid, int k,
                            RadixSel &rs, unsigned long long *out) {
    const int t = threadIdx.x;
    for (int i = t; i < k; i += blockDim.x) out[i] = 0ull;
    bool cv[KPT];
#pragma unroll
    for (int j = 0; j < KPT; j++) cv[j] = valid[j];
    int ncand = nvalid;
    if (PREFILTER && nvalid > k) {
        unsigned long long tmax = 0;
        bool any = false;
#pragma unroll
        for (int j = 0; j < KPT; j++)
            if (valid[j]) {
                tmax = key[j] > tmax ? key[j] : tmax;
                any = true;
            }
        if (t == 0) rs.n = 0;
        __syncthreads();
        if (any) atomicAdd(&rs.n, 1);
        __syncthreads();
        const int nany = rs.n;
        __syncthreads();
        if (nany >= k) {
            const unsigned long long km[1] = {tmax};
            const bool kv[1] = {any};
            unsigned long long p0, m0;
            radix_select<1>(km, kv, k, rs, p0, m0);
            // the k-th largest maximum: the smallest maximum inside the selection
            if (t == 0) rs.kmin = ~0ull;
            __syncthreads();
            if (any && (tmax & m0) >= p0) atomicMin(&rs.kmin, tmax);
            __syncthreads();
            const unsigned long long t0 = rs.kmin;
            int mine = 0;
#pragma unroll
            for (int j = 0; j < KPT; j++) {
                cv[j] = valid[j] && key[j] >= t0;
                mine += cv[j];
            }
            if (t == 0) rs.n = 0;
            __syncthreads();
            if (mine) atomicAdd(&rs.n, mine);
            __syncthreads();
            ncand = rs.n;
            __syncthreads();
        }
    }
    unsigned long long prefix = 0, mask = 0;  // (key & 0) >= 0: every candidate
    if (ncand > k) radix_select<KPT>(key, cv, k, rs, prefix, mask);
    if (t == 0) rs.n = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < KPT; j++) {
        if (cv[j] && (key[j] & mask) >= prefix) {
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
    bool valid[KPT];
#pragma unroll
    for (int j = 0; j < KPT; j++) {
        const int i = base + j * kBlock + threadIdx.x;
        key[j] = 0ull;
        valid[j] = i < a.V;
        if (valid[j]) {
            const float v = adjusted(a.logits, a.seen, st, i, greedy);
            if (v == v) key[j] = argmax_key(v, (uint32_t)i);
        }
    }
    block_top_k<KPT, false>(key, valid, min(kSampleSlice, a.V - base), K, rs,
                            a.cand + (size_t)blockIdx.x * kSampleMaxK);
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

// Lane l's float of wavefront-uniform lane i (a scalar read, no LDS).
__device__ __forceinline__ float lane_f(float v, int i) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}

constexpr int kSelectThreads = 512;

__global__ __launch_bounds__(kSelectThreads) void sample_select_kernel(const SampleArgs a, int nslices) {
    __shared__ RadixSel rs;
    __shared__ unsigned long long cand[kSampleMaxK];
    constexpr int KPT = kSampleSelectKeys / kSelectThreads;
    const DevState st = *a.st;
    const bool greedy = a.greedy != 0;
    const int K = greedy ? 1 : st.top_k;
    const int n = nslices * K;
    unsigned long long key[KPT];
    bool valid[KPT];
#pragma unroll
    for (int j = 0; j < KPT; j++) {
        const int i = j * kSelectThreads + threadIdx.x;
        const int sl = i / K, jj = i - sl * K;
        valid[j] = i < n;
        key[j] = valid[j] ? a.cand[(size_t)sl * kSampleMaxK + jj] : 0ull;
    }
    if (threadIdx.x < kSampleMaxK) cand[threadIdx.x] = 0ull;
    block_top_k<KPT, true>(key, valid, n, K, rs, cand);
    __syncthreads();
    if (threadIdx.x >= 64) return;
    // one wavefront from here: lane i holds candidate i.  Sort the (at most
    // 64) winners descending with a register bitonic sort.
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
    if (greedy) {
        // all -inf/NaN logits leave key 0 on top: the reference returns 0
        if (lane == 0) emit_token(a, v ? key_index(v) : 0);
        return;
    }
    // The reference's sequential tail, elementwise work across lanes and the
    // running sums in candidate order through lane reads, so every float
    // operation is the reference's, in its order.
    // softmax over the k candidates (src/tensor.rs:1177-1179)
    const float val = key_value(v);
    const float mx = lane_f(val, 0);
    float p = lane < K ? expf(val - mx) : 0.0f;
    float sum = 0.0f;
    for (int i = 0; i < K; i++) sum += lane_f(p, i);
    p = p / sum;
    // nucleus (src/tensor.rs:1182-1201): candidates are already in descending
    // probability order
    if (st.top_p < 1.0f) {
        float cum = 0.0f;
        int cutoff = K;
        for (int r = 0; r < K; r++) {
            cum += lane_f(p, r);
            if (cum > st.top_p) {
                cutoff = r + 1;
                break;
            }
        }
        float s2 = 0.0f;
        for (int r = 0; r < cutoff; r++) s2 += lane_f(p, r);
        p = lane < cutoff ? p / s2 : 0.0f;
    }
    // inverse-CDF walk in candidate order (src/tensor.rs:1203-1212)
    const float r = uniform_f32(st.seed, (unsigned long long)st.step);
    float cum = 0.0f;
    int pick = -1;
    for (int i = 0; i < K; i++) {
        cum += lane_f(p, i);
        if (r < cum) {
            pick = i;
            break;
        }
    }
    if (pick < 0) {
        const unsigned long long pos = __ballot(lane < K && p > 0.0f);
        pick = pos ? __builtin_ctzll(pos) : 0;
    }
    const uint32_t klo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, pick);
    const uint32_t khi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), pick);
    if (lane == 0) emit_token(a, key_index(((unsigned long long)khi << 32) | klo));
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
        hipLaunchKernelGGL(sample_select_kernel, dim3(1), dim3(kSelectThreads), 0, s, a, nslices);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(sample_full_kernel, dim3(1), dim3(1024), 0, s, a);
    return hipGetLastError();
}

}  // namespace tmg
