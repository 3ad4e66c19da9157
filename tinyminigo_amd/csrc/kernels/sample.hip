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
// Whole-vocabulary path (no top-k, or top_k > kSampleMaxK): each of the
// reference's sorts becomes a threshold search over the whole vocabulary,
// run as wide histogram launches (search_hist_kernel and the others below).
//
// Keys order by value descending, then id ascending, which is the reference
// argmax tie rule; the reference's sort_unstable_by leaves equal-value order
// unspecified, so any order among exact ties is as faithful as another.
// Keys are unique (they contain the id), so the top k set is exact.
#include "common.cuh"
#include "kernels.hpp"

namespace tmg {
namespace {

// The uniform draw of the running step (the reference's StdRng stream,
// computed on the host).
__device__ __forceinline__ float step_draw(const SampleArgs &a, int step) {
    return step >= 0 && step < a.n_draws ? a.draws[step] : 0.0f;
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
    const float r = step_draw(a, st.step);
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

// ---------------------------------------------------------------------------
// Whole-vocabulary path: no top-k (with or without a nucleus cut), or top_k
// above kSampleMaxK.  Every pass is a launch over many workgroups; only the
// bin and chunk selections run in one workgroup.
//
// The orders the reference gets by sorting are found by threshold searches:
// among the selected ids, in (key descending, id ascending) order, the first
// at which a running total of weights exceeds a target.
//   SK_COUNT   key = scaled logit, weight 1, target k - 1: the k-th best
//              logit (the reference's top-k sort);
//   SK_NUCLEUS key = probability, weight = probability, target top_p: the
//              nucleus cut (the reference sorts by probability, ties
//              unspecified); the kept mass is the running total at the cut;
//   SK_WALK    key = scaled logit, weight = probability, target = the draw:
//              the inverse-CDF walk over the sorted top-k candidates.
// A search is a radix search over the 32-bit key (12, 12, then 8 bits): per
// level a histogram launch (LDS bins, then global bins) and a pick launch
// (the bin where the running total crosses what is left of the target);
// ties at the final key go in id order (chunk masses, then one chunk
// scanned).  Without top-k the draw walks the ids in order (chunk masses,
// then one chunk).  Probability masses are summed in 2^-40 fixed point, so
// every sum is exact and independent of order.
// ---------------------------------------------------------------------------

constexpr int kGenWide = 2048;  // ids per workgroup of the elementwise passes
constexpr int kGenParts = kSampleMaxVocab / kGenWide;
constexpr int kHistIds = 4096;  // ids per workgroup of a histogram pass
constexpr int kGenBins = 4096;
constexpr int kPickThreads = 1024;
constexpr double kFx = 1099511627776.0;  // 2^40
static_assert(kGenParts == 128 && kGenParts <= kBlock, "scratch layout: 128 partials of each kind");
static_assert(kGenBins == 4 * kPickThreads, "the pick takes four bins per thread");

enum SearchKind { SK_COUNT = 0, SK_NUCLEUS = 1, SK_WALK = 2 };
constexpr int kSearchRunning = -2;  // SearchState::id while levels remain

struct SearchState {
    unsigned long long rest;     // target left after the heavier keys
    unsigned long long through;  // running total through the found id
    uint32_t pfx;                // key bits decided (the whole key after the last level)
    int id;                      // the found id; -1: the total does not exceed the target
    int pad[2];
};

// a.scratch: sc [V] | pr [V] | max partials [128] | sum partials [128] |
// u64 mass partials [128] | u64 histogram [4096] | SearchState [3]
struct GenBufs {
    float *sc, *pr, *pmax, *psum;
    unsigned long long *pmass, *hist;
    SearchState *ss;
};

__device__ __forceinline__ GenBufs gen_bufs(const SampleArgs &a) {
    GenBufs b;
    b.sc = a.scratch;
    b.pr = a.scratch + a.V;
    b.pmax = a.scratch + 2 * (size_t)a.V;
    b.psum = b.pmax + kGenParts;
    b.pmass = reinterpret_cast<unsigned long long *>(b.psum + kGenParts);
    b.hist = b.pmass + kGenParts;
    b.ss = reinterpret_cast<SearchState *>(b.hist + kGenBins);
    return b;
}

// floor(p * 2^40) for 0 <= p < 2 (exact: p's 24-bit significand shifted by
// its exponent); 0 for subnormals, negatives, NaN and p >= 2.
__device__ __forceinline__ unsigned long long fx(float p) {
    const uint32_t u = __float_as_uint(p);
    const int e = (int)(u >> 23);  // with the sign bit set e > 255
    if (e == 0 || e > 127) return 0ull;
    const unsigned long long m = (u & 0x7fffffu) | 0x800000u;
    const int sh = e - 110;  // value = m * 2^(e - 150), times 2^40
    return sh >= 0 ? m << sh : (sh > -24 ? m >> -sh : 0ull);
}

__device__ __forceinline__ unsigned long long wave_sum_u64(unsigned long long v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += shfl_xor_u64(v, off);
    return v;
}

__device__ __forceinline__ unsigned long long wave_incl_u64(unsigned long long v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t lo = __shfl_up((uint32_t)v, off, 64), hi = __shfl_up((uint32_t)(v >> 32), off, 64);
        if (lane >= off) v += ((unsigned long long)hi << 32) | lo;
    }
    return v;
}

// Exclusive prefix over the workgroup's threads in thread order (NW
// wavefronts); *total gets the sum.  wt holds NW values of LDS.
template <int NW>
__device__ unsigned long long block_excl_u64(unsigned long long v, unsigned long long *wt, unsigned long long *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const unsigned long long incl = wave_incl_u64(v);
    __syncthreads();
    if (lane == 63) wt[w] = incl;
    __syncthreads();
    unsigned long long before = 0, all = 0;
#pragma unroll
    for (int i = 0; i < NW; i++) {
        if (i < w) before += wt[i];
        all += wt[i];
    }
    *total = all;
    return before + incl - v;
}

__device__ __forceinline__ float wg_reduce(float v, bool is_max, float *red4) {
    v = is_max ? wave_max(v) : wave_sum(v);
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = v;
    __syncthreads();
    return is_max ? fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3])) : (red4[0] + red4[1]) + (red4[2] + red4[3]);
}

__device__ __forceinline__ bool use_topk(const DevState &st, int V) { return st.top_k > 0 && st.top_k < V; }

// Key and weight of id i for a search; false when the weight is 0 (such an
// id can never be where the running total crosses the target).
__device__ __forceinline__ bool kind_kw(int kind, float s, float p, uint32_t &k, unsigned long long &w) {
    if (kind == SK_COUNT) {
        k = f32_order(s);
        w = 1;
    } else if (kind == SK_NUCLEUS) {
        k = f32_order(p);
        w = fx(p);
    } else {
        k = f32_order(s);
        w = fx(p);
    }
    return w != 0;
}

__device__ __forceinline__ unsigned long long kind_target(int kind, const SampleArgs &a, const DevState &st) {
    return kind == SK_COUNT ? (unsigned long long)(st.top_k - 1)
                            : kind == SK_NUCLEUS ? fx(st.top_p) : fx(step_draw(a, st.step));
}

// pass 1: scaled logits (penalty, temperature; src/tensor.rs:1142-1154,
// :1168) and the workgroup maximum
__global__ __launch_bounds__(kBlock) void sample_scale_kernel(const SampleArgs a) {
    __shared__ float red4[4];
    const DevState st = *a.st;
    const GenBufs b = gen_bufs(a);
    const int base = blockIdx.x * kGenWide + threadIdx.x;
    float lv[kGenWide / kBlock];
#pragma unroll
    for (int j = 0; j < kGenWide / kBlock; j++) {
        const int i = base + j * kBlock;
        lv[j] = i < a.V ? a.logits[i] : 0.0f;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kGenWide / kBlock; j++) {
        const int i = base + j * kBlock;
        if (i < a.V) {
            float v = lv[j];
            if (st.penalty != 1.0f && a.seen && ((a.seen[i >> 5] >> (i & 31)) & 1u))
                v = v > 0.0f ? __fdiv_rn(v, st.penalty) : __fmul_rn(v, st.penalty);
            v = __fdiv_rn(v, st.temperature);
            b.sc[i] = v;
            mx = fmaxf(mx, v);
        }
    }
    const float m = wg_reduce(mx, true, red4);
    if (threadIdx.x == 0) b.pmax[blockIdx.x] = m;
}

// pass 2: softmax numerators over the candidates (src/tensor.rs:1177-1179):
// pr = exp(s - M) for candidates (all ids, or the top-k found by SK_COUNT),
// 0 for the others; M the overall maximum (always a candidate); workgroup sum
__global__ __launch_bounds__(kBlock) void sample_exp_kernel(const SampleArgs a) {
    __shared__ float red4[4];
    const DevState st = *a.st;
    const GenBufs b = gen_bufs(a);
    const int nparts = (a.V + kGenWide - 1) / kGenWide;
    float m = -INFINITY;
    for (int i = threadIdx.x; i < nparts; i += kBlock) m = fmaxf(m, b.pmax[i]);
    const float M = wg_reduce(m, true, red4);
    __syncthreads();
    const bool k_on = use_topk(st, a.V);
    uint32_t kk = 0;
    int kid = a.V;
    if (k_on) {
        kk = b.ss[SK_COUNT].pfx;
        kid = b.ss[SK_COUNT].id;
    }
    const int base = blockIdx.x * kGenWide + threadIdx.x;
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < kGenWide / kBlock; j++) {
        const int i = base + j * kBlock;
        if (i < a.V) {
            const float s = b.sc[i];
            const uint32_t k = f32_order(s);
            const float e = (!k_on || k > kk || (k == kk && i <= kid)) ? expf(s - M) : 0.0f;
            b.pr[i] = e;
            sum += e;
        }
    }
    const float S = wg_reduce(sum, false, red4);
    if (threadIdx.x == 0) b.psum[blockIdx.x] = S;
}

// pass 3: pr = pr / S, S the partial sums added in order
__global__ __launch_bounds__(kBlock) void sample_norm_kernel(const SampleArgs a) {
    __shared__ float Ssh;
    const GenBufs b = gen_bufs(a);
    const int nparts = (a.V + kGenWide - 1) / kGenWide;
    if (threadIdx.x == 0) {
        float S = 0.0f;
        for (int i = 0; i < nparts; i++) S += b.psum[i];
        Ssh = S;
    }
    __syncthreads();
    const float S = Ssh;
    const int base = blockIdx.x * kGenWide + threadIdx.x;
#pragma unroll
    for (int j = 0; j < kGenWide / kBlock; j++) {
        const int i = base + j * kBlock;
        if (i < a.V) b.pr[i] = b.pr[i] / S;
    }
}

// A search level's histogram: key digit `level` of the selected ids whose
// higher digits equal the prefix picked so far, weights into LDS bins, then
// the non-zero bins into the global histogram.
__global__ __launch_bounds__(kBlock) void search_hist_kernel(const SampleArgs a, int kind, int level) {
    __shared__ unsigned long long h[kGenBins];
    const GenBufs b = gen_bufs(a);
    const SearchState s = b.ss[kind];
    if (level > 0 && s.id != kSearchRunning) return;
    const int shift = level == 0 ? 20 : level == 1 ? 8 : 0;
    const uint32_t nb = level == 2 ? 256u : 4096u;
    const int above = level == 1 ? 20 : 8;  // levels 1, 2: the prefix is key >> above
    for (int i = threadIdx.x; i < (int)nb; i += kBlock) h[i] = 0;
    __syncthreads();
    constexpr int PER = kHistIds / kBlock;
    const int base = blockIdx.x * kHistIds + threadIdx.x;
    float sv[PER], pv[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = base + j * kBlock;
        sv[j] = (kind != SK_NUCLEUS && i < a.V) ? b.sc[i] : 0.0f;
        pv[j] = (kind != SK_COUNT && i < a.V) ? b.pr[i] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int i = base + j * kBlock;
        uint32_t k;
        unsigned long long w;
        if (i >= a.V || !kind_kw(kind, sv[j], pv[j], k, w)) continue;
        if (level > 0 && (k >> above) != s.pfx) continue;
        atomicAdd(&h[(k >> shift) & (nb - 1)], w);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < (int)nb; i += kBlock)
        if (h[i]) __hip_atomic_fetch_add(&b.hist[i], h[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A search level's pick: the bin (from the top) where the running total
// first exceeds what is left of the target; clears the global histogram for
// the next level.  At level 0 a total that does not exceed the target ends
// the search (id -1).
__global__ __launch_bounds__(kPickThreads) void search_pick_kernel(const SampleArgs a, int kind, int level) {
    __shared__ unsigned long long wt[kPickThreads / 64];
    __shared__ unsigned long long pk;
    const DevState st = *a.st;
    const GenBufs b = gen_bufs(a);
    const SearchState s = b.ss[kind];
    if (level > 0 && s.id != kSearchRunning) return;
    const int t = threadIdx.x;
    const unsigned long long rest = level == 0 ? kind_target(kind, a, st) : s.rest;
    const int nb = level == 2 ? 256 : 4096;
    unsigned long long c[4], mine = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int bin = nb - 1 - 4 * t - j;
        c[j] = bin >= 0 ? b.hist[bin] : 0ull;
        mine += c[j];
    }
    if (t == 0) pk = ~0ull;
    unsigned long long total;
    unsigned long long cum = block_excl_u64<kPickThreads / 64>(mine, wt, &total);
    if (cum <= rest && cum + mine > rest) {
        for (int j = 0; j < 4; j++) {
            if (cum + c[j] > rest) {
                // the bin (12 bits) and the weight before it (< 2^52)
                pk = ((unsigned long long)(nb - 1 - 4 * t - j) << 52) | cum;
                break;
            }
            cum += c[j];
        }
    }
    __syncthreads();
    const unsigned long long hit = pk;
    // every thread has read its bins: clear them for the next level
#pragma unroll
    for (int j = 0; j < 4; j++) b.hist[4 * t + j] = 0ull;
    if (t == 0) {
        SearchState n = s;
        if (total <= rest || hit == ~0ull) {
            n.id = -1;
        } else {
            n.pfx = ((level == 0 ? 0u : s.pfx) << (level == 2 ? 8 : 12)) | (uint32_t)(hit >> 52);
            n.rest = rest - (hit & ((1ull << 52) - 1));
            n.id = kSearchRunning;
        }
        b.ss[kind] = n;
    }
}

// Ties at the final key, in id order: pass 1, the mass of the tied ids per
// 2048-id chunk.
__global__ __launch_bounds__(kBlock) void search_tie_sums_kernel(const SampleArgs a, int kind) {
    __shared__ unsigned long long red4[4];
    const GenBufs b = gen_bufs(a);
    const SearchState s = b.ss[kind];
    if (s.id != kSearchRunning) return;
    const int i0 = blockIdx.x * kGenWide + 8 * threadIdx.x;
    unsigned long long m = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int i = i0 + j;
        if (i >= a.V) break;
        uint32_t k;
        unsigned long long w;
        if (kind_kw(kind, b.sc[i], b.pr[i], k, w) && k == s.pfx) m += w;
    }
    m = wave_sum_u64(m);
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) b.pmass[blockIdx.x] = (red4[0] + red4[1]) + (red4[2] + red4[3]);
}

// The first id, in id order, where the running mass of wv(i) (any i < V)
// exceeds `rest`, given each 2048-id chunk's mass in pmass: the chunk by a
// prefix over the chunk masses, then the id within it (thread t holds ids
// 8t .. 8t+7 of the chunk, so thread order is id order).  Returns -1 when
// the total does not exceed `rest`; *through gets the running mass through
// the id.  One workgroup of kBlock threads.
template <class Wv>
__device__ int chunk_threshold(const SampleArgs &a, const unsigned long long *pmass, Wv wv, unsigned long long rest,
                               unsigned long long *through) {
    __shared__ unsigned long long wt[4];
    __shared__ unsigned long long pk, pth;
    const int t = threadIdx.x;
    const int nparts = (a.V + kGenWide - 1) / kGenWide;  // <= kGenParts <= kBlock
    if (t == 0) pk = ~0ull;
    const unsigned long long c = t < nparts ? pmass[t] : 0ull;
    unsigned long long tot;
    const unsigned long long cum = block_excl_u64<4>(c, wt, &tot);
    if (t < nparts && cum <= rest && cum + c > rest) pk = ((unsigned long long)t << 48) | cum;
    __syncthreads();
    const unsigned long long hit = pk;
    __syncthreads();
    if (hit == ~0ull) return -1;
    const int g = (int)(hit >> 48);
    const unsigned long long before = hit & ((1ull << 48) - 1), left = rest - before;
    const int i0 = g * kGenWide + 8 * t;
    unsigned long long q[8], m = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        q[k] = i0 + k < a.V ? wv(i0 + k) : 0ull;
        m += q[k];
    }
    if (t == 0) pk = ~0ull;
    unsigned long long t2;
    unsigned long long cu = block_excl_u64<4>(m, wt, &t2);
    if (cu <= left && cu + m > left) {
        for (int k = 0; k < 8; k++) {
            cu += q[k];
            if (cu > left) {
                pk = (unsigned long long)(i0 + k);
                pth = before + cu;
                break;
            }
        }
    }
    __syncthreads();
    const unsigned long long r = pk;
    if (through) *through = pth;
    __syncthreads();
    return r == ~0ull ? -1 : (int)r;
}

// Ties, pass 2: the id; SK_WALK then emits the token (with the reference's
// fallback when the draw lies past the last cumulative sum: the first
// candidate with p > 0 in walk order, i.e. the best key).
__global__ __launch_bounds__(kBlock) void search_tie_pick_kernel(const SampleArgs a, int kind) {
    __shared__ unsigned long long best_sh;
    const DevState st = *a.st;
    const GenBufs b = gen_bufs(a);
    const SearchState s = b.ss[kind];
    const int t = threadIdx.x;
    int id = -1;
    unsigned long long through = 0;
    if (s.id == kSearchRunning) {
        id = chunk_threshold(
            a, b.pmass,
            [&](int i) -> unsigned long long {
                uint32_t k;
                unsigned long long w;
                return kind_kw(kind, b.sc[i], b.pr[i], k, w) && k == s.pfx ? w : 0ull;
            },
            s.rest, &through);
        // the running total from the search's start: the heavier keys'
        // target - rest, then the ties'
        through += kind_target(kind, a, st) - s.rest;
    }
    if (kind != SK_WALK) {
        if (t == 0) {
            SearchState n = s;
            n.id = s.id == kSearchRunning ? id : -1;
            n.through = through;
            b.ss[kind] = n;
        }
        return;
    }
    if (id < 0) {
        unsigned long long best = ~0ull;
        for (int i = t; i < a.V; i += kBlock) {
            const float p = b.pr[i];
            if (!(p > 0.0f)) continue;
            const unsigned long long k = ((unsigned long long)~f32_order(b.sc[i]) << 32) | (uint32_t)i;
            best = k < best ? k : best;
        }
        if (t == 0) best_sh = ~0ull;
        __syncthreads();
        atomicMin(&best_sh, best);
        __syncthreads();
        id = best_sh == ~0ull ? 0 : (int)(uint32_t)best_sh;
    }
    if (t == 0) emit_token(a, id);
}

// The nucleus cut (src/tensor.rs:1182-1201): ids after the cut in
// probability order get 0, the kept ones p / (kept mass).
__global__ __launch_bounds__(kBlock) void sample_renorm_kernel(const SampleArgs a) {
    const GenBufs b = gen_bufs(a);
    const SearchState s = b.ss[SK_NUCLEUS];
    if (s.id < 0) return;
    const float sumk = (float)((double)s.through / kFx);
    const int base = blockIdx.x * kGenWide + threadIdx.x;
#pragma unroll
    for (int j = 0; j < kGenWide / kBlock; j++) {
        const int i = base + j * kBlock;
        if (i < a.V) {
            const float p = b.pr[i];
            const uint32_t k = f32_order(p);
            b.pr[i] = (k > s.pfx || (k == s.pfx && i <= s.id)) ? p / sumk : 0.0f;
        }
    }
}

// Without top-k: the inverse-CDF walk in id order (src/tensor.rs:1203-1212),
// pass 1: each 2048-id chunk's probability mass.
__global__ __launch_bounds__(kBlock) void sample_walk_sums_kernel(const SampleArgs a) {
    __shared__ unsigned long long red4[4];
    const GenBufs b = gen_bufs(a);
    const int base = blockIdx.x * kGenWide + threadIdx.x;
    unsigned long long m = 0;
#pragma unroll
    for (int j = 0; j < kGenWide / kBlock; j++) {
        const int i = base + j * kBlock;
        if (i < a.V) m += fx(b.pr[i]);
    }
    m = wave_sum_u64(m);
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) b.pmass[blockIdx.x] = (red4[0] + red4[1]) + (red4[2] + red4[3]);
}

// pass 2: the id where the running mass first exceeds the draw, emitted
// (past the last cumulative sum: the lowest id with p > 0).
__global__ __launch_bounds__(kBlock) void sample_walk_kernel(const SampleArgs a) {
    __shared__ unsigned long long best_sh;
    const DevState st = *a.st;
    const GenBufs b = gen_bufs(a);
    const int t = threadIdx.x;
    int pick = chunk_threshold(
        a, b.pmass, [&](int i) { return fx(b.pr[i]); }, fx(step_draw(a, st.step)), nullptr);
    if (pick < 0) {
        unsigned long long best = ~0ull;
        for (int i = t; i < a.V; i += kBlock)
            if (b.pr[i] > 0.0f) {
                best = (unsigned long long)i;
                break;
            }
        if (t == 0) best_sh = ~0ull;
        __syncthreads();
        atomicMin(&best_sh, best);
        __syncthreads();
        pick = best_sh == ~0ull ? 0 : (int)best_sh;
    }
    if (t == 0) emit_token(a, pick);
}

}  // namespace

hipError_t launch_sample(const SampleArgs &a, hipStream_t s) {
    if (a.V <= 0 || a.V > kSampleMaxVocab) return hipErrorInvalidValue;
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
    if (!a.scratch) return hipErrorInvalidValue;
    const dim3 wide((a.V + kGenWide - 1) / kGenWide), hist((a.V + kHistIds - 1) / kHistIds);
    auto search = [&](int kind) {
        for (int level = 0; level < 3; level++) {
            hipLaunchKernelGGL(search_hist_kernel, hist, dim3(kBlock), 0, s, a, kind, level);
            hipLaunchKernelGGL(search_pick_kernel, dim3(1), dim3(kPickThreads), 0, s, a, kind, level);
        }
        hipLaunchKernelGGL(search_tie_sums_kernel, wide, dim3(kBlock), 0, s, a, kind);
        hipLaunchKernelGGL(search_tie_pick_kernel, dim3(1), dim3(kBlock), 0, s, a, kind);
    };
    hipLaunchKernelGGL(sample_scale_kernel, wide, dim3(kBlock), 0, s, a);
    if (a.use_k) search(SK_COUNT);
    hipLaunchKernelGGL(sample_exp_kernel, wide, dim3(kBlock), 0, s, a);
    hipLaunchKernelGGL(sample_norm_kernel, wide, dim3(kBlock), 0, s, a);
    if (a.use_p) {
        search(SK_NUCLEUS);
        hipLaunchKernelGGL(sample_renorm_kernel, wide, dim3(kBlock), 0, s, a);
    }
    if (a.use_k) {
        search(SK_WALK);
    } else {
        hipLaunchKernelGGL(sample_walk_sums_kernel, wide, dim3(kBlock), 0, s, a);
        hipLaunchKernelGGL(sample_walk_kernel, dim3(1), dim3(kBlock), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace tmg
