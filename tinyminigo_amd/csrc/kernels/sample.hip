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
// Whole-vocabulary path (no top-k, or top_k > kSampleMaxK): the same steps
// over up to the whole vocabulary, with a device sort for the orders and
// each running sum computed exactly in one workgroup (chain_kernel below).
//
// Keys order by value descending, then id ascending, which is the reference
// argmax tie rule; the reference's sort_unstable_by leaves equal-value order
// unspecified, so any order among exact ties is as faithful as another.
// Keys are unique (they contain the id), so the top k set is exact.
#include "common.cuh"
#include "kernels.hpp"
#include "ref_expf.h"

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
    float p = lane < K ? ref_expf(val - mx) : 0.0f;
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
// above kSampleMaxK.  The reference's steps, in its orders, with its float
// operations (src/tensor.rs:1157-1213):
//   candidate order  ids in id order without top-k; with top-k the k best
//                    scaled logits in descending order (the reference sorts;
//                    ties are unspecified there, id order here);
//   softmax          M = max, e = expf(s - M) (glibc's expf, ref_expf.h),
//                    Z = the f32 running sum of e in candidate order, p = e/Z;
//   nucleus          the f32 running sum of p in descending order until it
//                    exceeds top_p, the f32 running sum of the kept p, then
//                    p / kept sum;
//   walk             the f32 running sum of p in candidate order until it
//                    exceeds the draw; past the end, the first candidate
//                    with p > 0.
// Orders come from one bitonic sort of (scaled logit, id) keys.  Each running
// sum is one workgroup's `chain` (below), which gives the f32 sequential
// sum's every partial result exactly without a sequential loop over the
// terms.
// ---------------------------------------------------------------------------

constexpr int kGenWide = 2048;  // ids per workgroup of the elementwise passes
constexpr int kGenParts = kSampleMaxVocab / kGenWide;
static_assert(kGenParts == 128 && kGenParts <= kBlock, "scratch layout: 128 partial maxima");

// The running sums of the whole-vocabulary path.
enum ChainKind { CH_Z = 0, CH_N = 1, CH_K = 2, CH_W = 3 };

struct ChainOut {
    float total;  // the sum over all n terms (when no partial sum exceeds the threshold)
    int found;    // first index whose partial sum exceeds the threshold, or -1
    float at;     // that partial sum
    int n;        // terms summed
};

// a.scratch: sc [V] | pr [V] | max partials [128] | ChainOut [4] | sort
// keys [V] | keys2 [V] (8-byte aligned: V * 8 + 512 + 64 bytes before them) |
// radix counts [kSampleRadixCounts] | running-sum chunk metadata |
// running-sum group metadata
struct ChainChunkMeta;
struct ChainGroupMeta;

struct GenBufs {
    float *sc, *pr, *pmax;
    ChainOut *cs;
    unsigned long long *keys, *keys2;  // sort keys [V], and the radix passes' other buffer [V]
    uint32_t *radix;                    // radix digit counts / offsets [256][blocks]
    ChainChunkMeta *cmeta;  // [kChainMaxChunks]
    ChainGroupMeta *gmeta;  // [2][kChainMaxChunks * kChainPer]
};

__device__ __forceinline__ GenBufs gen_bufs(const SampleArgs &a) {
    GenBufs b;
    b.sc = a.scratch;
    b.pr = a.scratch + a.V;
    b.pmax = a.scratch + 2 * (size_t)a.V;
    b.cs = reinterpret_cast<ChainOut *>(b.pmax + kGenParts);
    b.keys = reinterpret_cast<unsigned long long *>(b.cs + 4);
    b.keys2 = b.keys + a.V;
    b.radix = reinterpret_cast<uint32_t *>(b.keys2 + a.V);
    b.cmeta = reinterpret_cast<ChainChunkMeta *>(b.radix + kSampleRadixCounts);
    b.gmeta = reinterpret_cast<ChainGroupMeta *>(reinterpret_cast<char *>(b.cmeta) + kSampleChainChunkBytes);
    return b;
}

__device__ __forceinline__ float wg_reduce(float v, bool is_max, float *red4) {
    v = is_max ? wave_max(v) : wave_sum(v);
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = v;
    __syncthreads();
    return is_max ? fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3])) : (red4[0] + red4[1]) + (red4[2] + red4[3]);
}

// Inclusive prefix sum over the wavefront's 64 lanes: shifts within rows of
// 16 lanes, then each row's total broadcast to the rows above it.
__device__ __forceinline__ uint32_t wave_incl_u32(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, true);  // row_shr:1
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, true);  // row_shr:2
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, true);  // row_shr:4
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, true);  // row_shr:8
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
    return v;
}

__device__ __forceinline__ uint32_t lane_u32(uint32_t v, int i) { return (uint32_t)__builtin_amdgcn_readlane((int)v, i); }

// pass 1: scaled logits (penalty, temperature; src/tensor.rs:1142-1154,
// :1168), the workgroup maximum, and pr cleared
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
            b.pr[i] = 0.0f;
            mx = fmaxf(mx, v);
        }
    }
    const float m = wg_reduce(mx, true, red4);
    if (threadIdx.x == 0) b.pmax[blockIdx.x] = m;
}

// The maximum scaled logit (f32::max ignores NaN, as fmaxf does): every
// workgroup's partial maxima reduced again.
__device__ float scaled_max(const SampleArgs &a, const GenBufs &b, float *red4) {
    const int nparts = (a.V + kGenWide - 1) / kGenWide;
    float m = -INFINITY;
    for (int i = threadIdx.x; i < nparts; i += kBlock) m = fmaxf(m, b.pmax[i]);
    return wg_reduce(m, true, red4);
}

// ---- the sort: keys (scaled logit order, then ~id) descending --------------
//
// A stable LSD radix sort of the V keys on their upper 32 bits (the scaled
// logit's order), descending, in four passes of 8-bit digits; equal values
// keep id order.  Per pass: per-block digit counts (kRadixBlock keys per
// block), one exclusive scan over them in (digit, block) order, and a stable
// scatter.  Passes alternate between keys and keys2 and end in keys.

// keys[i] = argmax_key(scaled, i) for ids with a non-NaN scaled logit, 0 for
// NaN ones (they sort last)
__global__ __launch_bounds__(kBlock) void sort_keys_kernel(const SampleArgs a) {
    const GenBufs b = gen_bufs(a);
    for (int i = blockIdx.x * kBlock + threadIdx.x; i < a.V; i += gridDim.x * kBlock) {
        const float v = b.sc[i];
        b.keys[i] = v == v ? argmax_key(v, (uint32_t)i) : 0ull;
    }
}

__device__ __forceinline__ uint32_t radix_digit(unsigned long long k, int pass) {
    return (~(uint32_t)(k >> 32) >> (8 * pass)) & 255u;  // ascending digits = descending keys
}

__device__ __forceinline__ void radix_src_dst(const GenBufs &b, int pass, const unsigned long long **src,
                                              unsigned long long **dst) {
    *src = (pass & 1) ? b.keys2 : b.keys;
    *dst = (pass & 1) ? b.keys : b.keys2;
}

// digit counts of block blockIdx.x, into off[digit * nb + block]
__global__ __launch_bounds__(kBlock) void radix_hist_kernel(const SampleArgs a, int pass) {
    __shared__ uint32_t h[256];
    const GenBufs b = gen_bufs(a);
    const unsigned long long *src;
    unsigned long long *dst;
    radix_src_dst(b, pass, &src, &dst);
    const int nb = (a.V + kRadixBlock - 1) / kRadixBlock;
    h[threadIdx.x] = 0u;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kRadixBlock / kBlock; r++) {
        const int i = blockIdx.x * kRadixBlock + r * kBlock + threadIdx.x;
        if (i < a.V) atomicAdd(&h[radix_digit(src[i], pass)], 1u);
    }
    __syncthreads();
    b.radix[threadIdx.x * nb + blockIdx.x] = h[threadIdx.x];
}

// exclusive prefix over off[0 .. 256 nb), in place (one workgroup): tile r
// of kRadixScanThreads values is thread-indexed (coalesced); each wavefront
// scans its 64 values of every tile, one wavefront scans the (tile,
// wavefront) totals in order, and the tiles are read and scanned again to
// write the result
constexpr int kRadixTiles = (int)(kSampleRadixCounts / kRadixScanThreads);
__global__ __launch_bounds__(kRadixScanThreads) void radix_scan_kernel(const SampleArgs a) {
    constexpr int NW = kRadixScanThreads / 64;
    __shared__ uint32_t wt[kRadixTiles * NW];
    const GenBufs b = gen_bufs(a);
    const int nb = (a.V + kRadixBlock - 1) / kRadixBlock;
    const int total = 256 * nb, tiles = (total + kRadixScanThreads - 1) / kRadixScanThreads;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    for (int r0 = 0; r0 < tiles; r0 += 4) {  // four tiles' loads in flight at a time
        uint32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = (r0 + k) * kRadixScanThreads + t;
            v[k] = r0 + k < tiles && i < total ? b.radix[i] : 0u;
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t incl = wave_incl_u32(v[k]);
            if (lane == 63 && r0 + k < tiles) wt[(r0 + k) * NW + w] = incl;
        }
    }
    __syncthreads();
    if (w == 0) {
        // exclusive scan of tiles * NW totals, in (tile, wavefront) order
        constexpr int PER = kRadixTiles * NW / 64;
        uint32_t x[PER], sum = 0u;
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int i = lane * PER + k;
            x[k] = i < tiles * NW ? wt[i] : 0u;
            sum += x[k];
        }
        uint32_t run = wave_incl_u32(sum) - sum;
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int i = lane * PER + k;
            if (i < tiles * NW) wt[i] = run;
            run += x[k];
        }
    }
    __syncthreads();
    for (int r0 = 0; r0 < tiles; r0 += 4) {
        uint32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = (r0 + k) * kRadixScanThreads + t;
            v[k] = r0 + k < tiles && i < total ? b.radix[i] : 0u;
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = (r0 + k) * kRadixScanThreads + t;
            const uint32_t ex = wave_incl_u32(v[k]) - v[k];
            if (r0 + k < tiles && i < total) b.radix[i] = wt[(r0 + k) * NW + w] + ex;
        }
    }
}

// stable scatter of block blockIdx.x: rounds of kBlock keys in id order;
// within a round, a key's rank among equal digits is its wavefront's earlier
// lanes (ballot matching) plus the earlier wavefronts' counts
__global__ __launch_bounds__(kBlock) void radix_scatter_kernel(const SampleArgs a, int pass) {
    __shared__ uint32_t cnt[256];
    __shared__ uint32_t wc[kBlock / 64][256];
    const GenBufs b = gen_bufs(a);
    const unsigned long long *src;
    unsigned long long *dst;
    radix_src_dst(b, pass, &src, &dst);
    const int nb = (a.V + kRadixBlock - 1) / kRadixBlock;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const unsigned long long below = (1ull << lane) - 1ull;
    cnt[t] = b.radix[t * nb + blockIdx.x];
#pragma unroll
    for (int k = 0; k < kBlock / 64; k++) wc[k][t] = 0u;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kRadixBlock / kBlock; r++) {
        const int i = blockIdx.x * kRadixBlock + r * kBlock + t;
        const bool valid = i < a.V;
        const unsigned long long key = valid ? src[i] : 0ull;
        const uint32_t d = radix_digit(key, pass);
        unsigned long long peers = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; bit++) {
            const unsigned long long m = __ballot((d >> bit) & 1u);
            peers &= ((d >> bit) & 1u) ? m : ~m;
        }
        if (valid && !(peers & below)) wc[w][d] = (uint32_t)__builtin_popcountll(peers);
        __syncthreads();
        if (valid) {
            uint32_t pos = cnt[d] + (uint32_t)__builtin_popcountll(peers & below);
            for (int k = 0; k < w; k++) pos += wc[k][d];
            dst[pos] = key;
        }
        __syncthreads();
        uint32_t add = 0u;
#pragma unroll
        for (int k = 0; k < kBlock / 64; k++) {
            add += wc[k][t];
            wc[k][t] = 0u;
        }
        cnt[t] += add;
        __syncthreads();
    }
}

// id of the candidate at rank j (0 for a NaN key, which holds no id)
__device__ __forceinline__ int rank_id(const GenBufs &b, int j) {
    const unsigned long long k = b.keys[j];
    return k ? key_index(k) : 0;
}

__device__ __forceinline__ bool use_topk(const DevState &st, int V) { return st.top_k > 0 && st.top_k < V; }

// ---- the f32 running sum --------------------------------------------------
//
// s_0 = 0, s_j = fl(s_{j-1} + x_j) with x_j >= 0.  While the partial sums
// stay in one binade [2^e, 2^(e+1)) (ulp u), fl(s + x) = s + q u with q the
// integer nearest x / u; when x / u is exactly half-way (a tie), q is the
// choice that leaves s + q u even, i.e. floor(x / u) + 1 exactly when the
// running significand after floor(x / u) is odd.  Writing m for s / u (the
// significand, 2^23 <= m < 2^24, or below 2^23 for subnormal s, whose u is
// 2^-149 like the first normal binade's), s's bits are ((e_u - 1) << 23) + m
// for e_u = max(biased exponent, 1), and within a binade the partial sums are
// m plus integer prefix sums of the q: order-free, except for the parity at
// ties, which is settled tie by tie in order.  A real f32 add is needed only
// at a term of 2^24 u or more, where the sum leaves the binade, and after a
// non-finite value.

// q = x / u rounded to nearest for u = 2^(eu - 150), or its floor with `tie`
// set when x / u is half-way; `flag` when x is negative, -0 or not finite,
// or x >= 2^24 u
__device__ __forceinline__ uint32_t chain_q(float x, int eu, bool &tie, bool &flag) {
    const uint32_t ux = __float_as_uint(x);
    if (ux == 0u) return 0u;
    int ex = (int)(ux >> 23);
    if (ex >= 255) {  // sign bit set (negative or -0), or inf / NaN
        flag = true;
        return 0u;
    }
    uint32_t mx = ux & 0x7fffffu;
    if (ex) mx |= 0x800000u;
    else ex = 1;
    const int k = eu - ex;  // x / u = mx / 2^k
    if (k < 0) {
        flag = true;
        return 0u;
    }
    if (k == 0) return mx;
    if (k > 24) return 0u;  // x / u < 1/2
    uint32_t q = mx >> k;
    const uint32_t rem = mx & ((1u << k) - 1u), half = 1u << (k - 1);
    if (rem > half) q++;
    else if (rem == half) tie = true;
    return q;
}

constexpr int kChainThreads = 1024;
constexpr int kChainChunk = 1024;  // terms per chunk: 16 per lane of one wavefront
constexpr int kChainPer = kChainChunk / 64;  // groups of 64 terms per chunk
constexpr int kChainMaxChunks = kSampleMaxVocab / kChainChunk;
constexpr int kChainTies = 32;  // ties per chunk its one-step advance settles
constexpr int kGroupTies = 2;   // ties per group its one-step advance settles
constexpr uint32_t kChainSat = 1u << 25;  // integer sums saturate here (>= 2^24 leaves any binade)
static_assert(kChainMaxChunks == 256 && kChainPer == 16, "chain layout");

// Per chunk: the double sum, the guessed starting binade, and under it the
// integer sum of the q (floors at ties; saturated), the ties' inclusive
// integer prefixes from the chunk start in order, and whether any term is
// flagged or there are more than kChainTies ties.
struct ChainChunkMeta {
    double dsum;
    uint32_t q;
    int ntie, flag, eguess;
    uint32_t ties[kChainTies];
};
// Per group of 64 terms, under the group's own guessed starting binade
// (bin 0) and the next one (bin 1): the integer sum, tie count, the first
// kGroupTies ties' inclusive prefixes from the group start, and the flag.
struct ChainGroupMeta {
    uint32_t q;
    uint32_t tie[kGroupTies];
    int16_t ntie_flag;  // tie count, or -1 when a term is flagged
    int16_t eguess;     // the group's guessed starting binade (bin 0)
};

static_assert(sizeof(ChainChunkMeta) * kChainMaxChunks == kSampleChainChunkBytes, "scratch layout");
static_assert(sizeof(ChainGroupMeta) * 2 * kChainMaxChunks * kChainPer == kSampleChainGroupBytes, "scratch layout");

__device__ __forceinline__ ChainChunkMeta *chain_chunks(const GenBufs &b) { return b.cmeta; }
__device__ __forceinline__ ChainGroupMeta *chain_groups(const GenBufs &b) { return b.gmeta; }

// One wavefront adds terms j0 .. j0 + 63 (lane l holds x of j0 + l; terms at
// or past n are absent) to the running sum whose bits are *sb.  With a
// threshold, returns the first index whose partial sum exceeds T (its sum in
// *at), else -1.
__device__ int chain_group(float x, int j0, int n, bool has_t, float T, uint32_t *sb, float *at) {
    const int lane = threadIdx.x & 63;
    const bool in = j0 + lane < n;
    const unsigned long long upto = lane == 63 ? ~0ull : (2ull << lane) - 1ull;  // lanes 0 .. lane
    int start = 0;
    uint32_t s = *sb;
    while (start < 64) {
        const bool pend = in && lane >= start;
        const unsigned long long pm = __ballot(pend);
        if (!pm) break;
        const int es = (int)(s >> 23);
        const bool nonfinite = es >= 255;
        const int eu = es > 1 ? es : 1;
        const uint32_t m = es ? ((s & 0x7fffffu) | 0x800000u) : s;
        bool tie = false, flag = false;
        uint32_t q = 0u;
        if (pend) {
            if (nonfinite) flag = true;
            else q = chain_q(x, eu, tie, flag);
        }
        uint32_t incl = wave_incl_u32(q);
        // ties in order: round up where the running significand is odd
        unsigned long long tm = __ballot(pend && tie), ups = 0ull;
        uint32_t adj = 0u;
        while (tm) {
            const int tl = __builtin_ctzll(tm);
            tm &= tm - 1ull;
            if ((m + lane_u32(incl, tl) + adj) & 1u) {
                adj++;
                ups |= 1ull << tl;
            }
        }
        incl += (uint32_t)__builtin_popcountll(ups & upto);
        const bool special = pend && (flag || (!nonfinite && m + incl >= (1u << 24)));
        const unsigned long long sm = __ballot(special);
        const int f = sm ? __builtin_ctzll(sm) : 64;
        const uint32_t sl = ((uint32_t)(eu - 1) << 23) + m + incl;  // partial sum of committed lanes
        if (has_t) {
            const unsigned long long hm = __ballot(pend && lane < f && __uint_as_float(sl) > T);
            if (hm) {
                const int h = __builtin_ctzll(hm);
                *at = __uint_as_float(lane_u32(sl, h));
                *sb = lane_u32(sl, h);
                return j0 + h;
            }
        }
        if (f == 64) {
            s = lane_u32(sl, 63 - __builtin_clzll(pm));
            break;
        }
        const uint32_t before = f > start ? lane_u32(sl, f - 1) : s;
        const float xf = __uint_as_float(lane_u32(__float_as_uint(x), f));
        s = __float_as_uint(__uint_as_float(before) + xf);
        if (has_t && __uint_as_float(s) > T) {
            *at = __uint_as_float(s);
            *sb = s;
            return j0 + f;
        }
        start = f + 1;
    }
    *sb = s;
    return -1;
}

// The chain's terms: pr by id in id order, or by rank (sorted order).
__device__ __forceinline__ float chain_x(const GenBufs &b, bool by_rank, int j) {
    return by_rank ? b.pr[rank_id(b, j)] : b.pr[j];
}

// Lane l's kChainPer terms of chunk c: c * kChainChunk + 64 i + l (0 past n).
__device__ __forceinline__ void chain_load(const GenBufs &b, bool by_rank, int c, int n, int lane,
                                           float (&xs)[kChainPer]) {
#pragma unroll
    for (int i = 0; i < kChainPer; i++) {
        const int j = c * kChainChunk + i * 64 + lane;
        xs[i] = j < n ? chain_x(b, by_rank, j) : 0.0f;
    }
}

// A chain's terms (order, count) and threshold.
struct ChainSpec {
    bool by_rank, has_t;
    float T;
    int n;
};

__device__ ChainSpec chain_spec(const SampleArgs &a, const GenBufs &b, const DevState &st, int kind) {
    const bool k_on = use_topk(st, a.V);
    ChainSpec c{k_on, false, 0.0f, k_on ? st.top_k : a.V};
    if (kind == CH_N) {
        c.by_rank = true;
        c.has_t = true;
        c.T = st.top_p;
    } else if (kind == CH_K) {
        c.by_rank = true;
        const int f = b.cs[CH_N].found;
        c.n = f >= 0 ? f + 1 : b.cs[CH_N].n;
    } else if (kind == CH_W) {
        c.has_t = true;
        c.T = step_draw(a, st.step);
    }
    return c;
}

// A running sum (kind CH_*) over n terms in three launches:
//   chain_sum_kernel    per chunk of kChainChunk terms (a wavefront each),
//                       a double sum in any order;
//   chain_quant_kernel  per chunk, the starting binade guessed from the
//                       double prefix, and under it the chunk's and its
//                       groups' integer sums and tie prefixes (the groups'
//                       also under the next binade);
//   chain_walk_kernel   one wavefront walks the chunks: a chunk whose guess
//                       holds (the running sum is in that binade, no flag,
//                       its ties settled, the integer sum stays inside the
//                       binade and, with a threshold, the sum at its end does
//                       not exceed it) advances in one step; in any other,
//                       each group of 64 terms advances in one step the same
//                       way under its binade, or is added term by term
//                       (chain_group).  CH_W then emits the token.
__global__ __launch_bounds__(64) void chain_sum_kernel(const SampleArgs a, int kind) {
    const DevState st = *a.st;
    const GenBufs b = gen_bufs(a);
    const ChainSpec cs = chain_spec(a, b, st, kind);
    const int lane = threadIdx.x;
    const int c = blockIdx.x;
    if (c * kChainChunk >= cs.n) return;
    float xs[kChainPer];
    chain_load(b, cs.by_rank, c, cs.n, lane, xs);
    double d = 0.0;
#pragma unroll
    for (int i = 0; i < kChainPer; i++) d += (double)xs[i];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) d += __shfl_xor(d, off, 64);
    if (lane == 0) chain_chunks(b)[c].dsum = d;
}

__global__ __launch_bounds__(128) void chain_quant_kernel(const SampleArgs a, int kind) {
    const DevState st = *a.st;
    const GenBufs b = gen_bufs(a);
    const ChainSpec cs = chain_spec(a, b, st, kind);
    const int lane = threadIdx.x & 63, bin = threadIdx.x >> 6;  // wavefront 0: bin 0 and the chunk, 1: bin 1
    const int c = blockIdx.x;
    if (c * kChainChunk >= cs.n) return;
    ChainChunkMeta *cm = chain_chunks(b);
    ChainGroupMeta *gm = chain_groups(b);
    // the double prefix at the chunk's start
    double pre = 0.0;
    for (int k = lane; k < c; k += 64) pre += cm[k].dsum;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) pre += __shfl_xor(pre, off, 64);
    float xs[kChainPer];
    chain_load(b, cs.by_rank, c, cs.n, lane, xs);
    // each group's guessed starting binade, from the prefix and the groups' sums
    int eg[kChainPer];
#pragma unroll
    for (int i = 0; i < kChainPer; i++) {
        const int e = (int)(__float_as_uint((float)pre) >> 23);
        eg[i] = e > 1 ? e : 1;
        pre += (double)wave_sum(xs[i]);
    }
    const unsigned long long below = (1ull << lane) - 1ull;
    uint32_t run = 0u;
    int nt = 0;
    bool cflag = false;
    {
#pragma unroll
        for (int i = 0; i < kChainPer; i++) {
            bool tie = false, fl = false;
            const uint32_t q = chain_q(xs[i], eg[i] + bin, tie, fl);
            const uint32_t incl = wave_incl_u32(q);
            const unsigned long long tm = __ballot(tie);
            const int gt = __builtin_popcountll(tm);
            const bool gflag = __ballot(fl) != 0ull;
            // the group's ties, first kGroupTies of them
            ChainGroupMeta g;
            g.q = lane_u32(incl, 63);
            g.tie[0] = g.tie[1] = 0u;
            unsigned long long tt = tm;
#pragma unroll
            for (int k = 0; k < kGroupTies; k++)
                if (tt) {
                    g.tie[k] = lane_u32(incl, __builtin_ctzll(tt));
                    tt &= tt - 1ull;
                }
            g.ntie_flag = (int16_t)(gflag ? -1 : gt);
            g.eguess = (int16_t)eg[i];
            if (lane == 0) gm[(size_t)bin * kChainMaxChunks * kChainPer + c * kChainPer + i] = g;
            if (bin == 0) {
                // the chunk's one-step advance: all its groups under the chunk's
                // guess (any group guessed otherwise makes it walk group by group)
                if (tie) {
                    const int slot = nt + __builtin_popcountll(tm & below);
                    if (slot < kChainTies) cm[c].ties[slot] = min(run + incl, kChainSat);
                }
                nt += gt;
                run = min(run + g.q, kChainSat);
                cflag |= gflag || eg[i] != eg[0];
            }
        }
    }
    if (bin == 0 && lane == 0) {
        cm[c].q = run;
        cm[c].ntie = nt;
        cm[c].flag = cflag || nt > kChainTies;
        cm[c].eguess = eg[0];
    }
}

// Chunks whose terms and group metadata the walk stages in LDS up front:
// the first chunk, flagged ones, ones whose guessed binade differs from the
// next chunk's, and, with a threshold, the one where the double prefix
// crosses it and its neighbours (in chunk order, the first kChainStaged).
constexpr int kChainStaged = 12;

__global__ __launch_bounds__(kChainThreads) void chain_walk_kernel(const SampleArgs a, int kind) {
    __shared__ uint32_t ties[kChainMaxChunks][kChainTies];
    __shared__ uint32_t cq[kChainMaxChunks];
    __shared__ int cnt[kChainMaxChunks], cfl[kChainMaxChunks], ceg[kChainMaxChunks], slot[kChainMaxChunks];
    __shared__ float sx[kChainStaged][kChainChunk];
    __shared__ ChainGroupMeta sg[kChainStaged][2 * kChainPer];
    __shared__ int staged[kChainStaged];
    __shared__ int nstaged, fb_sh;
    const DevState st = *a.st;
    const GenBufs b = gen_bufs(a);
    const ChainSpec cs = chain_spec(a, b, st, kind);
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int n = cs.n, nch = (n + kChainChunk - 1) / kChainChunk;
    const ChainChunkMeta *cm = chain_chunks(b);
    const ChainGroupMeta *gm = chain_groups(b);
    for (int k = t; k < nch * kChainTies; k += kChainThreads) {
        const int c = k / kChainTies, i = k % kChainTies;
        ties[c][i] = cm[c].ties[i];
    }
    for (int c = t; c < nch; c += kChainThreads) {
        cq[c] = cm[c].q;
        cnt[c] = cm[c].ntie;
        cfl[c] = cm[c].flag;
        ceg[c] = cm[c].eguess;
        slot[c] = -1;
    }
    __syncthreads();
    if (w == 0) {
        // pick the chunks to stage (one wavefront, chunks 64 at a time)
        int ns = 0;
        double pre = 0.0;
        for (int c0 = 0; c0 < nch && ns < kChainStaged; c0 += 64) {
            const int c = c0 + lane;
            const double d = c < nch ? cm[c].dsum : 0.0;
            double incl = d;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const double o = __shfl_up(incl, off, 64);
                if (lane >= off) incl += o;
            }
            const double before = pre + incl - d, after = pre + incl;
            bool want = false;
            if (c < nch) {
                want = c == 0 || cfl[c] || (c + 1 < nch && ceg[c + 1] != ceg[c]);
                // the threshold's chunk by the double prefix, and its neighbours
                if (cs.has_t && before <= 1.01 * cs.T && after >= 0.99 * cs.T) want = true;
            }
            const unsigned long long wm = __ballot(want);
            const int r = ns + __builtin_popcountll(wm & ((1ull << lane) - 1ull));
            if (want && r < kChainStaged) {
                slot[c] = r;
                staged[r] = c;
            }
            ns = min(kChainStaged, ns + __builtin_popcountll(wm));
            pre += __shfl(incl, 63, 64);
        }
        if (lane == 0) nstaged = ns;
    }
    __syncthreads();
    // stage them (all wavefronts)
    for (int k = w; k < nstaged; k += kChainThreads / 64) {
        const int c = staged[k];
        float xs[kChainPer];
        chain_load(b, cs.by_rank, c, n, lane, xs);
#pragma unroll
        for (int i = 0; i < kChainPer; i++) sx[k][i * 64 + lane] = xs[i];
        if (lane < 2 * kChainPer)
            sg[k][lane] = gm[(size_t)(lane / kChainPer) * kChainMaxChunks * kChainPer + c * kChainPer + lane % kChainPer];
    }
    __syncthreads();
    if (w == 0) {
        uint32_t s = 0u;  // +0.0
        int found = -1;
        float at = 0.0f;
        int c = 0;
        while (c < nch && found < 0) {
            // a run of chunks that each advance in one step without ties:
            // lanes hold chunks c .. c + 63; the integer sums are prefix-summed
            // and the run ends at the first chunk that does not qualify
            {
                const int cl = c + lane;
                const bool in = cl < nch;
                const int es = (int)(s >> 23);
                const int eu = es > 1 ? es : 1;
                const uint32_t m = es ? ((s & 0x7fffffu) | 0x800000u) : s;
                const bool ok = in && es < 255 && !cfl[cl] && ceg[cl] == eu && cnt[cl] == 0;
                const uint32_t incl = wave_incl_u32(ok ? cq[cl] : 0u);  // < 64 * 2^25: no wrap
                const uint32_t sl = ((uint32_t)(eu - 1) << 23) + m + incl;
                const bool good = ok && m + incl < (1u << 24) && !(cs.has_t && __uint_as_float(sl) > cs.T);
                const unsigned long long bad = __ballot(in && !good);
                const int f = bad ? __builtin_ctzll(bad) : min(64, nch - c);
                if (f > 0) s = lane_u32(sl, f - 1);
                c += f;
                if (f == 64 || c >= nch) continue;
            }
            // chunk c: in one step with its ties settled, or group by group
            {
                const int es = (int)(s >> 23);
                const int eg = ceg[c];
                if (es < 255 && !cfl[c]) {
                    const int eu = es > 1 ? es : 1;
                    const uint32_t m = es ? ((s & 0x7fffffu) | 0x800000u) : s;
                    if (eu == eg) {
                        uint32_t adj = 0u;
                        const int nt = cnt[c];
                        for (int i = 0; i < nt; i++) adj += (m + ties[c][i] + adj) & 1u;
                        const uint32_t mend = m + cq[c] + adj;  // < 2^26: no wrap
                        if (mend < (1u << 24)) {
                            const uint32_t sn = ((uint32_t)(eu - 1) << 23) + mend;
                            if (!cs.has_t || !(__uint_as_float(sn) > cs.T)) {
                                s = sn;
                                c++;
                                continue;
                            }
                        }
                    }
                }
            }
            // lanes 0-15 hold the groups' bin-0 metadata, 16-31 their bin-1
            float xs[kChainPer];
            ChainGroupMeta g{};
            const int sl = slot[c];
            if (sl >= 0) {
#pragma unroll
                for (int i = 0; i < kChainPer; i++) xs[i] = sx[sl][i * 64 + lane];
                if (lane < 2 * kChainPer) g = sg[sl][lane];
            } else {
                chain_load(b, cs.by_rank, c, n, lane, xs);
                if (lane < 2 * kChainPer)
                    g = gm[(size_t)(lane / kChainPer) * kChainMaxChunks * kChainPer + c * kChainPer + lane % kChainPer];
            }
            int i = 0;
            while (i < kChainPer && found < 0) {
                // a run of groups i .. that each advance in one step without
                // ties, under whichever bin matches the running binade
                {
                    const int gi = i + lane;
                    const bool in = lane < kChainPer - i;
                    const int es = (int)(s >> 23);
                    const int eu = es > 1 ? es : 1;
                    const uint32_t m = es ? ((s & 0x7fffffu) | 0x800000u) : s;
                    const int egi = __shfl((int)g.eguess, gi & (kChainPer - 1), 64);
                    const int bin = eu - egi;
                    const int srcl = (bin == 1 ? kChainPer : 0) + (gi & (kChainPer - 1));
                    const int ntf = __shfl((int)g.ntie_flag, srcl, 64);
                    const uint32_t q = (uint32_t)__shfl((int)g.q, srcl, 64);
                    const bool ok = in && es < 255 && (bin == 0 || bin == 1) && ntf == 0;
                    const uint32_t incl = wave_incl_u32(ok ? q : 0u);
                    const uint32_t sl2 = ((uint32_t)(eu - 1) << 23) + m + incl;
                    const bool good = ok && m + incl < (1u << 24) && !(cs.has_t && __uint_as_float(sl2) > cs.T);
                    const unsigned long long bad = __ballot(in && !good);
                    const int f = bad ? __builtin_ctzll(bad) : kChainPer - i;
                    if (f > 0) s = lane_u32(sl2, f - 1);
                    i += f;
                    if (i >= kChainPer) break;
                }
                // group i: in one step with up to kGroupTies ties settled, or term by term
                const int es2 = (int)(s >> 23);
                const int eu = es2 > 1 ? es2 : 1;
                const int bin = eu - (int)lane_u32((uint32_t)(int)g.eguess, i);
                bool done = false;
                if (es2 < 255 && (bin == 0 || bin == 1)) {
                    const int src = bin * kChainPer + i;
                    const int ntf = (int)lane_u32((uint32_t)(int)g.ntie_flag, src);
                    if (ntf >= 0 && ntf <= kGroupTies) {
                        const uint32_t m = es2 ? ((s & 0x7fffffu) | 0x800000u) : s;
                        uint32_t adj = 0u;
                        if (ntf > 0) adj += (m + lane_u32(g.tie[0], src) + adj) & 1u;
                        if (ntf > 1) adj += (m + lane_u32(g.tie[1], src) + adj) & 1u;
                        const uint32_t mend = m + lane_u32(g.q, src) + adj;
                        if (mend < (1u << 24)) {
                            const uint32_t sn = ((uint32_t)(eu - 1) << 23) + mend;
                            if (!cs.has_t || !(__uint_as_float(sn) > cs.T)) {
                                s = sn;
                                done = true;
                            }
                        }
                    }
                }
                if (!done) found = chain_group(xs[i], c * kChainChunk + i * 64, n, cs.has_t, cs.T, &s, &at);
                i++;
            }
            c++;
        }
        if (lane == 0) {
            ChainOut o;
            o.total = __uint_as_float(s);
            o.found = found;
            o.at = at;
            o.n = n;
            b.cs[kind] = o;
        }
    }
    if (kind != CH_W) return;
    __syncthreads();
    int pick = b.cs[CH_W].found;
    if (pick < 0) {
        // past the last partial sum: the first candidate with p > 0
        if (t == 0) fb_sh = 0x7fffffff;
        __syncthreads();
        int first = 0x7fffffff;
        for (int j = t; j < n; j += kChainThreads)
            if (chain_x(b, cs.by_rank, j) > 0.0f) {
                first = j;
                break;
            }
        if (first != 0x7fffffff) atomicMin(&fb_sh, first);
        __syncthreads();
        pick = fb_sh == 0x7fffffff ? 0 : fb_sh;
    }
    if (t == 0) emit_token(a, cs.by_rank ? rank_id(b, pick) : pick);
}

// Block-wide double sum of one value per thread (kBlock threads), returned
// to thread 0.
__device__ __forceinline__ double block_sum_d(double d, double *red4) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) d += __shfl_xor(d, off, 64);
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = d;
    __syncthreads();
    return (red4[0] + red4[1]) + (red4[2] + red4[3]);
}

// softmax numerators over the candidates (src/tensor.rs:1177-1179, :1057):
// e = expf(s - M) in candidate order (ids without top-k, ranks below k with
// it), one kChainChunk-term chunk per workgroup; each chunk's double sum
// goes to the running sum Z's metadata (chain_sum_kernel's work)
__global__ __launch_bounds__(kBlock) void sample_exp_kernel(const SampleArgs a) {
    __shared__ float red4[4];
    __shared__ double dred4[4];
    const DevState st = *a.st;
    const GenBufs b = gen_bufs(a);
    const float M = scaled_max(a, b, red4);
    const bool k_on = use_topk(st, a.V);
    const int n = k_on ? st.top_k : a.V;
    const int c = blockIdx.x;
    if (c * kChainChunk >= n) return;
    double d = 0.0;
#pragma unroll
    for (int r = 0; r < kChainChunk / kBlock; r++) {
        const int j = c * kChainChunk + r * kBlock + threadIdx.x;
        if (j < n) {
            const int id = k_on ? rank_id(b, j) : j;
            const float e = ref_expf(b.sc[id] - M);
            b.pr[id] = e;
            d += (double)e;
        }
    }
    d = block_sum_d(d, dred4);
    if (threadIdx.x == 0) chain_chunks(b)[c].dsum = d;
}

// p = e / Z over all ids (non-candidates hold 0)
// in candidate order, one chunk per workgroup; without a nucleus cut the
// chunk sums are those of the walk's running sum
__global__ __launch_bounds__(kBlock) void sample_norm_kernel(const SampleArgs a) {
    __shared__ double dred4[4];
    const DevState st = *a.st;
    const GenBufs b = gen_bufs(a);
    const float Z = b.cs[CH_Z].total;
    const bool k_on = use_topk(st, a.V);
    const int n = k_on ? st.top_k : a.V;
    const int c = blockIdx.x;
    if (c * kChainChunk >= n) return;
    double d = 0.0;
#pragma unroll
    for (int r = 0; r < kChainChunk / kBlock; r++) {
        const int j = c * kChainChunk + r * kBlock + threadIdx.x;
        if (j < n) {
            const int id = k_on ? rank_id(b, j) : j;
            const float p = b.pr[id] / Z;
            b.pr[id] = p;
            d += (double)p;
        }
    }
    if (a.use_p) return;
    d = block_sum_d(d, dred4);
    if (threadIdx.x == 0) chain_chunks(b)[c].dsum = d;
}

// The nucleus cut (src/tensor.rs:1192-1200): ranks below the cutoff get
// p / (kept sum), the others 0
__global__ __launch_bounds__(kBlock) void sample_renorm_kernel(const SampleArgs a) {
    const GenBufs b = gen_bufs(a);
    const ChainOut nc = b.cs[CH_N], kc = b.cs[CH_K];
    const int cutoff = kc.n;
    for (int j = blockIdx.x * kBlock + threadIdx.x; j < nc.n; j += gridDim.x * kBlock) {
        const int id = rank_id(b, j);
        b.pr[id] = j < cutoff ? b.pr[id] / kc.total : 0.0f;
    }
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
    const dim3 wide((a.V + kGenWide - 1) / kGenWide);
    hipLaunchKernelGGL(sample_scale_kernel, wide, dim3(kBlock), 0, s, a);
    if (a.use_k || a.use_p) {
        // all ids by (scaled logit, id) descending
        const dim3 rb((a.V + kRadixBlock - 1) / kRadixBlock);
        hipLaunchKernelGGL(sort_keys_kernel, wide, dim3(kBlock), 0, s, a);
        for (int pass = 0; pass < 4; pass++) {
            hipLaunchKernelGGL(radix_hist_kernel, rb, dim3(kBlock), 0, s, a, pass);
            hipLaunchKernelGGL(radix_scan_kernel, dim3(1), dim3(kRadixScanThreads), 0, s, a);
            hipLaunchKernelGGL(radix_scatter_kernel, rb, dim3(kBlock), 0, s, a, pass);
        }
    }
    // a running sum: chunk sums, chunk and group metadata, the walk
    const dim3 chunks((a.V + kChainChunk - 1) / kChainChunk);
    auto chain = [&](int kind, bool sums) {
        if (sums) hipLaunchKernelGGL(chain_sum_kernel, chunks, dim3(64), 0, s, a, kind);
        hipLaunchKernelGGL(chain_quant_kernel, chunks, dim3(128), 0, s, a, kind);
        hipLaunchKernelGGL(chain_walk_kernel, dim3(1), dim3(kChainThreads), 0, s, a, kind);
    };
    // the exp and norm passes leave the chunk sums of Z and (without a
    // nucleus cut) of the walk
    hipLaunchKernelGGL(sample_exp_kernel, chunks, dim3(kBlock), 0, s, a);
    chain(CH_Z, false);
    hipLaunchKernelGGL(sample_norm_kernel, chunks, dim3(kBlock), 0, s, a);
    if (a.use_p) {
        chain(CH_N, true);
        chain(CH_K, true);
        hipLaunchKernelGGL(sample_renorm_kernel, wide, dim3(kBlock), 0, s, a);
    }
    chain(CH_W, a.use_p != 0);
    return hipGetLastError();
}

}  // namespace tmg
