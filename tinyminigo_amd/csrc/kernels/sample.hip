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
// Whole-vocabulary path (no top-k, or top_k > kSampleMaxK): one workgroup
// replaces each of the reference's sorts with a threshold search over the
// whole vocabulary (sample_general_kernel below).
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
// above kSampleMaxK.  One workgroup of kGenThreads.  Wave w owns the ids
// [w*wsz, (w+1)*wsz) (wsz a multiple of 256), lane l of it the ids
// w*wsz + 64*j + l, so every pass is coalesced; rows of 256 ids are the
// units of the id-order searches.  a.scratch holds the scaled logits [V]
// and the probabilities [V]; three wide kernels before it compute them (the
// probabilities only without top-k).  The orders the reference gets by
// sorting are found by threshold searches instead: among the selected ids,
// in a given order, the first at which a running total of weights exceeds
// a target.  Weight 1 in (scaled logit descending, id ascending) order gives
// the k-th largest logit; the probability as weight gives the nucleus cut
// (first cumulative sum > top_p) and the inverse-CDF walk.  Probability
// masses are summed in 2^-40 fixed point, so every sum is exact and
// independent of summation order.
// ---------------------------------------------------------------------------

constexpr int kGenThreads = 1024;
constexpr int kGenWaves = kGenThreads / 64;
constexpr int kGenRow = 256;       // ids per row of an id-order search
constexpr int kGenMaxRows = 64;    // rows per wave: one per lane
constexpr int kGenBins = 4096;     // 12-bit digits: key bits 31..20, 19..8, then 7..0
constexpr double kFx = 1099511627776.0;  // 2^40
static_assert(kGenWaves * kGenMaxRows * kGenRow >= kSampleMaxVocab, "rows must cover the vocabulary");

struct GenShared {
    union {
        unsigned long long bins[kGenBins];                 // key histogram
        unsigned long long rowt[kGenWaves][kGenMaxRows];   // row totals
    };
    unsigned long long wtot[kGenWaves];
    unsigned long long res[4];
    float fred[kGenWaves];
};

// Which ids this thread owns: i = base + 64*j, i < end.
struct GenLayout {
    int V, wsz, nrow, base, end;
    __device__ explicit GenLayout(int v) : V(v) {
        nrow = (V + kGenWaves * kGenRow - 1) / (kGenWaves * kGenRow);
        wsz = nrow * kGenRow;
        const int w = (int)(threadIdx.x >> 6);
        base = w * wsz + (int)(threadIdx.x & 63);
        end = min(V, (w + 1) * wsz);
    }
};

// f(i, s, p) over this thread's ids, with s = sc[i] and p = pr[i] (0 when
// pr is null) loaded kGenUnroll ids at a time, so one memory round trip
// covers 16 ids per lane.
constexpr int kGenUnroll = 16;
template <class F>
__device__ __forceinline__ void gen_each(const GenLayout &L, const float *sc, const float *pr, F f) {
    for (int i0 = L.base; i0 < L.end; i0 += 64 * kGenUnroll) {
        float sv[kGenUnroll], pv[kGenUnroll];
#pragma unroll
        for (int u = 0; u < kGenUnroll; u++) {
            const int i = i0 + 64 * u;
            sv[u] = i < L.end ? sc[i] : 0.0f;
            pv[u] = pr && i < L.end ? pr[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kGenUnroll; u++) {
            const int i = i0 + 64 * u;
            if (i < L.end) f(i, sv[u], pv[u]);
        }
    }
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

// Exclusive prefix over the workgroup's threads in thread order; *total gets
// the sum.  Begins and ends with a barrier.
__device__ unsigned long long block_excl_u64(unsigned long long v, GenShared &sh, unsigned long long *total) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const unsigned long long incl = wave_incl_u64(v);
    __syncthreads();
    if (lane == 63) sh.wtot[w] = incl;
    __syncthreads();
    unsigned long long before = 0, all = 0;
    for (int i = 0; i < kGenWaves; i++) {
        if (i < w) before += sh.wtot[i];
        all += sh.wtot[i];
    }
    __syncthreads();
    *total = all;
    return before + incl - v;
}

__device__ float block_max_f(float v, GenShared &sh) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) sh.fred[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = -INFINITY;
    for (int i = 0; i < kGenWaves; i++) m = fmaxf(m, sh.fred[i]);
    __syncthreads();
    return m;
}

__device__ float block_sum_f(float v, GenShared &sh) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) sh.fred[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = 0.0f;
    for (int i = 0; i < kGenWaves; i++) m += sh.fred[i];
    __syncthreads();
    return m;
}

// A value one thread found (or ~0 if none did), broadcast to all.
__device__ unsigned long long block_pick(bool mine, unsigned long long v, GenShared &sh) {
    if (threadIdx.x == 0) sh.res[2] = ~0ull;
    __syncthreads();
    if (mine) sh.res[2] = v;
    __syncthreads();
    const unsigned long long r = sh.res[2];
    __syncthreads();
    return r;
}

// Threshold search in id order: the first id whose running total of
// wf(i, s, p) (the weight of id i with s = sc[i], p = pr[i]; 0 when not
// selected) exceeds `rest`, or -1 when the total does not; *through gets the
// running total through that id.  Row totals (row
// r of wave w = its ids w*wsz + 256 r .. +255, i.e. lane l's ids for j =
// 4r .. 4r+3; thread w*64 + r then holds row r, so thread order is id
// order), a prefix scan over them, then one wavefront scans the 256 ids of
// the crossing row.
template <class Wf>
__device__ int id_threshold(const GenLayout &L, const float *sc, const float *pr, Wf wf, unsigned long long rest,
                            GenShared &sh, unsigned long long *through = nullptr) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    constexpr int RB = kGenUnroll / 4;  // rows per batch
    for (int r0 = 0; r0 < L.nrow; r0 += RB) {
        float sv[kGenUnroll], pv[kGenUnroll];
#pragma unroll
        for (int u = 0; u < kGenUnroll; u++) {
            const int i = L.base + (r0 * 4 + u) * 64;
            sv[u] = i < L.end ? sc[i] : 0.0f;
            pv[u] = pr && i < L.end ? pr[i] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < RB; q++) {
            unsigned long long v = 0;
#pragma unroll
            for (int u = 4 * q; u < 4 * q + 4; u++) {
                const int i = L.base + (r0 * 4 + u) * 64;
                if (i < L.end) v += wf(i, sv[u], pv[u]);
            }
            v = wave_sum_u64(v);
            if (lane == 0 && r0 + q < L.nrow) sh.rowt[w][r0 + q] = v;
        }
    }
    __syncthreads();
    const unsigned long long c = lane < L.nrow ? sh.rowt[w][lane] : 0ull;
    unsigned long long tot;
    const unsigned long long cum = block_excl_u64(c, sh, &tot);
    if (tot <= rest) return -1;
    const unsigned long long hit =
        block_pick(lane < L.nrow && cum <= rest && cum + c > rest, ((unsigned long long)t << 48) | cum, sh);
    const int row = (int)(hit >> 48);
    const unsigned long long left = rest - (hit & ((1ull << 48) - 1));
    const int first = (row >> 6) * L.wsz + (row & 63) * kGenRow;  // lane l: ids first + 4l .. first + 4l + 3
    if (t == 0) sh.res[2] = ~0ull;
    __syncthreads();
    if (w == 0) {
        unsigned long long q[4], m = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = first + 4 * lane + k;
            q[k] = i < L.V ? wf(i, sc[i], pr ? pr[i] : 0.0f) : 0ull;
            m += q[k];
        }
        const unsigned long long incl = wave_incl_u64(m);
        unsigned long long cu = incl - m;
        if (cu <= left && incl > left) {
            for (int k = 0; k < 4; k++) {
                cu += q[k];
                if (cu > left) {
                    sh.res[2] = (unsigned long long)(first + 4 * lane + k);
                    sh.res[3] = rest - left + cu;  // running total through this id
                    break;
                }
            }
        }
    }
    __syncthreads();
    const unsigned long long r = sh.res[2];
    if (through) *through = sh.res[3];
    __syncthreads();
    return r == ~0ull ? -1 : (int)r;
}

// Threshold search in (key descending, id ascending) order.  kw(i, s, p, k,
// w) says whether id i (scaled logit s, pr value p) is selected and sets its
// key k (uint32, larger first) and weight w.  A radix search over the key
// (12, 12, then 8 bits) finds the key at which the running total crosses
// `target`; ties at that key go in id order.  Returns the id, or -1 when the
// total of all selected ids does not exceed the target; *through gets the
// running total through the returned id.  Ids of weight 0 can never be the
// answer and are skipped.
template <class Kw>
__device__ int desc_threshold(const GenLayout &L, const float *sc, const float *pr, Kw kw,
                              unsigned long long target, GenShared &sh, unsigned long long *through = nullptr) {
    const int t = threadIdx.x;
    uint32_t pfx = 0;                  // key bits decided so far
    unsigned long long rest = target;  // target left after the heavier bins
    for (int lv = 0; lv < 3; lv++) {
        const int shift = lv == 0 ? 20 : lv == 1 ? 8 : 0;
        const uint32_t nb = lv == 2 ? 256u : 4096u;
        const int above = lv == 0 ? 32 : lv == 1 ? 20 : 8;  // pfx holds key >> above
        for (int i = t; i < kGenBins; i += kGenThreads) sh.bins[i] = 0;
        __syncthreads();
        gen_each(L, sc, pr, [&](int i, float s, float p) {
            uint32_t k;
            unsigned long long v;
            if (!kw(i, s, p, k, v) || !v) return;
            if (lv > 0 && (k >> above) != pfx) return;
            atomicAdd(&sh.bins[(k >> shift) & (nb - 1)], v);
        });
        __syncthreads();
        // thread t takes 4 bins from the top: nb-1-4t .. nb-4-4t
        unsigned long long c[4], mine = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int bin = (int)nb - 1 - 4 * t - j;
            c[j] = bin >= 0 ? sh.bins[bin] : 0ull;
            mine += c[j];
        }
        unsigned long long total;
        unsigned long long cum = block_excl_u64(mine, sh, &total);
        if (total <= rest) return -1;  // only possible at level 0
        int hit = -1;
        unsigned long long before = 0;
        if (cum <= rest && cum + mine > rest) {
            for (int j = 0; j < 4; j++) {
                if (cum + c[j] > rest) {
                    hit = (int)nb - 1 - 4 * t - j;
                    before = cum;
                    break;
                }
                cum += c[j];
            }
        }
        // the bin (12 bits) and the weight before it (< 2^52 for V <= 2^18)
        const unsigned long long r = block_pick(hit >= 0, ((unsigned long long)hit << 52) | before, sh);
        pfx = (pfx << (lv == 2 ? 8 : 12)) | (uint32_t)(r >> 52);
        rest -= r & ((1ull << 52) - 1);
    }
    const int id = id_threshold(
        L, sc, pr,
        [&](int i, float s, float p) {
            uint32_t k;
            unsigned long long v;
            return kw(i, s, p, k, v) && k == pfx ? v : 0ull;
        },
        rest, sh, through);
    // the ties' running total starts after the heavier keys' target - rest
    if (id >= 0 && through) *through += target - rest;
    return id;
}

// The elementwise front of the whole-vocabulary path, over many workgroups:
// each workgroup of 256 threads takes 2048 ids (thread t: ids g*2048 +
// 256 j + t).  a.scratch: sc [V] | pr [V] | part [kGenParts] maxima |
// part [kGenParts] sums | u64 part [kGenParts] walk masses.
constexpr int kGenWide = 2048;
constexpr int kGenParts = kSampleMaxVocab / kGenWide;
static_assert(kGenParts == 128 && kGenParts <= kBlock, "the scratch layout reserves 128 partials of each kind");

__device__ __forceinline__ float wg_reduce(float v, bool is_max, float *red4) {
    v = is_max ? wave_max(v) : wave_sum(v);
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = v;
    __syncthreads();
    return is_max ? fmaxf(fmaxf(red4[0], red4[1]), fmaxf(red4[2], red4[3])) : (red4[0] + red4[1]) + (red4[2] + red4[3]);
}

// The maximum of the first n partials (every workgroup reads the same
// values in the same order, so all get the same result).
__device__ __forceinline__ float parts_max(const float *part, int n, float *red4) {
    float m = -INFINITY;
    for (int i = threadIdx.x; i < n; i += kBlock) m = fmaxf(m, part[i]);
    const float r = wg_reduce(m, true, red4);
    __syncthreads();
    return r;
}

// pass 1: scaled logits (penalty, temperature; src/tensor.rs:1142-1154,
// :1168) and the workgroup maximum
__global__ __launch_bounds__(kBlock) void sample_scale_kernel(const SampleArgs a) {
    __shared__ float red4[4];
    const DevState st = *a.st;
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
            a.scratch[i] = v;
            mx = fmaxf(mx, v);
        }
    }
    const float m = wg_reduce(mx, true, red4);
    if (threadIdx.x == 0) a.scratch[2 * (size_t)a.V + blockIdx.x] = m;
}

// pass 2 (no top-k): pr = exp(s - M) and the workgroup sum
__global__ __launch_bounds__(kBlock) void sample_exp_kernel(const SampleArgs a) {
    __shared__ float red4[4];
    const DevState st = *a.st;
    if (st.top_k > 0 && st.top_k < a.V) return;  // top-k: the candidates come first
    const int nparts = (a.V + kGenWide - 1) / kGenWide;
    const float M = parts_max(a.scratch + 2 * (size_t)a.V, nparts, red4);
    const int base = blockIdx.x * kGenWide + threadIdx.x;
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < kGenWide / kBlock; j++) {
        const int i = base + j * kBlock;
        if (i < a.V) {
            const float e = expf(a.scratch[i] - M);
            a.scratch[a.V + i] = e;
            sum += e;
        }
    }
    const float S = wg_reduce(sum, false, red4);
    if (threadIdx.x == 0) a.scratch[2 * (size_t)a.V + kGenParts + blockIdx.x] = S;
}

// pass 3 (no top-k): pr = pr / S, S the partial sums added in order
__global__ __launch_bounds__(kBlock) void sample_norm_kernel(const SampleArgs a) {
    __shared__ float Ssh;
    const DevState st = *a.st;
    if (st.top_k > 0 && st.top_k < a.V) return;
    const int nparts = (a.V + kGenWide - 1) / kGenWide;
    if (threadIdx.x == 0) {
        const float *ps = a.scratch + 2 * (size_t)a.V + kGenParts;
        float S = 0.0f;
        for (int i = 0; i < nparts; i++) S += ps[i];
        Ssh = S;
    }
    __syncthreads();
    const float S = Ssh;
    const int base = blockIdx.x * kGenWide + threadIdx.x;
#pragma unroll
    for (int j = 0; j < kGenWide / kBlock; j++) {
        const int i = base + j * kBlock;
        if (i < a.V) a.scratch[a.V + i] = a.scratch[a.V + i] / S;
    }
}

__global__ __launch_bounds__(kGenThreads) void sample_general_kernel(const SampleArgs a) {
    __shared__ GenShared sh;
    const DevState st = *a.st;
    const GenLayout L(a.V);
    const int V = a.V, t = threadIdx.x;
    float *sc = a.scratch, *pr = a.scratch + V;
    // sc holds the scaled logits (sample_scale_kernel); without top-k pr
    // already holds the probabilities (sample_exp_kernel, sample_norm_kernel)
    // and the draw is sample_walk_kernel's, so only a nucleus cut is left
    if (!(st.top_k > 0 && st.top_k < V) && !(st.top_p < 1.0f)) return;

    // The orders below are (key descending, id ascending) with the scaled
    // logit as key for top-k and the walk after it -- the reference's sort --
    // and the probability for the nucleus, whose sort leaves ties
    // unspecified.
    // the key of a cut id (read by its owner), from array v
    auto cut_key = [&](const float *v, int cut) {
        const bool own = cut >= L.base && cut < L.end && ((cut - L.base) & 63) == 0;
        return (uint32_t)block_pick(own, own ? f32_order(v[cut]) : 0u, sh);
    };
    // top-k (0 < k < V): the k-th best scaled logit (kk, id kid); ids after
    // it in the order are not candidates
    const bool use_k = st.top_k > 0 && st.top_k < V;
    uint32_t kk = 0;
    int kid = V;
    if (use_k) {
        kid = desc_threshold(
            L, sc, nullptr,
            [](int, float s, float, uint32_t &k, unsigned long long &w) {
                k = f32_order(s);
                w = 1;
                return true;
            },
            (unsigned long long)(st.top_k - 1), sh);
        if (kid < 0) kid = V;  // unreachable: the count always exceeds k - 1
        kk = kid < V ? cut_key(sc, kid) : 0u;
    }
    if (use_k) {
        // softmax over the candidates: pr = exp(s - M) (0 for the others), S
        // their sum, then pr = pr / S, the reference's probabilities; M is
        // the overall maximum (the best id is always a candidate)
        float m = -INFINITY;
        const int nparts = (V + kGenWide - 1) / kGenWide;
        for (int i = t; i < nparts; i += kGenThreads) m = fmaxf(m, sc[2 * (size_t)V + i]);
        const float M = block_max_f(m, sh);
        float sum = 0.0f;
        gen_each(L, sc, nullptr, [&](int i, float s, float) {
            const uint32_t k = f32_order(s);
            const float e = (k > kk || (k == kk && i <= kid)) ? expf(s - M) : 0.0f;
            pr[i] = e;
            sum += e;
        });
        const float S = block_sum_f(sum, sh);
        gen_each(L, pr, nullptr, [&](int i, float e, float) { pr[i] = e / S; });
    }
    // nucleus: keep through the first cumulative probability above top_p (in
    // probability order), then divide the kept probabilities by their sum
    if (st.top_p < 1.0f) {
        unsigned long long kept = 0;
        const int cut = desc_threshold(
            L, pr, nullptr,
            [&](int, float p, float, uint32_t &k, unsigned long long &w) {
                k = f32_order(p);
                w = fx(p);
                return true;
            },
            fx(st.top_p), sh, &kept);
        if (cut >= 0) {
            const uint32_t ck = cut_key(pr, cut);
            const float sumk = (float)((double)kept / kFx);
            gen_each(L, pr, nullptr, [&](int i, float p, float) {
                const uint32_t k = f32_order(p);
                pr[i] = (k > ck || (k == ck && i <= cut)) ? p / sumk : 0.0f;
            });
        }
    }
    // without top-k the draw walks the ids in order: sample_walk_kernel
    if (!use_k) return;
    // the draw: inverse-CDF walk in descending scaled-logit order (the
    // top-k candidates are the sorted ids)
    const float r = step_draw(a, st.step);
    int pick = desc_threshold(
        L, sc, pr,
        [&](int, float s, float p, uint32_t &k, unsigned long long &w) {
            k = f32_order(s);
            w = fx(p);
            return true;
        },
        fx(r), sh);
    if (pick < 0) {
        // past the last cumulative sum (rounding): the first candidate with
        // p > 0 in walk order, i.e. the best key
        unsigned long long best = ~0ull;
        gen_each(L, sc, pr, [&](int i, float s, float p) {
            if (!(p > 0.0f)) return;
            const unsigned long long k = ((unsigned long long)~f32_order(s) << 32) | (uint32_t)i;
            best = k < best ? k : best;
        });
        if (t == 0) sh.res[2] = ~0ull;
        __syncthreads();
        atomicMin(&sh.res[2], best);
        __syncthreads();
        const unsigned long long k = sh.res[2];
        pick = k == ~0ull ? 0 : (int)(uint32_t)k;
    }
    if (t == 0) emit_token(a, pick);
}

// Without top-k: the inverse-CDF walk in id order (src/tensor.rs:1203-1212)
// over the probabilities in pr (after any nucleus cut), in 2^-40 fixed
// point.  Pass 1, one workgroup per 2048 ids: the chunk's mass.
__global__ __launch_bounds__(kBlock) void sample_walk_sums_kernel(const SampleArgs a) {
    __shared__ unsigned long long red4[4];
    const DevState st = *a.st;
    if (st.top_k > 0 && st.top_k < a.V) return;
    const int base = blockIdx.x * kGenWide + threadIdx.x;
    unsigned long long m = 0;
#pragma unroll
    for (int j = 0; j < kGenWide / kBlock; j++) {
        const int i = base + j * kBlock;
        if (i < a.V) m += fx(a.scratch[a.V + i]);
    }
    m = wave_sum_u64(m);
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0)
        reinterpret_cast<unsigned long long *>(a.scratch + 2 * (size_t)a.V + 2 * kGenParts)[blockIdx.x] =
            (red4[0] + red4[1]) + (red4[2] + red4[3]);
}

// Pass 2, one workgroup: the chunk where the running mass first exceeds the
// draw (a prefix over the chunk masses), then the id inside it (thread t
// holds ids 8t .. 8t+7 of the chunk, so thread order is id order).
__global__ __launch_bounds__(kBlock) void sample_walk_kernel(const SampleArgs a) {
    __shared__ unsigned long long wt[4];
    __shared__ unsigned long long pick_sh;
    const DevState st = *a.st;
    if (st.top_k > 0 && st.top_k < a.V) return;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const float *pr = a.scratch + a.V;
    const unsigned long long *parts =
        reinterpret_cast<const unsigned long long *>(a.scratch + 2 * (size_t)a.V + 2 * kGenParts);
    const int nparts = (a.V + kGenWide - 1) / kGenWide;  // <= kGenParts <= kBlock
    const unsigned long long rf = fx(step_draw(a, st.step));
    auto block_excl = [&](unsigned long long v, unsigned long long *tot) {
        const unsigned long long incl = wave_incl_u64(v);
        __syncthreads();
        if (lane == 63) wt[w] = incl;
        __syncthreads();
        unsigned long long before = 0;
        for (int i = 0; i < w; i++) before += wt[i];
        *tot = (wt[0] + wt[1]) + (wt[2] + wt[3]);
        return before + incl - v;
    };
    if (t == 0) pick_sh = ~0ull;
    const unsigned long long c = t < nparts ? parts[t] : 0ull;
    unsigned long long tot;
    const unsigned long long cum = block_excl(c, &tot);
    __syncthreads();
    if (t < nparts && cum <= rf && cum + c > rf) pick_sh = ((unsigned long long)t << 48) | cum;
    __syncthreads();
    const unsigned long long hit = pick_sh;
    __syncthreads();
    int pick = -1;
    if (hit != ~0ull) {
        const int g = (int)(hit >> 48);
        const unsigned long long left = rf - (hit & ((1ull << 48) - 1));
        const int i0 = g * kGenWide + 8 * t;
        unsigned long long q[8], m = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            q[k] = i0 + k < a.V ? fx(pr[i0 + k]) : 0ull;
            m += q[k];
        }
        unsigned long long t2;
        unsigned long long cu = block_excl(m, &t2);
        if (t == 0) pick_sh = ~0ull;
        __syncthreads();
        if (cu <= left && cu + m > left) {
            for (int k = 0; k < 8; k++) {
                cu += q[k];
                if (cu > left) {
                    pick_sh = (unsigned long long)(i0 + k);
                    break;
                }
            }
        }
        __syncthreads();
        pick = pick_sh == ~0ull ? -1 : (int)pick_sh;
    }
    if (pick < 0) {
        // past the last cumulative sum (rounding): the lowest id with p > 0
        unsigned long long best = ~0ull;
        for (int i = t; i < a.V; i += kBlock)
            if (pr[i] > 0.0f) {
                best = (unsigned long long)i;
                break;
            }
        __syncthreads();
        if (t == 0) pick_sh = ~0ull;
        __syncthreads();
        atomicMin(&pick_sh, best);
        __syncthreads();
        pick = pick_sh == ~0ull ? 0 : (int)pick_sh;
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
    const dim3 wide((a.V + kGenWide - 1) / kGenWide);
    hipLaunchKernelGGL(sample_scale_kernel, wide, dim3(kBlock), 0, s, a);
    hipLaunchKernelGGL(sample_exp_kernel, wide, dim3(kBlock), 0, s, a);
    hipLaunchKernelGGL(sample_norm_kernel, wide, dim3(kBlock), 0, s, a);
    hipLaunchKernelGGL(sample_general_kernel, dim3(1), dim3(kGenThreads), 0, s, a);
    hipLaunchKernelGGL(sample_walk_sums_kernel, wide, dim3(kBlock), 0, s, a);
    hipLaunchKernelGGL(sample_walk_kernel, dim3(1), dim3(kBlock), 0, s, a);
    return hipGetLastError();
}

}  // namespace tmg
