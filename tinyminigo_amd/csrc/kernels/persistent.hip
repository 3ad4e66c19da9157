// Persistent greedy decode for gfx950: `steps` whole decode steps (reference
// generate -> forward_token -> argmax, src/model.rs:631-656 and :392-491) in
// ONE cooperative launch.
//
// Every workgroup stays resident and walks the phases of the step
//   per layer: QKV GEMV (+RMSNorm, RoPE, KV append) | attention (split-K) |
//              [split merge] | o_proj GEMV (+merge, residual) |
//              gate/up GEMV (+RMSNorm, SwiGLU) | down GEMV (+residual)
//   then lm_head GEMV (+RMSNorm, argmax partials) | argmax + step advance
// separated by grid barriers.  Before waiting at a barrier a workgroup
// already issues the weight loads of its first block in the next phase
// (weights never depend on activations), so barrier latency hides behind HBM
// streaming: waves 1-3 issue theirs before the barrier; wave 0, whose lane 0
// runs the barrier's atomics and must not wait behind loads, right after it.
//
// Data produced and consumed inside the launch (activations, the new KV row,
// split partials, argmax keys, the step state) moves through device-scope
// (sc1) loads and stores; every workgroup waits for its own stores before it
// arrives at a barrier.  Weights, the RoPE table and KV rows written by
// earlier launches are read with ordinary cached loads; a KV row written in
// this launch is only ever read after its (single) write.
//
// Barrier: per-XCD-group arrival counters (workgroup b is in group b % 8) feed
// one top counter; counters only grow, each launch starts from the bases the
// previous launch left.  Every wait is bounded: a barrier that does not
// complete within ~1 s raises an error flag and stops all later waits, so the
// grid always drains.
#include "attn.cuh"
#include "common.cuh"
#include "gemv.cuh"
#include "kernels.hpp"

namespace tmg {
namespace {

constexpr unsigned kSpinLimit = 1u << 24;

struct BarState {
    unsigned k = 0;          // barriers passed in this launch
    unsigned base_top = 0, base_sub = 0, n_sub = 0;
    int x = 0;               // arrival group
    unsigned long long *trace = nullptr;  // set on workgroup 0 when tracing
};

__device__ __forceinline__ void grid_sync(GridBar *gb, BarState &bs) {
    __syncthreads();
    if (threadIdx.x == 0) {
        if (bs.trace) bs.trace[2 * bs.k] = __builtin_amdgcn_s_memrealtime();
        bs.k++;
        const unsigned old = __hip_atomic_fetch_add(&gb->sub[bs.x][0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old + 1u == bs.base_sub + bs.k * bs.n_sub)
            __hip_atomic_fetch_add(&gb->top[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned target = bs.base_top + bs.k * kBarGroups;
        unsigned spins = 0;
        while ((int)(__hip_atomic_load(&gb->top[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
            if (__hip_atomic_load(&gb->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
            __builtin_amdgcn_s_sleep(2);
            if (++spins > kSpinLimit) {
                __hip_atomic_store(&gb->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
        if (bs.trace) bs.trace[2 * bs.k - 1] = __builtin_amdgcn_s_memrealtime();
    }
    __syncthreads();
}

// End of a phase: own stores complete, waves 1-3 prefetch the next phase's
// first block, grid barrier, then wave 0 prefetches its share.  The returned
// registers never carry an earlier phase's values (zero when this workgroup
// has no block), so the compiler sees one short live range per phase.
template <int KC, int R>
__device__ __forceinline__ WeightRegs<KC, R> phase_end(GridBar *gb, BarState &bs, const GemvArgs *next, int bid) {
    __builtin_amdgcn_s_waitcnt(0);
    WeightRegs<KC, R> W;
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int c = 0; c < KC; c++) W.w[r][c] = u32x4{0u, 0u, 0u, 0u};
    const bool have = next && bid < (next->out + R - 1) / R;
    const int wave = threadIdx.x >> 6;
    if (have && wave != 0) gemv_load<KC, R>(*next, bid, W);
    grid_sync(gb, bs);
    if (have && wave == 0) gemv_load<KC, R>(*next, bid, W);
    return W;
}

__device__ __forceinline__ void phase_end_plain(GridBar *gb, BarState &bs) {
    __builtin_amdgcn_s_waitcnt(0);
    grid_sync(gb, bs);
}

// All blocks of one GEMV phase owned by this workgroup; W holds the first.
template <int KC, int PRO, int EPI>
__device__ __forceinline__ void gemv_phase(const GemvArgs &a, int tok, int pos, int bid, int G,
                                           WeightRegs<KC, gemv_rows<KC>()> W, float *scratch,
                                           float (*red)[gemv_rows<KC>()]) {
    constexpr int R = gemv_rows<KC>();
    const int nblk = (a.out + R - 1) / R;
    if (bid >= nblk) return;
    float xv[KC][8];
    gemv_prologue<KC, PRO, true>(a, tok, pos, xv, scratch, bid == 0);
    for (int b = bid; b < nblk; b += G) {
        WeightRegs<KC, R> Wn;
        const bool more = b + G < nblk;
        if (more) gemv_load<KC, R>(a, b + G, Wn);
        gemv_finish<KC, R, EPI, true>(a, b, pos, W, xv, red);
        __syncthreads();  // red is reused by the next block
        if (more) W = Wn;
    }
}

template <int KC_H, int KC_Q, int KC_I, int HD, int GROUP>
__global__ __launch_bounds__(kBlock, 2) void decode_persistent(const PersistArgs p) {
    constexpr int RH = gemv_rows<KC_H>(), RQ = gemv_rows<KC_Q>(), RI = gemv_rows<KC_I>();
    __shared__ AttnShared<HD, GROUP> sm;
    __shared__ float redH[4][RH], redQ[4][RQ], redI[4][RI];
    __shared__ float scratch[4];
    __shared__ unsigned long long s_key[16];

    const int bid = blockIdx.x, G = gridDim.x;
    const PersistPlan *plan = p.plan;
    GridBar *gb = p.bar;
    BarState bs;
    if (threadIdx.x == 0) {
        bs.x = bid % kBarGroups;
        bs.n_sub = (unsigned)((G - bs.x + kBarGroups - 1) / kBarGroups);
        bs.base_top = __hip_atomic_load(&gb->base_top, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bs.base_sub = __hip_atomic_load(&gb->base_sub[bs.x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (bid == 0 && p.trace) {
            bs.trace = p.trace + 1;
            p.trace[0] = __builtin_amdgcn_s_memrealtime();
        }
    }
    const int qd = p.nq * HD;

    WeightRegs<KC_H, RH> Wh;  // QKV, gate/up and lm_head blocks
#pragma unroll
    for (int r = 0; r < RH; r++)
#pragma unroll
        for (int c = 0; c < KC_H; c++) Wh.w[r][c] = u32x4{0u, 0u, 0u, 0u};
    if (bid < (plan->qkv[0].out + RH - 1) / RH) gemv_load<KC_H, RH>(plan->qkv[0], bid, Wh);

    for (int step = 0; step < p.steps; step++) {
        const int pos = (int)__hip_atomic_load(&p.st->pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int tok = (int)__hip_atomic_load(&p.st->cur_token, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int active = active_splits(pos + 1, p.nsplit);
        for (int l = 0; l < p.L; l++) {
            // QKV (+ embedding gather on layer 0), RoPE, KV append
            if (l == 0)
                gemv_phase<KC_H, PRO_EMBED_NORM, EPI_QKV>(plan->qkv[0], tok, pos, bid, G, Wh, scratch, redH);
            else
                gemv_phase<KC_H, PRO_NORM, EPI_QKV>(plan->qkv[l], tok, pos, bid, G, Wh, scratch, redH);
            const WeightRegs<KC_Q, RQ> Wo = phase_end<KC_Q, RQ>(gb, bs, &plan->o[l], bid);
            // attention items (KV head, split)
            for (int it = bid; it < p.nkv * active; it += G) {
                attn_item<HD, GROUP, true, false>(plan->attn[l], it % active, it / active, 0, pos, active, sm);
                __syncthreads();
            }
            if (!p.fused_merge) {
                phase_end_plain(gb, bs);
                // merge the splits into attn_out: one thread per (head, dim)
                for (int i = bid * kBlock + threadIdx.x; i < qd; i += G * kBlock) {
                    const int hh = i / HD, d = i - hh * HD;
                    const int g = hh / GROUP, hq = hh - g * GROUP;
                    const size_t base = (size_t)g * p.nsplit * GROUP + hq;
                    float M = -INFINITY;
                    for (int sp = 0; sp < active; sp++)
                        M = fmaxf(M, ldf<true>(p.part_ml + (base + (size_t)sp * GROUP) * 2));
                    float L = 0.0f, O = 0.0f;
                    for (int sp = 0; sp < active; sp++) {
                        const size_t pi = base + (size_t)sp * GROUP;
                        const float m = ldf<true>(p.part_ml + pi * 2);
                        const float w = (m == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m - M);
                        L = fmaf(ldf<true>(p.part_ml + pi * 2 + 1), w, L);
                        O = fmaf(ldf<true>(p.part + pi * HD + d), w, O);
                    }
                    stf<true>(p.attn_out + i, O / L);
                }
            }
            phase_end_plain(gb, bs);
            // o_proj + residual (merging the splits in its prologue when fused)
            if (p.fused_merge)
                gemv_phase<KC_Q, PRO_ATTN_COMBINE, EPI_RESID>(plan->o[l], tok, pos, bid, G, Wo, scratch, redQ);
            else
                gemv_phase<KC_Q, PRO_PLAIN, EPI_RESID>(plan->o[l], tok, pos, bid, G, Wo, scratch, redQ);
            Wh = phase_end<KC_H, RH>(gb, bs, &plan->gu[l], bid);
            // gate/up + SwiGLU
            gemv_phase<KC_H, PRO_NORM, EPI_SWIGLU>(plan->gu[l], tok, pos, bid, G, Wh, scratch, redH);
            const WeightRegs<KC_I, RI> Wd = phase_end<KC_I, RI>(gb, bs, &plan->down[l], bid);
            // down + residual
            gemv_phase<KC_I, PRO_PLAIN, EPI_RESID>(plan->down[l], tok, pos, bid, G, Wd, scratch, redI);
            Wh = phase_end<KC_H, RH>(gb, bs, l + 1 < p.L ? &plan->qkv[l + 1] : &plan->lm, bid);
        }
        // lm_head + argmax partials
        gemv_phase<KC_H, PRO_NORM, EPI_LOGITS>(plan->lm, tok, pos, bid, G, Wh, scratch, redH);
        // the next step's first QKV block does not depend on the chosen token
        Wh = phase_end<KC_H, RH>(gb, bs, step + 1 < p.steps ? &plan->qkv[0] : nullptr, bid);
        // argmax + step advance (src/model.rs:636-655)
        if (bid == 0) {
            unsigned long long best = kArgmaxInit;
            for (int i = threadIdx.x; i < p.nparts; i += kBlock) {
                const unsigned long long k = ldu64<true>(p.argmax_part + i);
                best = k > best ? k : best;
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                const unsigned long long o = shfl_xor_u64(best, off);
                best = o > best ? o : best;
            }
            if ((threadIdx.x & 63) == 0) s_key[threadIdx.x >> 6] = best;
            __syncthreads();
            if (threadIdx.x == 0) {
                for (int w = 1; w < kBlock / 64; w++) best = s_key[w] > best ? s_key[w] : best;
                int t = (int)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
                if (t < 0 || t >= p.V) t = 0;
                const int stp = (int)__hip_atomic_load(&p.st->step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (stp >= 0 && stp < p.hist_cap)
                    __hip_atomic_store(&p.history[stp], t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&p.st->cur_token, t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&p.st->step, stp + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&p.st->pos, pos + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        phase_end_plain(gb, bs);
    }
    // the next launch starts from these counter values
    if (bid == 0 && threadIdx.x == 0) {
        __hip_atomic_store(&gb->base_top, bs.base_top + bs.k * kBarGroups, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int x = 0; x < kBarGroups; x++) {
            const unsigned n = (unsigned)((G - x + kBarGroups - 1) / kBarGroups);
            const unsigned b = __hip_atomic_load(&gb->base_sub[x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&gb->base_sub[x], b + bs.k * n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int KC_H, int KC_Q, int KC_I, int HD, int GROUP>
const void *kernel_ptr() {
    return reinterpret_cast<const void *>(&decode_persistent<KC_H, KC_Q, KC_I, HD, GROUP>);
}

}  // namespace

// Instantiated shapes: (KC of hidden, KC of q dim, KC of intermediate, head
// dim, GQA group).  Other models use the per-kernel graph path.
const void *persistent_kernel(int kc_h, int kc_q, int kc_i, int hd, int group) {
#define TMG_PK(a, b, c, d, e) \
    if (kc_h == a && kc_q == b && kc_i == c && hd == d && group == e) return kernel_ptr<a, b, c, d, e>();
    TMG_PK(1, 1, 1, 16, 2)   // tiny Llama (hidden 64, I 128)
    TMG_PK(1, 1, 3, 128, 2)  // 1B-class (hidden 2048, I 6144)
    TMG_PK(2, 2, 5, 128, 4)  // 4B-class (hidden 2560, q 4096, I 10240)
#undef TMG_PK
    return nullptr;
}

hipError_t launch_persistent(const void *kernel, int grid, const PersistArgs &a, hipStream_t s) {
    void *args[] = {const_cast<PersistArgs *>(&a)};
    return hipLaunchCooperativeKernel(kernel, dim3(grid), dim3(kBlock), args, 0, s);
}

}  // namespace tmg
