// GQA attention over the f32 KV cache as a device function of the decode
// attention kernel (decode.hip), also used for the per-row prefill attention
// of short prompts.
//
// Reference: decode attention src/model.rs:434-459, attention_batch
// src/tensor.rs:1099-1139, softmax src/tensor.rs:1055-1060.
//
// One call handles one (query row, KV head, split) item: the split's
// 64-position blocks of the row's context, for all GROUP query heads of the
// KV head, so every K/V load serves GROUP heads.  TS = HD/(4 VPL) lanes own
// one position (VPL float4s of K and of V each, interleaved so one load
// instruction covers TS x 16 contiguous bytes); the NT threads form NTEAM
// such teams.  Each team keeps its own online-softmax state (running max,
// sum, output) over the positions it visits, so the chunk loop has no
// block-wide synchronization; K and V of a 64-position chunk are loaded
// together and the next chunk is prefetched while the current one is
// computed.  At the end the teams of a wavefront are merged across lanes,
// then the wavefronts in LDS.
#pragma once

#include "common.cuh"
#include "kernels.hpp"

namespace tmg {

// Lane geometry: VPL float4s per lane, TS lanes per position, NTEAM teams, J
// positions per team per chunk of CH positions.  Two float4s per lane at
// head_dim 128 halve the cross-lane reduction steps per score against one
// (measured faster with two query heads per KV head, slower with four, where
// the doubled accumulator registers cost more than the reductions saved).
template <int HD, int GROUP, int NT = kBlock, int CHW = kAttnBlockLong>
struct AttnGeom {
    static constexpr int VPL = attn_vpl(HD, GROUP);
    static constexpr int TS = HD / (4 * VPL);
    static constexpr int NTEAM = NT / TS;
    static constexpr int J = CHW > NTEAM ? CHW / NTEAM : 1;
    static constexpr int CH = NTEAM * J;
    static_assert(CH == attn_chunk(HD, GROUP, NT, CHW), "host and device chunk widths agree");
};

// One merged (o, max, sum) state per wavefront: the teams of a wavefront are
// merged across lanes before the wavefronts are merged through LDS.
template <int HD, int GROUP, int NT = kBlock>
struct AttnShared {
    static constexpr int NWAVE = NT / 64;
    float o[NWAVE][GROUP][HD];
    float m[NWAVE][GROUP];
    float l[NWAVE][GROUP];
};

// Split count of a decode attention row at context n_ctx: the same formula in
// the attention kernel, its combine kernel and the fused combine prologue.
__device__ __forceinline__ int active_splits(int n_ctx, int nsplit, int block) {
    return min(nsplit, (n_ctx + block - 1) / block);
}

// Partition of a row's context [0, n_ctx) over the splits: blocks of CH
// positions (one chunk of the lane geometry) dealt round robin, split s
// taking blocks s, s + nsplit, s + 2 nsplit, ...  So split s always starts at
// position CH s, and the active splits are min(nsplit, ceil(n_ctx / CH)).

// With out_f32/out_hi null, or more than one active split, writes (o, max,
// sum) partials (a split without positions writes max = -inf, sum = 0);
// otherwise writes the normalized row.
// With SPEC (decode), the split's first chunk [CH split, + CH) is loaded
// before the position is read from a.pos_dev (rows clamped to the cache
// capacity a.cap), so the K/V loads do not wait for it; qpos and active are
// then computed here and the arguments ignored.  Splits found inactive
// return at once.
// x combined with its copies in the lanes OFF, 2 OFF, ... < 64 apart (the
// teams of a wavefront): the 16- and 32-lane exchanges are permlane swaps
// (VALU), the others LDS-crossbar shuffles.
template <int OFF, bool MAX>
__device__ __forceinline__ float team_reduce(float x) {
#pragma unroll
    for (int off = OFF; off < 64; off <<= 1) {
        float y;
        if (off == 16 || off == 32) {
            const auto r = off == 32 ? __builtin_amdgcn_permlane32_swap(as_u32(x), as_u32(x), false, false)
                                     : __builtin_amdgcn_permlane16_swap(as_u32(x), as_u32(x), false, false);
            // r[0] and r[1] hold x and its partner in one order or the other
            x = from_u32<float>(r[0]);
            y = from_u32<float>(r[1]);
        } else {
            y = __shfl_xor(x, off, 64);
        }
        x = MAX ? fmaxf(x, y) : x + y;
    }
    return x;
}

template <int HD, int GROUP, bool SPEC = false, int NT = kBlock, int CHW = kAttnBlockLong>
__device__ __forceinline__ void attn_item(const AttnArgs &a, int split, int g, int ti, int qpos, int active,
                                          AttnShared<HD, GROUP, NT> &sm) {
    using G = AttnGeom<HD, GROUP, NT, CHW>;
    constexpr int VPL = G::VPL, TS = G::TS, NTEAM = G::NTEAM;
    constexpr int J = G::J;  // positions per team per chunk
    constexpr int CH = G::CH;
    const int t = threadIdx.x, lt = t % TS, team = t / TS;
    const int kvd = a.nkv * HD;
    const int qd = a.nq * HD;
    // lane lt owns dims (v TS + lt) 4 .. + 3 for v < VPL
    const float *kbase = (a.k_seq ? a.k_seq[ti] + a.kv_layer_off : a.k_cache) + g * HD + lt * 4;
    const float *vbase = (a.v_seq ? a.v_seq[ti] + a.kv_layer_off : a.v_cache) + g * HD + lt * 4;

    float4 qv[GROUP][VPL];
    const float *qrow = a.q + (size_t)ti * qd;
#pragma unroll
    for (int h = 0; h < GROUP; h++)
#pragma unroll
        for (int v = 0; v < VPL; v++) qv[h][v] = *reinterpret_cast<const float4 *>(qrow + (g * GROUP + h) * HD + (v * TS + lt) * 4);

    float4 kr[J][VPL], vr[J][VPL];
    auto load_kv = [&](float4(&kd)[J][VPL], float4(&vd)[J][VPL], int c0, int lim) {
#pragma unroll
        for (int j = 0; j < J; j++) {
            const int p = min(c0 + team + j * NTEAM, lim);
#pragma unroll
            for (int v = 0; v < VPL; v++) {
                kd[j][v] = *reinterpret_cast<const float4 *>(kbase + (size_t)p * kvd + v * TS * 4);
                vd[j][v] = *reinterpret_cast<const float4 *>(vbase + (size_t)p * kvd + v * TS * 4);
            }
        }
    };
    const int c_first = split * CH, c_step = a.nsplit * CH;
    if constexpr (SPEC) {
        const int pos0 = *a.pos_dev;  // a scalar load, first used after the K/V loads are issued
        load_kv(kr, vr, c_first, a.cap - 1);
        // keep the loads above the position read: without this fence the
        // compiler sinks them behind it (into the branch that uses them)
        asm volatile("" ::: "memory");
        qpos = pos0 + ti;
        active = active_splits(qpos + 1, a.nsplit, CH);
        if (split >= active) return;
    }
    const int n_ctx = qpos + 1;
    const float sl2 = a.scale * 1.4426950408889634f;  // scores in log2 units: softmax by exp2

    float m_run[GROUP], l_run[GROUP];
    float4 o_acc[GROUP][VPL];
#pragma unroll
    for (int h = 0; h < GROUP; h++) {
        m_run[h] = -INFINITY;
        l_run[h] = 0.0f;
#pragma unroll
        for (int v = 0; v < VPL; v++) o_acc[h][v] = make_float4(0.f, 0.f, 0.f, 0.f);
    }

    // Rows past the context are loaded clamped (branch-free) and masked where
    // used: their score is -inf and their V row is replaced by zeros (0 *
    // garbage could be NaN).
    const int last = n_ctx - 1;
    if constexpr (!SPEC) load_kv(kr, vr, c_first, last);
    for (int c0 = c_first; c0 < n_ctx; c0 += c_step) {
        float4 kn[J][VPL], vn[J][VPL];
        const bool more = c0 + c_step < n_ctx;
        if (more) load_kv(kn, vn, c0 + c_step, last);
        // scores of this team's positions (every lane of the team gets them)
        float s[J][GROUP];
#pragma unroll
        for (int j = 0; j < J; j++) {
            const bool ok = c0 + team + j * NTEAM < n_ctx;
#pragma unroll
            for (int h = 0; h < GROUP; h++) {
                float d = 0.0f;
                if (ok) {
                    d = qv[h][0].x * kr[j][0].x;
                    d = fmaf(qv[h][0].y, kr[j][0].y, d);
                    d = fmaf(qv[h][0].z, kr[j][0].z, d);
                    d = fmaf(qv[h][0].w, kr[j][0].w, d);
#pragma unroll
                    for (int v = 1; v < VPL; v++) {
                        d = fmaf(qv[h][v].x, kr[j][v].x, d);
                        d = fmaf(qv[h][v].y, kr[j][v].y, d);
                        d = fmaf(qv[h][v].z, kr[j][v].z, d);
                        d = fmaf(qv[h][v].w, kr[j][v].w, d);
                    }
                }
                d = group_sum<TS>(d);
                s[j][h] = ok ? d * sl2 : -INFINITY;
            }
        }
        // online softmax update of the team's state
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            float mc = -INFINITY;
#pragma unroll
            for (int j = 0; j < J; j++) mc = fmaxf(mc, s[j][h]);
            if (mc == -INFINITY) continue;  // no position of this team in the chunk
            const float m_new = fmaxf(m_run[h], mc);
            const float corr = (m_run[h] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run[h] - m_new);
            float l = l_run[h] * corr;
            float4 o[VPL];
#pragma unroll
            for (int v = 0; v < VPL; v++)
                o[v] = make_float4(o_acc[h][v].x * corr, o_acc[h][v].y * corr, o_acc[h][v].z * corr,
                                   o_acc[h][v].w * corr);
#pragma unroll
            for (int j = 0; j < J; j++) {
                const bool ok = s[j][h] != -INFINITY;
                const float p = ok ? __builtin_amdgcn_exp2f(s[j][h] - m_new) : 0.0f;
                l += p;
#pragma unroll
                for (int v = 0; v < VPL; v++) {
                    const float4 x = ok ? vr[j][v] : make_float4(0.f, 0.f, 0.f, 0.f);
                    o[v].x = fmaf(p, x.x, o[v].x);
                    o[v].y = fmaf(p, x.y, o[v].y);
                    o[v].z = fmaf(p, x.z, o[v].z);
                    o[v].w = fmaf(p, x.w, o[v].w);
                }
            }
            m_run[h] = m_new;
            l_run[h] = l;
#pragma unroll
            for (int v = 0; v < VPL; v++) o_acc[h][v] = o[v];
        }
        if (more) {
#pragma unroll
            for (int j = 0; j < J; j++)
#pragma unroll
                for (int v = 0; v < VPL; v++) {
                    kr[j][v] = kn[j][v];
                    vr[j][v] = vn[j][v];
                }
        }
    }

    // merge the team states: the 64 / TS teams of a wavefront (lanes TS
    // apart) by cross-lane max and sums, then the wavefronts through LDS
    constexpr int NWAVE = NT / 64;
    const int wave = t >> 6, lane = t & 63;
#pragma unroll
    for (int h = 0; h < GROUP; h++) {
        const float M = team_reduce<TS, true>(m_run[h]);
        const float w = (m_run[h] == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run[h] - M);
        const float l = team_reduce<TS, false>(l_run[h] * w);
#pragma unroll
        for (int v = 0; v < VPL; v++) {
            const float4 o = make_float4(
                team_reduce<TS, false>(o_acc[h][v].x * w), team_reduce<TS, false>(o_acc[h][v].y * w),
                team_reduce<TS, false>(o_acc[h][v].z * w), team_reduce<TS, false>(o_acc[h][v].w * w));
            if (lane < TS) *reinterpret_cast<float4 *>(&sm.o[wave][h][(v * TS + lt) * 4]) = o;
        }
        if (lane == 0) {
            sm.m[wave][h] = M;
            sm.l[wave][h] = l;
        }
    }
    __syncthreads();
    const size_t row_hd = (size_t)ti * qd + g * GROUP * HD;
    const size_t pbase = (((size_t)ti * a.nkv + g) * a.nsplit + split) * GROUP;
    const bool direct = active == 1 && (a.out_f32 || a.out_hi);
    for (int idx = t; idx < GROUP * HD; idx += NT) {
        const int h = idx / HD, d = idx % HD;
        float M = -INFINITY;
#pragma unroll
        for (int tm = 0; tm < NWAVE; tm++) M = fmaxf(M, sm.m[tm][h]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int tm = 0; tm < NWAVE; tm++) {
            const float mt = sm.m[tm][h];
            const float w = (mt == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mt - M);
            L = fmaf(sm.l[tm][h], w, L);
            O = fmaf(sm.o[tm][h][d], w, O);
        }
        if (direct) {
            const float o = O / L;
            if (a.out_f32) a.out_f32[row_hd + idx] = o;
            if (a.out_hi) split_bf16(o, a.out_hi + row_hd + idx, a.out_lo + row_hd + idx);
        } else {
            a.part[(pbase + h) * HD + d] = O;
            if (d == 0) {
                a.part_ml[(pbase + h) * 2 + 0] = M;
                a.part_ml[(pbase + h) * 2 + 1] = L;
            }
        }
    }
}

}  // namespace tmg
