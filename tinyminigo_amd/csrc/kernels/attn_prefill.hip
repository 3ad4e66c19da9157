// Causal GQA prefill attention on bf16 MFMA (reference attention_batch,
// src/tensor.rs:1099-1139, used by forward_seq, src/model.rs:555-566).
//
// A workgroup owns 128 query columns -- 128/GROUP consecutive positions of
// the GROUP query heads that share KV head g -- and walks the causal range of
// the KV cache in blocks of 64 keys.  Each block of K and V is staged once in
// LDS for all GROUP heads.  The f32 operands are carried as split-bf16 pairs
// x = hi + lo (|x - hi - lo| <= 2^-18 |x|) and every product takes three MFMAs
// (hi*hi + hi*lo + lo*hi), so the scores and the output keep close to f32
// accuracy.
//
// Scores are computed transposed, S^T = K Q^T (v_mfma_f32_16x16x32_bf16: A =
// 16 keys x 32 dims, B = 32 dims x 16 query columns), which leaves every lane
// with the scores of one query column.  The online softmax (running max and
// sum per column, exp2 of log2-scaled scores) therefore needs no transposes,
// and the probabilities feed O^T += V^T P^T directly from registers: the
// contraction over keys may visit the keys in any order as long as both
// operands agree, so a lane's k-slots are the keys it already holds (4 from
// each of two adjacent 16-key tiles), and V^T is read from an LDS copy
// stored [dim][key] in the same order.
//
// The K and V rows are split into bf16 pairs once per layer by
// kv_split_kernel (V transposed per head), so the attention workgroups stage
// ready-made MFMA operands: each block's 64 KB are plain 16-byte copies, and
// the next block's copies are in flight while the current one is multiplied.
#include "common.cuh"
#include "kernels.hpp"

namespace tmg {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kPHD = 128;        // head dim
constexpr int kPKB = 64;         // keys per block
constexpr int kPCols = 128;      // query columns per workgroup
constexpr int kPWaves = 8;       // wavefronts per workgroup (two per SIMD)
constexpr int kPQT = kPCols / (16 * kPWaves);  // 16-column query tiles per wavefront
constexpr int kSVP = kPKB + 8;   // kv_split_kernel's transpose buffer row pitch, bf16
// One staged block: K hi / lo [64 keys][256 B] and V^T hi / lo [128 dims][128 B]
constexpr int kPKTile = kPKB * kPHD * 2, kPVTile = kPHD * kPKB * 2;
constexpr int kPStage = 2 * kPKTile + 2 * kPVTile;
constexpr int kPDma = kPStage / 1024 / kPWaves;  // 1 KB DMA instructions per wave per block

__device__ __forceinline__ void split2(float x, uint16_t &h, uint16_t &l) {
    h = f32_to_bf16_rne(x);
    l = f32_to_bf16_rne(x - bf16_to_f32(h));
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// 8 floats -> (hi, lo) bf16x8 fragments, two values per packed conversion
// (the same rounding as split2: hi = bf16(x), lo = bf16(x - hi), RNE)
__device__ __forceinline__ void split8(const float (&v)[8], bf16x8 &hi, bf16x8 &lo) {
    u32x4 h, l;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const f32x2 x = {v[2 * i], v[2 * i + 1]};
        const bf16x2 hb = __builtin_convertvector(x, bf16x2);
        const f32x2 hf = __builtin_convertvector(hb, f32x2);
        const bf16x2 lb = __builtin_convertvector(x - hf, bf16x2);
        h[i] = __builtin_bit_cast(uint32_t, hb);
        l[i] = __builtin_bit_cast(uint32_t, lb);
    }
    hi = __builtin_bit_cast(bf16x8, h);
    lo = __builtin_bit_cast(bf16x8, l);
}

__device__ __forceinline__ float max_xor16_32(float v) {
    {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    return v;
}

// Slot of a key (its position within its 64-key block) in a V^T row.  The
// P^T operand of O^T += V^T P^T gives lane (q4, r) the keys 4 q4 .. +3 of two
// adjacent 16-key tiles; within each 32-key group those eight keys are
// stored next to each other, so the lane reads its V^T operand as one
// 16-byte chunk: key y of the group (y < 16: tile one, else tile two) goes to
// slot 8 (y mod 16) / 4 + 4 (y / 16) + y mod 4.
__host__ __device__ constexpr int vt_slot(int row) {
    return (row & 32) | (((row & 15) >> 2) << 3) | ((row & 16) >> 2) | (row & 3);
}

// One workgroup per (64 positions, KV head): f32 K/V rows -> split-bf16 K
// [pos][kvd] and V^T [head][dim][slot] (through an LDS transpose; the keys of
// each 64-key block in vt_slot order); rows at or past n are zeros.
__global__ __launch_bounds__(kBlock) void kv_split_kernel(const KVSplitArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t sT[2][kPHD][kSVP];
    const int t = threadIdx.x;
    const int p0 = blockIdx.x * kPKB, g = blockIdx.y;
    const int kvd = a.nkv * kPHD;
    // K: 64 rows x 128 dims of head g, 4 floats per thread per step
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int row = (t >> 5) + 8 * i, d = 4 * (t & 31);
        const int pos = p0 + row;
        float4 k = make_float4(0.f, 0.f, 0.f, 0.f), v = k;
        if (pos < a.n) {
            k = *reinterpret_cast<const float4 *>(a.k_cache + (size_t)pos * kvd + g * kPHD + d);
            v = *reinterpret_cast<const float4 *>(a.v_cache + (size_t)pos * kvd + g * kPHD + d);
        }
        const float kk[4] = {k.x, k.y, k.z, k.w}, vv[4] = {v.x, v.y, v.z, v.w};
        uint16_t kh[4], kl[4];
        const int prow = vt_slot(row);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            split2(kk[j], kh[j], kl[j]);
            uint16_t vh, vl;
            split2(vv[j], vh, vl);
            sT[0][d + j][prow] = vh;
            sT[1][d + j][prow] = vl;
        }
        const size_t o = (size_t)pos * kvd + g * kPHD + d;
        *reinterpret_cast<u32x2 *>(a.kh + o) =
            u32x2{(uint32_t)kh[0] | ((uint32_t)kh[1] << 16), (uint32_t)kh[2] | ((uint32_t)kh[3] << 16)};
        *reinterpret_cast<u32x2 *>(a.kl + o) =
            u32x2{(uint32_t)kl[0] | ((uint32_t)kl[1] << 16), (uint32_t)kl[2] | ((uint32_t)kl[3] << 16)};
    }
    __syncthreads();
    // V^T: 128 dim rows x 64 positions, 16 bytes per thread per step
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = t + kBlock * i;
        const int d = c >> 3, col = (c & 7) * 8;
        const size_t o = ((size_t)g * kPHD + d) * a.vt_pitch + p0 + col;
        *reinterpret_cast<u32x4 *>(a.vth + o) = *reinterpret_cast<const u32x4 *>(&sT[0][d][col]);
        *reinterpret_cast<u32x4 *>(a.vtl + o) = *reinterpret_cast<const u32x4 *>(&sT[1][d][col]);
    }
}

// K and V^T blocks go global -> LDS by DMA (global_load_lds_dwordx4) into a
// two-stage ring: block kb + 1 is in flight while block kb is multiplied.
// LDS rows are unpadded, their 16-byte chunks XOR-swizzled so that a
// fragment read's 16 rows hit 16 distinct bank groups: K rows (256 B, 16
// chunks) by key & 15, V^T rows (128 B, 8 chunks) by (dim >> 1) & 7.  A DMA
// wave-instruction fills 1 KB: 4 K rows or 8 V^T rows.
__device__ __forceinline__ int k_chunk(int key, int c) { return c ^ (key & 15); }
__device__ __forceinline__ int vt_chunk(int dim, int c) { return c ^ ((dim >> 1) & 7); }

__device__ __forceinline__ void dma16(const uint16_t *src, unsigned char *dst) {
    __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

template <int GROUP>
__global__ __launch_bounds__(kPWaves * 64) void attn_prefill_kernel(const AttnArgs a) {
    constexpr int QB = kPCols / GROUP;  // query positions per workgroup
    __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * kPStage];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int r = lane & 15, q4 = lane >> 4;
    // workgroup L: KV head L % nkv, the (L / nkv)-th longest query block, so
    // the dispatch order is longest causal range first across all heads, and
    // as workgroups go to the 8 XCDs round robin, with nkv dividing 8 each
    // XCD streams only its heads' K/V through its L2
    const int nqb = (a.T + QB - 1) / QB;
    const int g = (int)blockIdx.x % a.nkv;
    const int qb = nqb - 1 - (int)blockIdx.x / a.nkv;
    const int kvd = a.nkv * kPHD, qd = a.nq * kPHD;

    // this lane's query column in each of its 16-column tiles
    int ti[kPQT], qpos[kPQT], qhead[kPQT];
#pragma unroll
    for (int qt = 0; qt < kPQT; qt++) {
        const int c = wave * kPQT * 16 + qt * 16 + r;
        const int hh = c / QB, p = c - hh * QB;
        ti[qt] = qb * QB + p;
        qpos[qt] = a.start + ti[qt];
        qhead[qt] = g * GROUP + hh;
    }
    const int last_pos = a.start + min(a.T, (qb + 1) * QB) - 1;  // the workgroup's last query position
    const int nkb = last_pos / kPKB + 1;

    // Q is pre-scaled by scale / ln 2, so the scores come out in log2 units
    const float sl2 = a.scale * 1.4426950408889634f;
    // Q^T fragments (MFMA B operand): dims 32 ds + 8 q4 .. +7 of the column.
    // Loaded and consumed before any DMA is issued: the DMA waits below count
    // only DMAs.
    bf16x8 qh[kPQT][4], ql[kPQT][4];
#pragma unroll
    for (int qt = 0; qt < kPQT; qt++) {
        const float *src = a.q + (size_t)min(ti[qt], a.T - 1) * qd + qhead[qt] * kPHD + 8 * q4;
#pragma unroll
        for (int ds = 0; ds < 4; ds++) {
            const float4 v0 = *reinterpret_cast<const float4 *>(src + 32 * ds);
            const float4 v1 = *reinterpret_cast<const float4 *>(src + 32 * ds + 4);
            const float v[8] = {v0.x * sl2, v0.y * sl2, v0.z * sl2, v0.w * sl2,
                                v1.x * sl2, v1.y * sl2, v1.z * sl2, v1.w * sl2};
            split8(v, qh[qt][ds], ql[qt][ds]);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // DMA map: wave w's instruction i fills 1 KB slice 2 w + (i & 1) of part
    // i / 2 (K hi, K lo, V^T hi, V^T lo): K rows 4 slice .., V^T rows 8 slice ..
    // K blocks go to a two-stage K ring, V^T blocks to a two-stage V ring.
    static_assert(kPDma == 8 && kPWaves == 8, "two slices of each part per wave");
    const uint16_t *dsrc[kPDma];
    int ddst[kPDma];
#pragma unroll
    for (int i = 0; i < kPDma; i++) {
        const int part = i / 2, sl = 2 * wave + (i & 1);
        if (part < 2) {
            const int key = 4 * sl + (lane >> 4), pc = lane & 15;
            dsrc[i] = (part ? a.kl : a.kh) + (size_t)key * kvd + g * kPHD + k_chunk(key, pc) * 8;
            ddst[i] = part * kPKTile + sl * 1024;
        } else {
            const int dim = 8 * sl + (lane >> 3), pc = lane & 7;
            dsrc[i] = (part == 3 ? a.vtl : a.vth) + ((size_t)g * kPHD + dim) * a.vt_pitch + vt_chunk(dim, pc) * 8;
            ddst[i] = (part - 2) * kPVTile + sl * 1024;
        }
    }
    constexpr int kKStage = 2 * kPKTile, kVStage = 2 * kPVTile;
    unsigned char *const sKring = smem, *const sVring = smem + 2 * kKStage;
    auto issue_k = [&](int kb) {  // K rows advance by 64 keys per block
#pragma unroll
        for (int i = 0; i < 4; i++) dma16(dsrc[i] + (size_t)kb * kPKB * kvd, sKring + (kb & 1) * kKStage + ddst[i]);
    };
    auto issue_v = [&](int kb) {  // V^T columns advance by 64 positions
#pragma unroll
        for (int i = 4; i < 8; i++) dma16(dsrc[i] + (size_t)kb * kPKB, sVring + (kb & 1) * kVStage + ddst[i]);
    };

    float m[kPQT], l[kPQT];
    f32x4 o[kPQT][8];
#pragma unroll
    for (int qt = 0; qt < kPQT; qt++) {
        m[qt] = -INFINITY;
        l[qt] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) o[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // S^T = K Q^T of block kb (K ring stage kb & 1): 4 key tiles x kPQT
    // query tiles.  The K fragments of dim step ds + 1 are read while step
    // ds is multiplied (the scheduling barriers keep the reads ahead).
    auto scores = [&](int kb, f32x4 (&s)[4][kPQT]) {
        const unsigned char *sK0 = sKring + (kb & 1) * kKStage, *sK1 = sK0 + kPKTile;
        bf16x8 kf[2][4][2];
        auto load = [&](int ds, bf16x8 (&f)[4][2]) {
#pragma unroll
            for (int kt = 0; kt < 4; kt++) {
                const int key = kt * 16 + r, ko = key * 256 + k_chunk(key, 4 * ds + q4) * 16;
                f[kt][0] = *reinterpret_cast<const bf16x8 *>(sK0 + ko);
                f[kt][1] = *reinterpret_cast<const bf16x8 *>(sK1 + ko);
            }
        };
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int qt = 0; qt < kPQT; qt++) s[kt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
        load(0, kf[0]);
#pragma unroll
        for (int ds = 0; ds < 4; ds++) {
            if (ds + 1 < 4) load(ds + 1, kf[(ds + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int qt = 0; qt < kPQT; qt++) {
                    const bf16x8 &kh = kf[ds & 1][kt][0], &kl = kf[ds & 1][kt][1];
                    s[kt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qh[qt][ds], s[kt][qt], 0, 0, 0);
                    s[kt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, ql[qt][ds], s[kt][qt], 0, 0, 0);
                    s[kt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qh[qt][ds], s[kt][qt], 0, 0, 0);
                }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // online softmax of block kb per query column (this lane holds keys
    // kb * 64 + 16 kt + 4 q4 + i); s becomes the probabilities.  Only blocks
    // that reach past the workgroup's first query position need the causal
    // mask.  The running maximum is raised only when a column's block
    // maximum exceeds it by more than 2^8: the probabilities are taken
    // against that reference (at most 2^8, no overflow) and O and the sum
    // stay consistently scaled, so most blocks skip the rescale of O.
    const int first_pos = a.start + qb * QB;
    auto softmax = [&](int kb, f32x4 (&s)[4][kPQT]) {
        const int k0 = kb * kPKB;
        const bool diag = k0 + kPKB - 1 > first_pos;
#pragma unroll
        for (int qt = 0; qt < kPQT; qt++) {
            if (diag) {
#pragma unroll
                for (int kt = 0; kt < 4; kt++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (k0 + 16 * kt + 4 * q4 + i > qpos[qt]) s[kt][qt][i] = -INFINITY;
            }
            float mx = s[0][qt][0];
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) mx = fmaxf(mx, s[kt][qt][i]);
            mx = max_xor16_32(mx);  // finite: key 0 precedes every query
            const bool raise = mx > m[qt] + 8.0f;
            if (__builtin_amdgcn_ballot_w64(raise)) {
                const float corr = raise ? __builtin_amdgcn_exp2f(m[qt] - mx) : 1.0f;
                m[qt] = raise ? mx : m[qt];
                l[qt] *= corr;
#pragma unroll
                for (int dt = 0; dt < 8; dt++) o[qt][dt] *= corr;
            }
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float p = __builtin_amdgcn_exp2f(s[kt][qt][i] - m[qt]);
                    s[kt][qt][i] = p;
                    l[qt] += p;
                }
        }
    };
    // O^T += V^T P^T of block kb (V ring stage kb & 1), 32 keys per step:
    // tiles 2 ks and 2 ks + 1.  All 16 V^T fragments of a step are read
    // before its MFMAs, which then wait only for the ones they use.
    auto accumulate = [&](int kb, const f32x4 (&s)[4][kPQT]) {
        const unsigned char *sV0 = sVring + (kb & 1) * kVStage, *sV1 = sV0 + kPVTile;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            bf16x8 vf[8][2];
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                // keys 32 ks + 4 q4 .. +3 and 32 ks + 16 + 4 q4 .. +3: slots 32 ks + 8 q4 .. +7
                const int dim = dt * 16 + r, vo = dim * 128 + vt_chunk(dim, 4 * ks + q4) * 16;
                vf[dt][0] = *reinterpret_cast<const bf16x8 *>(sV0 + vo);
                vf[dt][1] = *reinterpret_cast<const bf16x8 *>(sV1 + vo);
            }
            bf16x8 ph[kPQT], pl[kPQT];
#pragma unroll
            for (int qt = 0; qt < kPQT; qt++) {
                const float pv[8] = {s[2 * ks][qt][0],     s[2 * ks][qt][1],     s[2 * ks][qt][2],
                                     s[2 * ks][qt][3],     s[2 * ks + 1][qt][0], s[2 * ks + 1][qt][1],
                                     s[2 * ks + 1][qt][2], s[2 * ks + 1][qt][3]};
                split8(pv, ph[qt], pl[qt]);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int dt = 0; dt < 8; dt++)
#pragma unroll
                for (int qt = 0; qt < kPQT; qt++) {
                    o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[dt][0], ph[qt], o[qt][dt], 0, 0, 0);
                    o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[dt][0], pl[qt], o[qt][dt], 0, 0, 0);
                    o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[dt][1], ph[qt], o[qt][dt], 0, 0, 0);
                }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Software pipeline: iteration kb computes the scores of block kb + 1
    // and the softmax of block kb, then O += V^T P^T of block kb.  The two
    // wavefronts of a SIMD (w and w + 4) take those first two in opposite
    // orders, so one's score MFMAs run while the other's softmax occupies
    // the vector ALU.  K(kb + 1) and V(kb) are needed in iteration kb:
    // issued in iteration kb - 1, waited for (vmcnt 0, only DMAs are
    // outstanding) before the barrier that also retires every wave's reads
    // of the stages K(kb + 2) and V(kb + 1) then overwrite.
    issue_k(0);
    issue_v(0);
    if (nkb > 1) issue_k(1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    f32x4 sc[2][4][kPQT];
    scores(0, sc[0]);
    const bool scores_first = wave < 4;
    auto iteration = [&](int kb, f32x4 (&cur)[4][kPQT], f32x4 (&nxt)[4][kPQT]) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (kb + 2 < nkb) issue_k(kb + 2);
        if (kb + 1 < nkb) issue_v(kb + 1);
        if (scores_first) {
            if (kb + 1 < nkb) scores(kb + 1, nxt);
            softmax(kb, cur);
        } else {
            softmax(kb, cur);
            if (kb + 1 < nkb) scores(kb + 1, nxt);
        }
        accumulate(kb, cur);
    };
    int kb = 0;
    for (; kb + 1 < nkb; kb += 2) {
        iteration(kb, sc[0], sc[1]);
        iteration(kb + 1, sc[1], sc[0]);
    }
    if (kb < nkb) iteration(kb, sc[0], sc[1]);
    // normalize and write the split-bf16 output: O^T rows dims 16 dt + 4 q4 + i
#pragma unroll
    for (int qt = 0; qt < kPQT; qt++) {
        const float L = add_xor32(add_xor16(l[qt]));  // the column's four lane groups
        if (ti[qt] >= a.T) continue;
        const float inv = 1.0f / L;
        const size_t ob = (size_t)ti[qt] * qd + qhead[qt] * kPHD;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int d = dt * 16 + 4 * q4 + i;
                split_bf16(o[qt][dt][i] * inv, a.out_hi + ob + d, a.out_lo + ob + d);
            }
        }
    }
}

}  // namespace

hipError_t launch_kv_split(const KVSplitArgs &a, hipStream_t s) {
    if (a.hd != kPHD || a.n <= 0 || a.vt_pitch < (a.n + kPKB - 1) / kPKB * kPKB || a.vt_pitch % 8)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(kv_split_kernel, dim3((a.n + kPKB - 1) / kPKB, a.nkv), dim3(kBlock), 0, s, a);
    return hipGetLastError();
}

bool attn_prefill_supported(const AttnArgs &a) {
    const int group = a.nkv > 0 ? a.nq / a.nkv : 0;
    // short prompts keep the per-row kernel: a few query blocks cannot fill the chip
    return a.hd == kPHD && a.out_hi && a.out_lo && a.nq == group * a.nkv && a.T >= kTiledMinTokens &&
           (group == 1 || group == 2 || group == 4 || group == 8);
}

hipError_t launch_attn_prefill(const AttnArgs &a, hipStream_t s) {
    if (!attn_prefill_supported(a) || a.T <= 0 || !a.kh || !a.kl || !a.vth || !a.vtl ||
        a.vt_pitch < (a.start + a.T + kPKB - 1) / kPKB * kPKB || a.vt_pitch % 8)
        return hipErrorInvalidValue;
    const int group = a.nq / a.nkv;
    const int QB = kPCols / group;
    const dim3 grid(((a.T + QB - 1) / QB) * a.nkv);
    switch (group) {
        case 1: hipLaunchKernelGGL(attn_prefill_kernel<1>, grid, dim3(kPWaves * 64), 0, s, a); break;
        case 2: hipLaunchKernelGGL(attn_prefill_kernel<2>, grid, dim3(kPWaves * 64), 0, s, a); break;
        case 4: hipLaunchKernelGGL(attn_prefill_kernel<4>, grid, dim3(kPWaves * 64), 0, s, a); break;
        case 8: hipLaunchKernelGGL(attn_prefill_kernel<8>, grid, dim3(kPWaves * 64), 0, s, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace tmg
