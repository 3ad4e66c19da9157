// Launch interface of the gfx950 kernels.  Host code includes this header;
// the kernels themselves live in decode.hip / prefill.hip / sample.hip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tmg {

// Packed argmax key: (orderable f32 bits << 32) | (0xFFFFFFFF - index), so a
// 64-bit atomicMax keeps the largest value and, among equal values, the
// lowest index -- the tie rule of the reference argmax (src/tensor.rs:1063).
// The initial key stands for (-inf, index 0): all -inf/NaN logits give 0.
constexpr unsigned long long kArgmaxInit = (0x007FFFFFull << 32) | 0xFFFFFFFFull;

// Per-cache device state read and advanced by the captured decode step.
struct DevState {
    int pos;                        // cache length = write position of the next token
    int cur_token;                  // input token of the next step
    int step;                       // index into the generated-token history
    int pad;
    unsigned long long argmax_key;  // running argmax of the current logits
    // sampling parameters of the running generate call (GenParams,
    // src/model.rs:597-604), read by the sampling kernels
    float temperature;
    int top_k;   // 0 or >= vocab: no top-k
    float top_p;
    float penalty;
};

enum GemvPro { PRO_PLAIN = 0, PRO_NORM = 1, PRO_NORM_BATCH = 2, PRO_EMBED_NORM = 3, PRO_ATTN_COMBINE = 4 };
enum GemvEpi { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_QKV = 3, EPI_LOGITS = 4 };

struct GemvArgs {
    const uint16_t *W;  // [out, in] BF16 rows (pair-interleaved for SWIGLU/QKV)
    // int8 rows instead (the TMG_I8 mode): [out, in] codes and [out] f32 row
    // scales, same row order as W; null selects the BF16 rows
    const int8_t *W8;
    const float *wscale;
    // f32 rows instead (WMat::F32: F32 / F16 matrices converted at load),
    // same row order as W; used when set and W8 is null
    const float *Wf;
    int out, in;
    const float *x;       // activation (PRO_PLAIN) or residual stream (PRO_NORM*)
    const float *norm_w;  // [in] f32 RMSNorm weight
    float eps;
    // PRO_EMBED_NORM: x is gathered from the embedding row of *token
    const int *token;
    const uint16_t *embed_bf16;  // [V, in] (one of the two is set)
    const float *embed_f32;
    float *x_store;  // block 0 stores the gathered row (the residual stream)
    // epilogue
    float *y;  // STORE/LOGITS: y[out]; RESID: y[out] += ; SWIGLU: y[out/2]
    // EPI_QKV
    const float *rope_cos, *rope_sin;  // [pos][hd/2]
    const int *pos;
    int hd, nq, nkv;
    float *q_out;            // [nq*hd]
    float *k_cache, *v_cache;  // layer base, [pos][nkv*hd]
    // EPI_LOGITS: one packed (value, row) argmax key per workgroup, or null
    unsigned long long *argmax_part;
    // PRO_ATTN_COMBINE: the activation is the attention output, merged from
    // the split-K partials of the decode attention kernel (see AttnArgs)
    const float *part, *part_ml;
    int nsplit, group, attn_block;
    // several sequences (launch_gemv_mt): nb activation rows x[b * in], outputs
    // y[b * out] (RESID) / y[b * out / 2] (SWIGLU) / q_out[b * nq * hd] (QKV),
    // argmax keys argmax_part[b * blocks + block] (LOGITS); sequence b is at
    // position pos_seq[b] with its K/V rows in k_seq[b] / v_seq[b] +
    // kv_layer_off
    int nb;
    const int *pos_seq;
    float *const *k_seq;
    float *const *v_seq;
    size_t kv_layer_off;
};

hipError_t launch_gemv(int pro, int epi, const GemvArgs &a, hipStream_t s);

// argmax of x[0, n) into *out (argmax.hip): argmax_parts(n) chunk keys in
// `part`, then one reduction.
uint32_t argmax_parts(uint32_t n);
hipError_t launch_argmax(const float *x, uint32_t n, uint32_t *out, unsigned long long *part, hipStream_t s);
// The decode GEMV over a.nb <= kMtMaxSeq activation rows at once (batched
// decode of several sequences): every weight row is read once and dotted
// with all rows.  PRO_NORM or PRO_PLAIN; EPI_QKV, EPI_RESID, EPI_SWIGLU or
// EPI_LOGITS (argmax keys only).  gemv_mt_blocks: workgroups of a launch.
constexpr int kMtMaxSeq = 8;
hipError_t launch_gemv_mt(int pro, int epi, const GemvArgs &a, hipStream_t s);
int gemv_mt_blocks(int out, int in, int nb);
// WMat::quantize_i8 of BF16 rows (src/tensor.rs:275-293, widened from BF16 as
// wmat_maybe_i8 does, src/model.rs:60-68): q8 [rows, in] codes and scale
// [rows].  With rewrite, w is overwritten with the codes as BF16 (exact), the
// dequantized weight up to the row scale, for the prefill GEMMs.
hipError_t launch_quantize_i8(uint16_t *w, int rows, int in, int8_t *q8, float *scale, bool rewrite,
                              hipStream_t s);
// The same from f32 rows (quantize_i8 of WMat::F32 values, src/model.rs:69-72):
// q8 codes, scales, and the codes as BF16 in `codes` [rows, in].
hipError_t launch_quantize_i8_f32(const float *w, int rows, int in, int8_t *q8, float *scale, uint16_t *codes,
                                  hipStream_t s);
// Workgroups (= argmax partials) of a GEMV launch with `out` rows of `in`
// (BF16 rows, or f32 rows with f32).
int gemv_blocks(int out, int in, bool f32 = false);

struct AttnArgs {
    const float *q;  // [T][nq*hd], RoPE applied
    const float *k_cache, *v_cache;  // layer base, [pos][nkv*hd]
    int nq, nkv, hd;
    int T;            // query rows (1 for decode)
    int start;        // position of query row 0 (decode: *pos_dev is used when pos_dev != null)
    const int *pos_dev;
    float scale;      // 1/sqrt(hd)
    int nsplit;       // grid.x
    int block;        // positions per block of the split partition (decode; 0 means kAttnBlockLong)
    int cap;          // rows of k_cache / v_cache (bounds the speculative first-chunk loads; 0 disables them)
    int spec_splits;  // splits that load their first chunk before the position read (0: kSpecSplits)
    float *part;      // [T][nkv][nsplit][group][hd] partial outputs
    float *part_ml;   // [T][nkv][nsplit][group][2] (max of the log2-scaled scores, sum)
    float *out_f32;   // [T][nq*hd] when one split covers the row, or null
    uint16_t *out_hi, *out_lo;  // [T][nq*hd] split-bf16 output (prefill), or null
    // several sequences at once (batched decode, nsplit 1): query row ti is
    // sequence ti at position pos_seq[ti] over its own cache k_seq[ti] /
    // v_seq[ti] + kv_layer_off
    const int *pos_seq;
    float *const *k_seq;
    float *const *v_seq;
    size_t kv_layer_off;
    // MFMA prefill attention: the cache rows [0, start+T) as split-bf16, keys
    // [pos][nkv*hd] and values transposed [nkv][hd][vt_pitch]
    const uint16_t *kh, *kl, *vth, *vtl;
    int vt_pitch;
};

// Split-bf16 copies of one layer's KV cache rows [0, n) for the MFMA prefill
// attention (rows up to the next multiple of 64 are zeros).
struct KVSplitArgs {
    const float *k_cache, *v_cache;  // [pos][nkv*hd]
    int n, nkv, hd;
    uint16_t *kh, *kl;               // [round64(n)][nkv*hd]
    uint16_t *vth, *vtl;             // [nkv][hd][vt_pitch], vt_pitch >= round64(n)
    int vt_pitch;
};
hipError_t launch_kv_split(const KVSplitArgs &a, hipStream_t s);

hipError_t launch_attn(const AttnArgs &a, hipStream_t s);
// Causal prefill attention on MFMA (head_dim 128, split-bf16 output): the
// shapes it takes, and the launch.
bool attn_prefill_supported(const AttnArgs &a);
hipError_t launch_attn_prefill(const AttnArgs &a, hipStream_t s);
// Merges the split-K partials of a decode attention launch (a.T rows) into
// out_f32 [T][nq*hd]: where the merge is not fused into the o_proj GEMV
// prologue (more than kFusedSplits splits; batched decode).
hipError_t launch_attn_combine(const AttnArgs &a, hipStream_t s);

struct FinalizeArgs {
    DevState *st;
    int *history;  // generated ids, indexed by st->step
    int advance_pos;  // 1 after a decode step, 0 after prefill
    int V;            // ids outside [0, V) become 0 before they index anything
    const unsigned long long *argmax_part;  // per-workgroup keys of the lm_head GEMV
    int nparts;
    int hist_cap;  // entries of history; ids at later steps are not recorded
};

hipError_t launch_finalize(const FinalizeArgs &a, hipStream_t s);

// Batched greedy decode (several sequences per step): the argmax of each of
// the B logit rows [B][V] becomes that sequence's next input token, is
// written to out[b * out_stride + pos[b] - plen[b]] when that index is below
// out_stride, and pos[b] advances.
struct BatchSelectArgs {
    const float *logits;
    int V, B;
    int *tokens, *pos;
    const int *plen;
    int *out;
    int out_stride;
};
hipError_t launch_batch_select(const BatchSelectArgs &a, hipStream_t s);
// The same selection from per-workgroup argmax keys [B][nparts] (the
// multi-row lm_head GEMV's).
hipError_t launch_batch_select_parts(const unsigned long long *parts, int nparts, const BatchSelectArgs &a,
                                     hipStream_t s);
// The first generated id of sequence b from a prefill's per-workgroup argmax
// keys: tokens[b] = id, out[b * out_stride] = id.
hipError_t launch_batch_first(const unsigned long long *argmax_part, int nparts, int V, int b, int *tokens, int *out,
                              int out_stride, hipStream_t s);

// ---- prefill -------------------------------------------------------------

hipError_t launch_embed_gather(const int *tokens, int T, int H, const uint16_t *embed_bf16, const float *embed_f32,
                               float *x, hipStream_t s);

// Row-wise RMSNorm with the batch association v*(inv*w) (or, with
// decode_assoc, forward_token's (v*inv)*w), written as split-bf16 hi/lo
// operands for the MFMA GEMM.
hipError_t launch_rmsnorm_split(const float *x, const float *w, float eps, int T, int H, uint16_t *hi, uint16_t *lo,
                                hipStream_t s, bool decode_assoc = false);

enum GemmEpi { GEPI_STORE = 0, GEPI_RESID = 1, GEPI_SWIGLU = 2, GEPI_QKV = 3 };

struct GemmArgs {
    const uint16_t *W;  // [M, K] BF16
    const float *Wf;    // [M, K] f32 weights instead (WMat::F32), or null
    const float *wscale;  // [M] row scales applied before the epilogue (int8 weights held as BF16 codes), or null
    const uint16_t *Bhi, *Blo;  // [N, K] split-bf16 activations
    int M, N, K;
    // epilogues
    float *y;  // STORE: [N][M]; RESID: [N][M] +=
    uint16_t *h_hi, *h_lo;  // SWIGLU: [N][M/2]
    // QKV
    const float *rope_cos, *rope_sin;
    int start;  // position of token 0
    int hd, nq, nkv;
    float *q_out;  // [N][nq*hd]
    float *k_cache, *v_cache;
    // several sequences at once (batched decode): token n is sequence n at
    // position pos_seq[n], its K/V rows go to k_seq[n] / v_seq[n] +
    // kv_layer_off; null pos_seq: one sequence, token n at start + n
    const int *pos_seq;
    float *const *k_seq;
    float *const *v_seq;
    size_t kv_layer_off;
    // RMSNorm handed from one GEMM to the next (prefill; kernels whose output
    // goes through stage_epilogue, see gemm_stages_output).  Producer (RESID,
    // M a multiple of 64): with nrm_w set it also writes the new residual
    // rows times nrm_w as split-bf16 planes nx_hi / nx_lo [N][M] and, per
    // token n and 64-row group g, the rows' sum of squares to
    // nss[n * (M / 64) + g].  Consumer: with nss_in set (ngroups = K / 64, a
    // multiple of 4 up to kMaxNormGroups) it scales its output by
    // 1 / sqrt(sum of token n's partials in group order / K + nrm_eps) before
    // the epilogue, so that its operand needs no separate normalization.
    const float *nrm_w;
    float *nss;
    uint16_t *nx_hi, *nx_lo;
    const float *nss_in;
    int ngroups;
    float nrm_eps;
    // split-K workspace of the short-prompt kernel: partial tiles and one
    // arrival counter per quarter tile (zero between launches; each launch
    // leaves them zero).  Null disables split-K.
    float *part;
    unsigned *cnt;
};

// Prompts of at least kTiledMinTokens tokens (and K a multiple of 64) use the
// LDS-tiled 128x128 kernel; shorter ones the 64x64 split-K kernel (K a
// multiple of 64) or the 16x64 streaming kernel.
constexpr int kTiledMinTokens = 256;
hipError_t launch_gemm(int epi, const GemmArgs &a, hipStream_t s);
// Whether launch_gemm takes a kernel whose output goes through
// stage_epilogue for these shapes (the only ones that honour nrm_w / nss_in).
bool gemm_stages_output(int M, int N, int K);
constexpr int kMaxNormGroups = 40;  // hidden sizes up to 2560 for the norm hand-off
// Workspace the short-prompt kernel needs: floats of partials and counters
// for any GEMM with at most `max_m` rows and fewer than kTiledMinTokens tokens.
constexpr size_t kSkinnyPartFloats = (size_t)768 * 64 * 64;
inline size_t skinny_counters(int max_m) { return (size_t)((max_m + 63) / 64) * ((kTiledMinTokens + 63) / 64) * 4; }

// Copy row `row` of x[T,H] to dst[H] (last prefill row -> decode residual).
hipError_t launch_copy_row(const float *x, int row, int H, float *dst, hipStream_t s);

// ---- step floor (measurement only) ------------------------------------------

// One streaming phase: nwg workgroups of 256 threads, each reading
// nchunk x nb (1..32) 4-KiB blocks of w from w + b * nchunk * nb * 4 KiB and
// dotting them with act[0..2047] (the previous phase's output); out[b] per
// workgroup (out holds at least max(nwg, 2048) floats).
hipError_t launch_stream_phase(const void *w, int nwg, int nb, int nchunk, const float *act, float *out,
                               hipStream_t s);
// nwg workgroups of 256 threads that do nothing.
hipError_t launch_empty(int nwg, hipStream_t s);

// ---- decode attention -------------------------------------------------------

// Decode attention with at most this many splits is merged in the o_proj
// GEMV prologue; with more, by attn_combine_kernel.
constexpr int kFusedSplits = 8;
// Decode attention deals the context to its splits in blocks of positions,
// round robin (split s takes blocks s, s + nsplit, ...); a block is one chunk
// of the kernel's lane geometry.  Caches of at most kShortAttnCache rows use
// blocks of about kAttnBlockShort positions over at most kFusedSplits
// splits (more, smaller workgroups at short contexts, merged in the o_proj
// prologue); longer caches use kAttnBlockLong.
constexpr int kAttnBlockLong = 64;
constexpr int kAttnBlockShort = 16;
constexpr int kShortAttnCache = 512;
constexpr int kAttnThreads = 256;  // workgroup size of the decode attention (except the 512-thread long form)
// Positions per chunk of the decode attention's lane geometry for head_dim
// hd, `group` query heads per KV head, nt threads, a requested chunk width
// chw: TS = hd / (4 VPL) lanes per position (VPL float4s of K and of V per
// lane), NTEAM = nt / TS teams, J = max(1, chw / NTEAM) positions per team.
__host__ __device__ constexpr int attn_vpl(int hd, int group) { return (hd >= 128 && group <= 2) ? 2 : 1; }
__host__ __device__ constexpr int attn_nteam(int hd, int group, int nt) { return nt / (hd / (4 * attn_vpl(hd, group))); }
__host__ __device__ constexpr int attn_chunk(int hd, int group, int nt, int chw) {
    return attn_nteam(hd, group, nt) * (chw > attn_nteam(hd, group, nt) ? chw / attn_nteam(hd, group, nt) : 1);
}
// Splits below this index load their first block before reading the
// position (speculatively: most of them are active at any context); the
// others read it first, so a long cache at a short context does not stream
// the blocks of its inactive splits.
constexpr int kSpecSplits = 8;

// ---- sampling --------------------------------------------------------------

// Largest top_k the device sampler supports, and the per-workgroup slice of
// the vocabulary the first pass sorts.
constexpr int kSampleMaxK = 64;
constexpr int kSampleSlice = 2048;
// Candidates the second sampling pass holds (16 per thread of 512): slices x
// kSampleMaxK may not exceed it, i.e. vocabularies up to 262144 ids.
constexpr int kSampleSelectKeys = 8192;
// Largest vocabulary either sampling path takes.
constexpr int kSampleMaxVocab = 262144;
// The whole-vocabulary sampler's radix sort: kRadixBlock keys per block
// (at most 256 blocks), the offsets scanned by kRadixScanThreads threads.
constexpr int kRadixBlock = 1024;
constexpr int kRadixScanThreads = 1024;
constexpr size_t kSampleRadixCounts = 256 * (kSampleMaxVocab / kRadixBlock);
// The running sums' metadata: per 1024-term chunk (256 chunks) 152 bytes,
// per 64-term group and binade (2 x 4096) 16 bytes.
constexpr size_t kSampleChainChunkBytes = 256 * 152;
constexpr size_t kSampleChainGroupBytes = 2 * 4096 * 16;
// Scratch bytes of the whole-vocabulary sampler for a vocabulary of V ids:
// scaled logits and probabilities [V] f32, 128 partial maxima, 4 running-sum
// results of 16 bytes, two sort key buffers [V] u64, the radix counts and
// the running sums' metadata.
constexpr size_t kSampleScratchBytes(size_t V) {
    return V * 8 + 576 + V * 16 + kSampleRadixCounts * 4 + kSampleChainChunkBytes + kSampleChainGroupBytes;
}

struct SampleArgs {
    float *logits;  // [V]; penalized in place like the reference
    int V;
    DevState *st;
    const unsigned *seen;  // bitmap of generated ids (repetition penalty)
    unsigned *seen_rw;     // same bitmap, updated with the chosen id
    unsigned long long *cand;  // [nslices][kSampleMaxK] packed (value, id) keys; null selects the full-vocabulary path
    int *history;
    int hist_cap;
    int greedy;       // temperature <= 0: argmax of the penalized logits
    int advance_pos;  // 1 after a decode step, 0 after prefill
    // whole-vocabulary path (cand null, not greedy): kSampleScratchBytes(V)
    // of zero-initialized device memory (scaled logits, probabilities,
    // partials, a 4096-bin histogram, search states), and whether the
    // running generate call uses top-k (top_k > kSampleMaxK here) and a
    // nucleus cut
    float *scratch;
    int use_k, use_p;
    // uniform draw of each step (the reference's StdRng stream), indexed by
    // st->step; steps at or past n_draws use 0
    const float *draws;
    int n_draws;
};

hipError_t launch_sample(const SampleArgs &a, hipStream_t s);

}  // namespace tmg
