/*
 * tmg.h -- C ABI of the MI355X (gfx950) TinyMiniGo decode path.
 *
 * This is the drop-in boundary for the reference crate's public model API
 * (reference src/lib.rs:1-6).  A Rust `extern "C"` block can bind every
 * entry point one-to-one, with the structs below mirrored as #[repr(C)].
 *
 * Conventions
 *  - Every function returns an int status (TMG_OK == 0, negative = error
 *    class) unless it is a free/getter; tmg_last_error() gives the context
 *    string of the last failure on the calling thread, mirroring the
 *    reference's anyhow context strings.
 *  - Host pointers are caller-owned.  Model weights and KV caches live in HBM
 *    for the lifetime of their handles.
 *  - One model handle is used by one host thread at a time (the reference's
 *    forward_* take &mut self).  Each model owns one HIP stream.
 */
#ifndef TMG_H
#define TMG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define TMG_OK 0
#define TMG_E_INVALID (-1)  /* bad argument, shape mismatch, token out of range */
#define TMG_E_IO (-2)       /* file open / read / mmap failure */
#define TMG_E_FORMAT (-3)   /* malformed safetensors header or JSON */
#define TMG_E_MISSING (-4)  /* missing tensor, config field or config.json */
#define TMG_E_DTYPE (-5)    /* unsupported tensor dtype */
#define TMG_E_EMPTY (-6)    /* empty prompt */
#define TMG_E_CAPACITY (-7) /* KV cache full (max_pos reached) */
#define TMG_E_DEVICE (-8)   /* HIP error or no usable GPU */
#define TMG_E_NOMEM (-9)    /* host or device allocation failed */

typedef struct tmg_model tmg_model;
typedef struct tmg_cache tmg_cache;

/* ModelConfig (reference src/config.rs:6-20). */
typedef struct tmg_config {
    uint32_t hidden_size;
    uint32_t num_hidden_layers;
    uint32_t num_attention_heads;
    uint32_t num_key_value_heads;
    uint32_t head_dim;
    uint32_t intermediate_size;
    uint32_t vocab_size;
    uint32_t bos_token_id;
    float rms_norm_eps;
    float rope_theta;
    uint32_t n_eos;               /* number of valid entries in eos_token_ids */
    uint32_t eos_token_ids[16];
    int32_t tied_lm_head;         /* 1 when lm_head.weight is absent (tied to the embedding) */
} tmg_config;

/* GenParams (reference src/model.rs:597-604). */
typedef struct tmg_gen_params {
    uint32_t max_tokens;
    float temperature;        /* <= 0: greedy argmax */
    uint32_t top_k;           /* 0: no top-k */
    float top_p;              /* >= 1: no nucleus cut */
    float repetition_penalty; /* 1.0: off */
    uint64_t seed;
} tmg_gen_params;

/* on_token callback of generate (reference src/model.rs:618, :648). */
typedef void (*tmg_on_token_fn)(uint32_t token, void *user);

/* Thread-local text of the last error (reference: anyhow context strings,
 * e.g. src/model.rs:43-47, src/config.rs:22-27). Never NULL. */
const char *tmg_last_error(void);

/* ModelConfig::load (reference src/config.rs:112-172): parse an HF
 * config.json with the reference's defaults. */
int tmg_config_load(const char *config_json_path, tmg_config *out);

/* Model::load (reference src/model.rs:384-389 -> load_model_safetensors,
 * src/model.rs:181-244): config.json must sit next to the .safetensors file
 * (src/config.rs:174-184).  BF16 weight matrices are uploaded raw to HBM on
 * `device`; F16 and F32 ones are widened to f32 rows (WMat::F32,
 * src/model.rs:49-55) and multiplied as f32 (tmg_gemv_f32's arithmetic in
 * decode, an fp32 GEMM in prefill).  Norm weights and the embedding may be
 * BF16, F16 or F32 (converted as in src/safetensors_loader.rs:103-147).  With
 * TMG_I8=1 in the environment (the reference's gate, src/model.rs:57-76) the
 * q, k, v, o, gate, up and down projections are quantized to per-row int8 at
 * load (tmg_quantize_i8, from the f32 values for F16/F32 matrices): decode
 * steps stream the int8 rows (tmg_gemv_i8's arithmetic), prefill multiplies
 * by the same codes, dequantized, in f32 (src/tensor.rs:795-858); lm_head is
 * not quantized. */
int tmg_model_load(const char *safetensors_path, int device, tmg_model **out);

/* A TMB1 file (reference src/tmb.rs) is accepted by tmg_model_load too: a
 * file that starts with "TMB1" is read as load_model_tmb does
 * (src/model.rs:90-179) -- config from the file, BF16 weight views, f32
 * embedding and norms -- and TMG_I8 does not apply to it. */

/* write_tmb (src/tmb.rs:137-262), the reference's `--repack`: converts the
 * safetensors model (config.json next to it) into a TMB1 file.  Host only. */
int tmg_tmb_repack(const char *safetensors_path, const char *tmb_path);

/* The config a TMB1 file carries (parse_tmb_header + ModelConfig::from_json,
 * src/tmb.rs:81-120, src/config.rs:37-91).  Host only.  As in the
 * reference, the EOS ids written under "eos_token_ids" are not read back
 * (from_json reads "eos_token_id"), so n_eos is 0 for files this or the
 * reference's writer produced.  tied_lm_head is 1 when the file has no
 * lm_head.weight. */
int tmg_tmb_config(const char *tmb_path, tmg_config *out);
/* Drop of Model (src/model.rs:338-347).  May be called before the model's
 * caches are freed (Rust drops struct fields in declaration order): the
 * model's device memory and stream are then released by the last
 * tmg_cache_free.  After this call the model handle itself must not be used
 * again; its caches may still be read, reset and freed.  The model and its
 * caches may be freed from different threads. */
void tmg_model_free(tmg_model *model);
int tmg_model_config(const tmg_model *model, tmg_config *out);

/* KvCache (reference src/model.rs:250-332) as a preallocated HBM slab of
 * max_pos rows per layer: f32 keys and values, [pos, n_kv*head_dim] per
 * layer, like the reference's flat per-layer Vec<f32>. */
int tmg_cache_new(tmg_model *model, uint32_t max_pos, tmg_cache **out);
void tmg_cache_free(tmg_cache *cache);
/* KvCache::len(layer) (src/model.rs:283-285). */
int tmg_cache_len(const tmg_cache *cache, uint32_t layer, uint32_t *len);
/* KvCache::reset (src/model.rs:324-331). */
int tmg_cache_reset(tmg_cache *cache);
/* KvCache::keys_flat / values_flat (src/model.rs:309-317): copy the layer's
 * [len, kv_dim] rows to host buffers (either may be NULL). */
int tmg_cache_read(const tmg_cache *cache, uint32_t layer, float *keys, float *values);

/* Model::forward_token (src/model.rs:392-491): one decode step at
 * pos = cache length; writes vocab_size logits when `logits` is non-NULL. */
int tmg_forward_token(tmg_model *model, tmg_cache *cache, uint32_t token, float *logits);

/* Model::forward_seq (src/model.rs:503-590): batched prefill from the current
 * cache length; writes the last token's logits when non-NULL. */
int tmg_forward_seq(tmg_model *model, tmg_cache *cache, const uint32_t *tokens, size_t n, float *last_logits);

/* Model::prefill (src/model.rs:494-499): forward_seq that rejects an empty
 * prompt with TMG_E_EMPTY. */
int tmg_prefill(tmg_model *model, tmg_cache *cache, const uint32_t *tokens, size_t n, float *last_logits);

/* generate (src/model.rs:614-663).  Tokens are written to out_tokens
 * (capacity out_cap >= max_tokens), their count to *n_out.  first_logits
 * (vocab_size floats) and prefill_secs may be NULL.  Sampling (temperature >
 * 0) runs on the GPU; its uniform draws are a restatement of the
 * reference's StdRng::seed_from_u64(seed) stream (tmg_stdrng_uniform), one
 * per step. */
int tmg_generate(tmg_model *model, const uint32_t *prompt, size_t n_prompt, const tmg_gen_params *params,
                 tmg_on_token_fn on_token, void *user, uint32_t *out_tokens, size_t out_cap, size_t *n_out,
                 float *first_logits, float *prefill_secs);

/* Greedy generation for n_seq independent prompts in one batch (1..128
 * sequences).  No counterpart in the reference, which decodes one sequence
 * per generate call; this is the multi-sequence batching its design notes
 * list next.  For every sequence b the ids are the ones generate
 * (src/model.rs:614-663) gives for prompts[b] alone with temperature 0 and
 * repetition penalty 1 -- stopping after an EOS id -- up to f32 rounding at
 * a near tie: each decode step streams the layer weights once for all
 * sequences (MFMA GEMM over the batch) instead of once per sequence.
 * out_tokens is [n_seq][max_tokens]; n_out[b] receives sequence b's count;
 * *decode_ms (may be NULL) the device time of the batched decode steps.
 * Models loaded with TMG_I8=1 are rejected (TMG_E_INVALID). */
int tmg_generate_batch(tmg_model *model, const uint32_t *const *prompts, const size_t *n_prompt, size_t n_seq,
                       uint32_t max_tokens, uint32_t *out_tokens, size_t *n_out, float *decode_ms);

/* The first n draws generate samples with, restating StdRng::seed_from_u64
 * (src/model.rs:629) followed by one StandardUniform f32 per call
 * (src/tensor.rs:1204): rand 0.10.2's ChaCha12 StdRng seeded through
 * rand_core's PCG32 expansion, (next_u32 >> 8) * 2^-24, as published.  The
 * crates are absent here and give no test vectors, so equality with the
 * reference's stream is unpinned.  Host only. */
int tmg_stdrng_uniform(uint64_t seed, size_t n, float *out);

/* Kernel level: y[out] = W[out,in] x[in] with W raw BF16 row-major and x, y
 * f32, all DEVICE pointers (reference tensor::matmul_w / matmul_w_into,
 * src/tensor.rs:315-338, BF16 case).  `stream` is a hipStream_t (NULL = the
 * default stream).  in must be a multiple of 8 and W 16-byte aligned. */
int tmg_gemv_bf16(const uint16_t *w_dev, const float *x_dev, float *y_dev, uint32_t out, uint32_t in,
                  void *stream);
/* The same with W f32 row-major (matmul_w_into's WMat::F32 arm,
 * src/tensor.rs:387-420: `dot` per row).  in must be a multiple of 8, W and x
 * 16-byte aligned. */
int tmg_gemv_f32(const float *w_dev, const float *x_dev, float *y_dev, uint32_t out, uint32_t in, void *stream);

/* Kernel level: tensor::argmax (src/tensor.rs:1063-1073) of x[0, n), a DEVICE
 * f32 vector, written to *out_dev (a DEVICE uint32): the index of the first
 * maximum.  NaN entries are skipped, -0.0 and +0.0 count as equal, and the
 * result is 0 when every entry is -inf or NaN or n is 0 -- the reference's
 * `v > best_val` scan from (0, -inf).  Two passes on `stream` (NULL = the
 * default stream); the per-4096-element chunk keys of the first pass live in
 * a buffer allocated and freed on that stream for the call. */
int tmg_argmax_f32(const float *x_dev, uint32_t n, uint32_t *out_dev, void *stream);

/* tmg_argmax_f32 for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  Same arguments and result; no hipMalloc,
 * hipFree or allocating call is made: the chunk keys live in a fixed 32 KiB
 * array per GPU, held until the process ends, so n is limited to
 * 16,777,216 elements (larger n: TMG_E_INVALID, nothing launched).  The
 * current device must be the stream's device.  Calls that overlap on one GPU
 * (on different streams, or from different threads) share that array and
 * race; calls in one stream order are safe. */
int tmg_argmax_f32_noalloc(const float *x_dev, uint32_t n, uint32_t *out_dev, void *stream);

/* Kernel level, int8 weight-only mode (TMG_I8=1): y[out] = the reference's
 * matmul_w_into over WMat::I8 (src/tensor.rs:341-364): x is quantized with
 * one symmetric scale (quantize_row_i8, src/tensor.rs:125-139), each row dot
 * is exact in int32 (dot_i8, src/tensor.rs:144-170) and
 * y[o] = (dot as f32) * xs * scale[o].  q [out, in] int8 codes, scale [out]
 * f32, x [in] f32, y [out] f32, all DEVICE pointers.  in must be a multiple
 * of 8 and <= 16384; q 8-byte, x 16-byte aligned. */
int tmg_gemv_i8(const int8_t *q_dev, const float *scale_dev, const float *x_dev, float *y_dev, uint32_t out,
                uint32_t in, void *stream);

/* WMat::quantize_i8 (src/tensor.rs:275-293) of BF16 rows widened to f32, as
 * wmat_maybe_i8 loads them (src/model.rs:60-68): scale[r] = max|w|/127 (1.0
 * for a zero row), q = round(w/scale) (halves away from zero) clamped to
 * [-127, 127].  w [rows, in] BF16 (read only), q [rows, in], scale [rows],
 * DEVICE pointers; in a multiple of 8; w 16-byte, q 8-byte aligned.  Models
 * loaded with TMG_I8=1 in the environment quantize their q/k/v/o/gate/up/
 * down projections this way; lm_head, norms and the embedding stay as they
 * are (src/model.rs:227-233). */
int tmg_quantize_i8(const uint16_t *w_dev, uint32_t rows, uint32_t in, int8_t *q_dev, float *scale_dev,
                    void *stream);

/* ---------------------------------------------------------------------- */
/* Measurement entry points.  No counterpart in the reference: they expose  */
/* the inner loop of generate (src/model.rs:631-656) without the host       */
/* callback, and per-kernel timing, for benchmarks.                          */
/* ---------------------------------------------------------------------- */

/* Run n_steps greedy decode steps on the device starting from `token` at the
 * current cache length (one captured step graph per step; each step is
 * forward_token followed by argmax, as in generate).  Generated ids go to
 * tokens_out (n_steps entries, may be NULL); *ms receives the elapsed time
 * between HIP events recorded on the model's stream around the steps. */
int tmg_decode_greedy(tmg_model *model, tmg_cache *cache, uint32_t token, uint32_t n_steps, uint32_t *tokens_out,
                      float *ms);

/* One launched kernel of a decode step, timed with HIP events on the model's
 * stream; bytes = algorithmic HBM bytes of that launch. */
typedef struct tmg_kernel_record {
    char name[48];     /* kernel kind, e.g. "gemv_gateup_swiglu" */
    double bytes;      /* algorithmic HBM bytes of one launch */
    float ms;          /* average duration of one launch */
    uint32_t launches; /* launches of this kind in one decode step */
} tmg_kernel_record;

/* Per-kernel timing of one decode step at the cache's current position: for
 * each kernel kind, that kind's launches of one step are captured into a graph
 * and replayed back to back between two HIP events.  One record per kind, in
 * launch order.  Leaves the cache as it was (length and contents up to len).
 * No counterpart in the reference (measurement only). */
int tmg_profile_decode_step(tmg_model *model, tmg_cache *cache, uint32_t token, tmg_kernel_record *records,
                            size_t cap, size_t *n_records);

typedef struct tmg_floor_record {
    char name[48];       /* kernel kind of the step */
    double bytes;        /* algorithmic HBM bytes of one launch of that kind */
    double floor_bytes;  /* bytes one streaming phase in its place reads */
    float floor_ms;      /* average duration of one such phase */
    uint32_t launches;   /* launches of this kind in one decode step */
    uint32_t workgroups; /* grid of the kind's launch, and of its phase */
} tmg_floor_record;

/* The decode step next to its floor, at the cache's current position.  The
 * greedy step is captured as the decode loop captures it and replayed as
 * consecutive steps (*step_ms per step).  Every launch of it is then replaced
 * by a streaming phase with the same grid that reads the launch's
 * algorithmic bytes (to whole 4-KiB blocks per workgroup, all in flight at
 * once) from a slab of its own (larger than the last-level cache) and dots
 * them with the previous phase's output: the step's launch chain and weight
 * stream with none of its other work.  *floor_ms is that
 * chain per replay, one record per kind gives its phases back to back, and
 * *empty_ms is one empty 256-workgroup launch in a graph.  Needs 9 free
 * cache rows past the length; leaves the cache as it was.  Allocates the
 * slab (about the step's bytes) for the call.  No counterpart in the
 * reference (measurement only). */
int tmg_profile_step_floor(tmg_model *model, tmg_cache *cache, uint32_t token, tmg_floor_record *records,
                           size_t cap, size_t *n_records, float *step_ms, float *floor_ms, float *empty_ms);

/* The streaming rate of the device: *us per launch of a kernel that streams
 * `bytes` (rounded up to whole workgroups; *bytes_read) of HBM-cold data as
 * workgroups of 256 threads reading wg_kib KiB each (a multiple of 4 in
 * [4, 128]), all of a workgroup's loads in flight at once, dotted with a
 * constant activation, one store per workgroup.  Launches replayed back to
 * back from a graph that rotates over more than 1 GiB of copies, timed by
 * HIP events on a stream of its own.  The floor a GEMV of that many weight
 * bytes can reach.  Allocates about 1 GiB for the call.  No counterpart in
 * the reference (measurement only). */
int tmg_profile_stream(size_t bytes, uint32_t wg_kib, int device, float *us, size_t *bytes_read);

#ifdef __cplusplus
}
#endif

#endif /* TMG_H */
