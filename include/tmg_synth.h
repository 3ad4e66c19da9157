/*
 * tmg_synth.h -- seeded synthetic models and inputs.
 *
 * No counterpart in the reference, which runs real Hugging Face checkpoints
 * (reference README.md:23-29).  These functions write safetensors models and
 * draw inputs from a documented counter-based generator so the GPU path, the
 * CPU baseline and the tests all read the same bytes.
 *
 * Generator: SplitMix64.  Stream key for tensor `name` under `seed`:
 *   key = mix64(seed * 0x9E3779B97F4A7C15 ^ fnv1a64(name))
 * value i of the stream: u_i = mix64(key + (i + 1) * 0x9E3779B97F4A7C15).
 * Normal element e uses u_{2e}, u_{2e+1}:
 *   a = ((u_{2e} >> 11) + 1) * 2^-53 in (0,1],  b = (u_{2e+1} >> 11) * 2^-53,
 *   z = sqrt(-2 ln a) * cos(2 pi b)  (double, glibc),
 *   w = (float)(stddev * z), rounded to BF16 with round-to-nearest-even.
 * Token ids: id_i = (u_i * vocab) >> 64 over the stream of name "tokens".
 */
#ifndef TMG_SYNTH_H
#define TMG_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tmg_synth_spec {
    uint32_t hidden_size;
    uint32_t num_hidden_layers;
    uint32_t num_attention_heads;
    uint32_t num_key_value_heads;
    uint32_t head_dim;
    uint32_t intermediate_size;
    uint32_t vocab_size;
    float rms_norm_eps;
    float rope_theta;
    int32_t tied_lm_head; /* 1: write no lm_head.weight */
    uint64_t seed;
    float stddev;         /* weight N(0, stddev); norm weights are 1.0 */
} tmg_synth_spec;

/* Write <dir>/model.safetensors (BF16, HF Llama tensor names) and
 * <dir>/config.json.  The config carries no eos_token_id so generation never
 * stops early.  Creates `dir` if needed. */
int tmg_synth_model(const char *dir, const tmg_synth_spec *spec);

/* n token ids uniform in [0, vocab) from `seed`. */
int tmg_synth_tokens(uint64_t seed, size_t n, uint32_t vocab, uint32_t *out);

/* n BF16 values N(0, stddev) of stream `name` under `seed` (C1 weights). */
int tmg_synth_normal_bf16(uint64_t seed, const char *name, size_t n, float stddev, uint16_t *out);

/* n f32 values N(0, stddev) of stream `name` under `seed` (C1 activations). */
int tmg_synth_normal_f32(uint64_t seed, const char *name, size_t n, float stddev, float *out);

#ifdef __cplusplus
}
#endif

#endif /* TMG_SYNTH_H */
