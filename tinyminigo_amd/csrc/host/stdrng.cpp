// The reference's sampling draws: generate (src/model.rs:629) seeds
// StdRng::seed_from_u64(params.seed) and sample (src/tensor.rs:1204) takes
// one StandardUniform f32 per sampled step.  StdRng and StandardUniform come
// from the crates rand 0.10.2, rand_core 0.10.1 and chacha20 0.10.2; this is
// their published algorithm:
//   seed_from_u64: 32-byte key = eight PCG32 outputs (state advanced by
//     state * 6364136223846793005 + 11634580027462260723 before each, XSH-RR
//     output of the new state), little-endian;
//   StdRng = ChaCha12: that key, 64-bit block counter from 0 (words 12-13),
//     stream 0 (words 14-15), 12 rounds, words emitted in block order;
//   StandardUniform f32: (next_u32 >> 8) * 2^-24.
// generate computes the draws of a call on the host (4 bytes per token) and
// the device sampler reads draw `step` at step `step`.
#include "common.hpp"

namespace tmg {

namespace {

inline uint32_t rotl(uint32_t x, int n) { return (x << n) | (x >> (32 - n)); }

inline void quarter(uint32_t *x, int a, int b, int c, int d) {
    x[a] += x[b];
    x[d] = rotl(x[d] ^ x[a], 16);
    x[c] += x[d];
    x[b] = rotl(x[b] ^ x[c], 12);
    x[a] += x[b];
    x[d] = rotl(x[d] ^ x[a], 8);
    x[c] += x[d];
    x[b] = rotl(x[b] ^ x[c], 7);
}

void chacha12_block(const uint32_t key[8], uint64_t counter, uint32_t out[16]) {
    uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
    for (int i = 0; i < 8; i++) s[4 + i] = key[i];
    s[12] = (uint32_t)counter;
    s[13] = (uint32_t)(counter >> 32);
    s[14] = 0;
    s[15] = 0;
    uint32_t x[16];
    for (int i = 0; i < 16; i++) x[i] = s[i];
    for (int r = 0; r < 12; r += 2) {
        quarter(x, 0, 4, 8, 12);
        quarter(x, 1, 5, 9, 13);
        quarter(x, 2, 6, 10, 14);
        quarter(x, 3, 7, 11, 15);
        quarter(x, 0, 5, 10, 15);
        quarter(x, 1, 6, 11, 12);
        quarter(x, 2, 7, 8, 13);
        quarter(x, 3, 4, 9, 14);
    }
    for (int i = 0; i < 16; i++) out[i] = x[i] + s[i];
}

}  // namespace

void stdrng_uniform(uint64_t seed, size_t n, float *out) {
    uint32_t key[8];
    uint64_t state = seed;
    for (int i = 0; i < 8; i++) {
        state = state * 6364136223846793005ull + 11634580027462260723ull;
        const uint32_t xs = (uint32_t)(((state >> 18) ^ state) >> 27);
        const unsigned rot = (unsigned)(state >> 59);
        key[i] = (xs >> rot) | (xs << ((32 - rot) & 31));
    }
    uint32_t blk[16];
    for (size_t j = 0; j < n; j++) {
        if (j % 16 == 0) chacha12_block(key, (uint64_t)(j / 16), blk);
        out[j] = (float)(blk[j % 16] >> 8) * 0x1.0p-24f;
    }
}

}  // namespace tmg

extern "C" int tmg_stdrng_uniform(uint64_t seed, size_t n, float *out) {
    tmg::clear_error();
    if (n && !out) return tmg::set_error(TMG_E_INVALID, "null argument");
    tmg::stdrng_uniform(seed, n, out);
    return TMG_OK;
}
