// Seeded synthetic models and inputs (generator documented in tmg_synth.h).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "../../../include/tmg_synth.h"
#include "common.hpp"

namespace tmg {
namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t fnv1a64(const std::string &s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 0x100000001b3ull;
    }
    return h;
}

inline uint64_t stream_key(uint64_t seed, const std::string &name) { return mix64((seed * kGamma) ^ fnv1a64(name)); }
inline uint64_t stream_u64(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * kGamma); }

inline double normal_at(uint64_t key, uint64_t e) {
    double a = (double)((stream_u64(key, 2 * e) >> 11) + 1) * 0x1.0p-53;
    double b = (double)(stream_u64(key, 2 * e + 1) >> 11) * 0x1.0p-53;
    return sqrt(-2.0 * log(a)) * cos(2.0 * M_PI * b);
}

inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;  // NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

unsigned worker_count() {
    unsigned n = std::thread::hardware_concurrency();
    if (n == 0) n = 1;
    return std::min(n, 16u);
}

template <class F>
void parallel_range(uint64_t n, F &&fn) {
    unsigned nt = worker_count();
    if (n < (1u << 16) || nt == 1) {
        fn(0, n);
        return;
    }
    std::vector<std::thread> th;
    uint64_t per = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; t++) {
        uint64_t b = (uint64_t)t * per, e = std::min(n, b + per);
        if (b >= e) break;
        th.emplace_back([&fn, b, e] { fn(b, e); });
    }
    for (auto &t : th) t.join();
}

void fill_normal_bf16(uint64_t seed, const std::string &name, uint64_t n, float stddev, uint16_t *out) {
    uint64_t key = stream_key(seed, name);
    parallel_range(n, [&](uint64_t b, uint64_t e) {
        for (uint64_t i = b; i < e; i++) out[i] = f32_to_bf16_rne((float)((double)stddev * normal_at(key, i)));
    });
}

struct SynthTensor {
    std::string name;
    std::vector<uint64_t> shape;
    bool ones;  // norm weight: all 1.0
    uint64_t numel() const {
        uint64_t n = 1;
        for (auto d : shape) n *= d;
        return n;
    }
};

std::string fmt_float(float f) {
    char buf[64];
    snprintf(buf, sizeof(buf), "%.9g", (double)f);
    std::string s(buf);
    if (s.find_first_of(".eEn") == std::string::npos) s += ".0";
    return s;
}

}  // namespace
}  // namespace tmg

using namespace tmg;

extern "C" int tmg_synth_tokens(uint64_t seed, size_t n, uint32_t vocab, uint32_t *out) {
    if ((!out && n) || vocab == 0) return set_error(TMG_E_INVALID, "tmg_synth_tokens: bad argument");
    uint64_t key = stream_key(seed, "tokens");
    for (size_t i = 0; i < n; i++) out[i] = (uint32_t)(((unsigned __int128)stream_u64(key, i) * vocab) >> 64);
    return TMG_OK;
}

extern "C" int tmg_synth_normal_bf16(uint64_t seed, const char *name, size_t n, float stddev, uint16_t *out) {
    if (!name || (!out && n)) return set_error(TMG_E_INVALID, "tmg_synth_normal_bf16: bad argument");
    fill_normal_bf16(seed, name, n, stddev, out);
    return TMG_OK;
}

extern "C" int tmg_synth_normal_f32(uint64_t seed, const char *name, size_t n, float stddev, float *out) {
    if (!name || (!out && n)) return set_error(TMG_E_INVALID, "tmg_synth_normal_f32: bad argument");
    uint64_t key = stream_key(seed, name);
    parallel_range(n, [&](uint64_t b, uint64_t e) {
        for (uint64_t i = b; i < e; i++) out[i] = (float)((double)stddev * normal_at(key, i));
    });
    return TMG_OK;
}

extern "C" int tmg_synth_model(const char *dir, const tmg_synth_spec *s) {
    if (!dir || !s) return set_error(TMG_E_INVALID, "tmg_synth_model: null argument");
    if (!s->hidden_size || !s->num_hidden_layers || !s->num_attention_heads || !s->num_key_value_heads ||
        !s->head_dim || !s->intermediate_size || !s->vocab_size)
        return set_error(TMG_E_INVALID, "tmg_synth_model: zero dimension");
    mkdir(dir, 0755);
    const uint64_t H = s->hidden_size, I = s->intermediate_size, V = s->vocab_size;
    const uint64_t qd = (uint64_t)s->num_attention_heads * s->head_dim;
    const uint64_t kvd = (uint64_t)s->num_key_value_heads * s->head_dim;

    std::vector<SynthTensor> ts;
    ts.push_back({"model.embed_tokens.weight", {V, H}, false});
    for (uint32_t l = 0; l < s->num_hidden_layers; l++) {
        std::string p = "model.layers." + std::to_string(l) + ".";
        ts.push_back({p + "self_attn.q_proj.weight", {qd, H}, false});
        ts.push_back({p + "self_attn.k_proj.weight", {kvd, H}, false});
        ts.push_back({p + "self_attn.v_proj.weight", {kvd, H}, false});
        ts.push_back({p + "self_attn.o_proj.weight", {H, qd}, false});
        ts.push_back({p + "mlp.gate_proj.weight", {I, H}, false});
        ts.push_back({p + "mlp.up_proj.weight", {I, H}, false});
        ts.push_back({p + "mlp.down_proj.weight", {H, I}, false});
        ts.push_back({p + "input_layernorm.weight", {H}, true});
        ts.push_back({p + "post_attention_layernorm.weight", {H}, true});
    }
    ts.push_back({"model.norm.weight", {H}, true});
    if (!s->tied_lm_head) ts.push_back({"lm_head.weight", {V, H}, false});
    std::sort(ts.begin(), ts.end(), [](const SynthTensor &a, const SynthTensor &b) { return a.name < b.name; });

    std::string hdr = "{\"__metadata__\":{\"format\":\"pt\"}";
    std::vector<uint64_t> offs;
    uint64_t off = 0;
    for (const auto &t : ts) {
        uint64_t bytes = t.numel() * 2;
        hdr += ",\"" + t.name + "\":{\"dtype\":\"BF16\",\"shape\":[";
        for (size_t i = 0; i < t.shape.size(); i++) hdr += (i ? "," : "") + std::to_string(t.shape[i]);
        hdr += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + bytes) + "]}";
        offs.push_back(off);
        off += bytes;
    }
    hdr += "}";
    while ((8 + hdr.size()) % 8) hdr += ' ';
    const uint64_t total = 8 + hdr.size() + off;

    std::string path = std::string(dir) + "/model.safetensors";
    std::string tmp = path + ".tmp";
    int fd = ::open(tmp.c_str(), O_RDWR | O_CREAT | O_TRUNC, 0644);
    if (fd < 0) return set_error(TMG_E_IO, "creating " + tmp + ": " + strerror(errno));
    if (ftruncate(fd, (off_t)total) != 0) {
        ::close(fd);
        return set_error(TMG_E_IO, "sizing " + tmp + ": " + strerror(errno));
    }
    void *m = mmap(nullptr, total, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) return set_error(TMG_E_IO, "mmapping " + tmp + ": " + strerror(errno));
    uint8_t *base = (uint8_t *)m;
    uint64_t n = hdr.size();
    memcpy(base, &n, 8);
    memcpy(base + 8, hdr.data(), hdr.size());
    uint8_t *data = base + 8 + hdr.size();
    for (size_t i = 0; i < ts.size(); i++) {
        uint16_t *dst = (uint16_t *)(data + offs[i]);
        if (ts[i].ones) {
            for (uint64_t k = 0; k < ts[i].numel(); k++) dst[k] = 0x3f80;
        } else {
            fill_normal_bf16(s->seed, ts[i].name, ts[i].numel(), s->stddev, dst);
        }
    }
    munmap(m, total);
    if (rename(tmp.c_str(), path.c_str()) != 0) return set_error(TMG_E_IO, "renaming " + tmp);

    std::string cfg = "{\n  \"architectures\": [\"LlamaForCausalLM\"],\n  \"model_type\": \"llama\",\n";
    cfg += "  \"hidden_size\": " + std::to_string(H) + ",\n";
    cfg += "  \"num_hidden_layers\": " + std::to_string(s->num_hidden_layers) + ",\n";
    cfg += "  \"num_attention_heads\": " + std::to_string(s->num_attention_heads) + ",\n";
    cfg += "  \"num_key_value_heads\": " + std::to_string(s->num_key_value_heads) + ",\n";
    cfg += "  \"head_dim\": " + std::to_string(s->head_dim) + ",\n";
    cfg += "  \"intermediate_size\": " + std::to_string(I) + ",\n";
    cfg += "  \"vocab_size\": " + std::to_string(V) + ",\n";
    cfg += "  \"rms_norm_eps\": " + fmt_float(s->rms_norm_eps) + ",\n";
    cfg += "  \"rope_theta\": " + fmt_float(s->rope_theta) + ",\n";
    cfg += "  \"bos_token_id\": 0,\n";
    cfg += std::string("  \"tie_word_embeddings\": ") + (s->tied_lm_head ? "true" : "false") + "\n}\n";
    std::string cpath = std::string(dir) + "/config.json";
    FILE *f = fopen(cpath.c_str(), "w");
    if (!f) return set_error(TMG_E_IO, "writing " + cpath);
    fwrite(cfg.data(), 1, cfg.size(), f);
    fclose(f);
    return TMG_OK;
}
