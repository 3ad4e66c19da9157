// TMB1 repack writer (reference write_tmb, src/tmb.rs:137-262) and the
// tmg_tmb_* C entry points.  The reader lives in io.cpp
// (SafeTensorsFile::open_tmb) so the model loader sees one interface.
//
// Layout, little-endian:
//   "TMB1" | cfg_len u64 | n_tensors u32 | config JSON (cfg_len bytes)
//   | weights_len u64 | zero pad to 8 | weights (each tensor 8-aligned,
//   zero padded, in consumption order) | index: n x (name_len u32, name,
//   file offset u64, byte length u64) | trailer: index_off u64, meta_off u64,
//   weights_len u64, file_size u64
// Consumption order: embedding (f32), per layer q, k, v, o, gate, up, down
// (raw BF16) and the two norms (f32), the final norm (f32), lm_head (raw
// BF16) when the file has one.
#include <cerrno>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>

#include "common.hpp"
#include "json.hpp"

namespace tmg {

namespace {

constexpr uint64_t kAlign = 8;  // TENSOR_ALIGN (src/tmb.rs:26)

uint64_t align_up(uint64_t n) { return (n + kAlign - 1) & ~(kAlign - 1); }

// A JSON number for an f32 config value: the f64 it widens to, in the
// shortest digits that read back to it, written the way serde_json writes
// floats (decimal notation for 1e-5 <= |v| < 1e16, else d.ddde-N).  The
// value round-trips exactly; the spelling of the reference's float
// formatter is followed, not pinned.
std::string json_f32(float f) {
    const double d = (double)f;
    if (d == 0.0) return std::signbit(d) ? "-0.0" : "0.0";
    char buf[64];
    auto r = std::to_chars(buf, buf + sizeof(buf), d, std::chars_format::scientific);
    std::string sci(buf, r.ptr);  // [-]D[.DDD]e[+-]XX
    std::string sign;
    if (sci[0] == '-') {
        sign = "-";
        sci.erase(0, 1);
    }
    const size_t e = sci.find('e');
    std::string digits;
    for (size_t i = 0; i < e; i++)
        if (sci[i] != '.') digits += sci[i];
    while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
    const int exp10 = atoi(sci.c_str() + e + 1);  // value = D.DDD x 10^exp10
    const int n = (int)digits.size();
    const int kk = exp10 + 1;  // 10^(kk-1) <= |v| < 10^kk
    const int k = kk - n;      // value = digits x 10^k
    std::string out;
    if (k >= 0 && kk <= 16) {
        out = digits + std::string(k, '0') + ".0";
    } else if (kk > 0 && kk <= 16) {
        out = digits.substr(0, kk) + "." + digits.substr(kk);
    } else if (kk > -5 && kk <= 0) {
        out = "0." + std::string(-kk, '0') + digits;
    } else if (n == 1) {
        out = digits + "e" + std::to_string(kk - 1);
    } else {
        out = digits.substr(0, 1) + "." + digits.substr(1) + "e" + std::to_string(kk - 1);
    }
    return sign + out;
}

// ModelConfig::to_json (src/config.rs:92-108) as serde_json::to_string
// writes it: compact, keys in sorted order (serde_json's default map).
// Note the key "eos_token_ids": the reader (ModelConfig::from_json) looks
// for "eos_token_id", so a TMB file carries no EOS ids back -- kept as is.
std::string config_json(const tmg_config &c) {
    std::string eos = "[";
    for (uint32_t i = 0; i < c.n_eos; i++) eos += (i ? "," : "") + std::to_string(c.eos_token_ids[i]);
    eos += "]";
    return std::string("{") + "\"bos_token_id\":" + std::to_string(c.bos_token_id) + ",\"eos_token_ids\":" + eos +
           ",\"head_dim\":" + std::to_string(c.head_dim) + ",\"hidden_size\":" + std::to_string(c.hidden_size) +
           ",\"intermediate_size\":" + std::to_string(c.intermediate_size) +
           ",\"num_attention_heads\":" + std::to_string(c.num_attention_heads) +
           ",\"num_hidden_layers\":" + std::to_string(c.num_hidden_layers) +
           ",\"num_key_value_heads\":" + std::to_string(c.num_key_value_heads) +
           ",\"rms_norm_eps\":" + json_f32(c.rms_norm_eps) + ",\"rope_theta\":" + json_f32(c.rope_theta) +
           ",\"vocab_size\":" + std::to_string(c.vocab_size) + "}";
}

struct Item {
    std::string name;
    const TensorEntry *e;
    bool f32;       // converted to f32 (embedding, norms); else raw BF16
    uint64_t off;   // file offset
    uint64_t len;   // bytes
};

struct FileCloser {
    void operator()(FILE *f) const {
        if (f) fclose(f);
    }
};

}  // namespace

int tmb_write(const std::string &src, const std::string &dst) {
    std::string cpath;
    if (!config_path_for_model(src, &cpath)) return set_error(TMG_E_MISSING, "config.json not found next to " + src);
    tmg_config cfg;
    int rc = config_load(cpath, &cfg);
    if (rc) return rc;
    SafeTensorsFile f;
    if ((rc = f.open(src))) return rc;

    std::vector<Item> items;
    auto add = [&](const std::string &name, bool f32, const std::string &missing) -> int {
        const TensorEntry *e = f.find(name);
        if (!e) return set_error(TMG_E_MISSING, missing);
        if (f32) {
            if (e->dtype == DType::Other)
                return set_error(TMG_E_DTYPE, "unsupported dtype " + e->dtype_name + " for tensor " + name);
        } else if (e->dtype != DType::BF16) {
            // the reference panics here (bf16_bytes on a non-BF16 tensor)
            return set_error(TMG_E_DTYPE, "tensor " + name + " is " + e->dtype_name + ": TMB stores BF16 weights");
        }
        items.push_back({name, e, f32, 0, e->numel() * (f32 ? 4 : 2)});
        return TMG_OK;
    };
    if ((rc = add("model.embed_tokens.weight", true, "missing embed_tokens.weight"))) return rc;
    static const char *kLayer[] = {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                                   "self_attn.o_proj.weight", "mlp.gate_proj.weight",    "mlp.up_proj.weight",
                                   "mlp.down_proj.weight",    "input_layernorm.weight",  "post_attention_layernorm.weight"};
    for (uint32_t l = 0; l < cfg.num_hidden_layers; l++)
        for (int j = 0; j < 9; j++) {
            const std::string full = "model.layers." + std::to_string(l) + "." + kLayer[j];
            if ((rc = add(full, j >= 7, "missing " + full))) return rc;
        }
    if ((rc = add("model.norm.weight", true, "missing model.norm.weight"))) return rc;
    if (f.find("lm_head.weight") && (rc = add("lm_head.weight", false, ""))) return rc;

    const std::string cj = config_json(cfg);
    const uint64_t wlen_field = 16 + cj.size();
    const uint64_t weights_off = align_up(wlen_field + 8);
    uint64_t rel = 0;
    for (auto &it : items) {
        rel = align_up(rel);
        it.off = weights_off + rel;
        rel += it.len;
    }
    const uint64_t weights_len = rel;

    std::unique_ptr<FILE, FileCloser> out(fopen(dst.c_str(), "wb"));
    if (!out) return set_error(TMG_E_IO, "creating " + dst + ": " + strerror(errno));
    FILE *fp = out.get();
    bool ok = true;
    auto put = [&](const void *p, size_t n) {
        if (ok && n && fwrite(p, 1, n, fp) != n) ok = false;
    };
    auto put64 = [&](uint64_t v) { put(&v, 8); };
    auto zeros = [&](uint64_t n) {
        static const char z[kAlign] = {0};
        while (n) {
            const uint64_t c = n < kAlign ? n : kAlign;
            put(z, c);
            n -= c;
        }
    };
    const uint32_t nt = (uint32_t)items.size();
    put("TMB1", 4);
    put64(cj.size());
    put(&nt, 4);
    put(cj.data(), cj.size());
    put64(weights_len);
    zeros(weights_off - (wlen_field + 8));
    uint64_t at = weights_off;
    std::vector<float> conv;
    for (const auto &it : items) {
        zeros(it.off - at);
        if (it.f32) {
            if ((rc = tensor_to_f32(f, *it.e, &conv))) return rc;
            put(conv.data(), conv.size() * 4);
        } else {
            put(f.data(*it.e), it.len);
        }
        at = it.off + it.len;
    }
    const uint64_t index_off = weights_off + weights_len;
    uint64_t index_len = 0;
    for (const auto &it : items) {
        const uint32_t nl = (uint32_t)it.name.size();
        put(&nl, 4);
        put(it.name.data(), nl);
        put64(it.off);
        put64(it.len);
        index_len += 4 + nl + 16;
    }
    const uint64_t meta_off = index_off + index_len;
    put64(index_off);
    put64(meta_off);
    put64(weights_len);
    put64(meta_off + 32);
    if (!ok || fflush(fp) != 0) return set_error(TMG_E_IO, "writing " + dst + ": " + strerror(errno));
    return TMG_OK;
}

}  // namespace tmg

extern "C" int tmg_tmb_repack(const char *safetensors_path, const char *tmb_path) {
    tmg::clear_error();
    if (!safetensors_path || !tmb_path) return tmg::set_error(TMG_E_INVALID, "null argument");
    return tmg::tmb_write(safetensors_path, tmb_path);
}

extern "C" int tmg_tmb_config(const char *tmb_path, tmg_config *out) {
    tmg::clear_error();
    if (!tmb_path || !out) return tmg::set_error(TMG_E_INVALID, "null argument");
    tmg::SafeTensorsFile f;
    tmg_config c;
    memset(&c, 0, sizeof(c));
    int rc = f.open_tmb(tmb_path, &c);
    if (rc) return rc;
    c.tied_lm_head = f.find("lm_head.weight") ? 0 : 1;
    *out = c;
    return TMG_OK;
}
