// Error state, safetensors reader and config loader.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <fstream>
#include <sstream>

#include "common.hpp"
#include "json.hpp"

namespace tmg {

static thread_local std::string g_last_error;

int set_error(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

void clear_error() { g_last_error.clear(); }

}  // namespace tmg

extern "C" const char *tmg_last_error(void) { return tmg::g_last_error.c_str(); }

namespace tmg {

// ---------------------------------------------------------------------------
// safetensors
// ---------------------------------------------------------------------------

SafeTensorsFile::~SafeTensorsFile() {
    if (base_) munmap(base_, size_);
}

static DType parse_dtype(const std::string &s) {
    if (s == "BF16") return DType::BF16;
    if (s == "F16") return DType::F16;
    if (s == "F32") return DType::F32;
    return DType::Other;
}

static uint64_t dtype_size(const std::string &s) {
    if (s == "BF16" || s == "F16" || s == "I16" || s == "U16") return 2;
    if (s == "F32" || s == "I32" || s == "U32") return 4;
    if (s == "F64" || s == "I64" || s == "U64") return 8;
    if (s == "I8" || s == "U8" || s == "BOOL" || s == "F8_E4M3" || s == "F8_E5M2") return 1;
    return 0;
}

int SafeTensorsFile::map_file(const std::string &path) {
    path_ = path;
    int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) return set_error(TMG_E_IO, "opening " + path + ": " + strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        return set_error(TMG_E_IO, "stat " + path + ": " + strerror(errno));
    }
    size_ = (size_t)st.st_size;
    if (size_ == 0) {
        ::close(fd);
        return TMG_OK;
    }
    void *m = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE | MAP_POPULATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) return set_error(TMG_E_IO, "mmapping " + path + ": " + strerror(errno));
    base_ = (uint8_t *)m;
    return TMG_OK;
}

int SafeTensorsFile::open(const std::string &path) {
    int rc = map_file(path);
    if (rc) return rc;
    if (size_ < 8) return set_error(TMG_E_FORMAT, "safetensors file too small: " + path);
    uint64_t n;
    memcpy(&n, base_, 8);  // little-endian header length
    if (n > size_ - 8) return set_error(TMG_E_FORMAT, "safetensors header truncated: " + path);
    JsonValue hdr;
    std::string err;
    if (!json_parse((const char *)base_ + 8, (size_t)n, &hdr, &err) || hdr.kind != JsonValue::Object)
        return set_error(TMG_E_FORMAT, "invalid safetensors header JSON in " + path + ": " + err);
    data_off_ = 8 + n;
    uint64_t data_len = size_ - data_off_;
    for (const auto &kv : hdr.obj) {
        if (kv.first == "__metadata__") continue;
        const JsonValue &t = kv.second;
        const JsonValue *dt = t.get("dtype"), *sh = t.get("shape"), *off = t.get("data_offsets");
        if (!dt || dt->kind != JsonValue::String || !sh || sh->kind != JsonValue::Array || !off ||
            off->kind != JsonValue::Array || off->arr.size() != 2)
            return set_error(TMG_E_FORMAT, "malformed safetensors entry `" + kv.first + "` in " + path);
        TensorEntry e;
        e.name = kv.first;
        e.dtype_name = dt->str;
        e.dtype = parse_dtype(dt->str);
        for (const auto &d : sh->arr) {
            unsigned long long u;
            if (!d.as_u64(&u)) return set_error(TMG_E_FORMAT, "bad shape for `" + kv.first + "`");
            e.shape.push_back(u);
        }
        unsigned long long b, en;
        if (!off->arr[0].as_u64(&b) || !off->arr[1].as_u64(&en) || b > en || en > data_len)
            return set_error(TMG_E_FORMAT, "bad data_offsets for `" + kv.first + "` in " + path);
        e.begin = b;
        e.end = en;
        uint64_t es = dtype_size(e.dtype_name);
        if (es && e.numel() * es != en - b)
            return set_error(TMG_E_FORMAT, "byte length of `" + kv.first + "` does not match its shape");
        index_[e.name] = entries_.size();
        entries_.push_back(std::move(e));
    }
    return TMG_OK;
}

// parse_tmb_header (src/tmb.rs:81-120) with every read bounds-checked: the
// reference slices the map and panics on a short file; here that is a
// format error.  Tensor ranges are checked up front, where the reference
// checks them when a tensor is first borrowed.
static bool tmb_is_bf16(const std::string &name) {
    auto ends = [&](const char *suf) {
        size_t n = strlen(suf);
        return name.size() >= n && name.compare(name.size() - n, n, suf) == 0;
    };
    return ends("_proj.weight") || name == "lm_head.weight";
}

int SafeTensorsFile::open_tmb(const std::string &path, tmg_config *cfg) {
    int rc = map_file(path);
    if (rc) return rc;
    const std::string where = " in " + path;
    if (size_ < 16) return set_error(TMG_E_FORMAT, "TMB file too small" + where);
    if (memcmp(base_, "TMB1", 4) != 0) return set_error(TMG_E_FORMAT, "not a TMB1 file (wrong magic)" + where);
    uint64_t cfg_len;
    uint32_t n;
    memcpy(&cfg_len, base_ + 4, 8);
    memcpy(&n, base_ + 12, 4);
    uint64_t pos = 16;
    if (cfg_len > size_ - pos) return set_error(TMG_E_FORMAT, "TMB config extends past the end of the file" + where);
    JsonValue cj;
    std::string err;
    if (!json_parse((const char *)base_ + pos, (size_t)cfg_len, &cj, &err))
        return set_error(TMG_E_FORMAT, "TMB config JSON: " + err + where);
    pos += cfg_len;
    if (size_ - pos < 8) return set_error(TMG_E_FORMAT, "TMB weights length missing" + where);
    uint64_t weights_len;
    memcpy(&weights_len, base_ + pos, 8);
    const uint64_t weights_off = (pos + 8 + 7) & ~(uint64_t)7;
    if (weights_off > size_ || weights_len > size_ - weights_off)
        return set_error(TMG_E_FORMAT, "TMB weights section extends past the end of the file" + where);
    pos = weights_off + weights_len;
    entries_.clear();
    index_.clear();
    for (uint32_t i = 0; i < n; i++) {
        uint32_t name_len;
        if (size_ - pos < 4) return set_error(TMG_E_FORMAT, "TMB index truncated" + where);
        memcpy(&name_len, base_ + pos, 4);
        pos += 4;
        if (size_ - pos < (uint64_t)name_len + 16) return set_error(TMG_E_FORMAT, "TMB index truncated" + where);
        TensorEntry e;
        e.name.assign((const char *)base_ + pos, name_len);
        pos += name_len;
        uint64_t off, len;
        memcpy(&off, base_ + pos, 8);
        memcpy(&len, base_ + pos + 8, 8);
        pos += 16;
        if (off > size_ || len > size_ - off)
            return set_error(TMG_E_FORMAT, "TMB tensor range out of bounds: `" + e.name + "`" + where);
        const bool bf = tmb_is_bf16(e.name);
        if (len % (bf ? 2 : 4))
            return set_error(TMG_E_FORMAT, std::string(bf ? "TMB BF16 tensor has odd byte length"
                                                          : "TMB f32 tensor has non-multiple-of-4 byte length") +
                                               ": `" + e.name + "`" + where);
        e.dtype = bf ? DType::BF16 : DType::F32;
        e.dtype_name = bf ? "BF16" : "F32";
        e.shape = {len / (bf ? 2 : 4)};
        e.begin = off;  // data section = the whole file
        e.end = off + len;
        auto it = index_.find(e.name);  // a repeated name: the later entry wins, as in a HashMap
        if (it != index_.end()) {
            entries_[it->second] = std::move(e);
        } else {
            index_[e.name] = entries_.size();
            entries_.push_back(std::move(e));
        }
    }
    data_off_ = 0;
    if (cj.kind != JsonValue::Object)
        return set_error(TMG_E_MISSING, "config missing integer field `hidden_size`");
    return config_from_json(cj, cfg);
}

bool is_tmb(const std::string &path) {
    std::ifstream in(path, std::ios::binary);
    char m[4];
    return in && in.read(m, 4) && memcmp(m, "TMB1", 4) == 0;
}

const TensorEntry *SafeTensorsFile::find(const std::string &name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &entries_[it->second];
}

float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t frac = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (frac == 0) {
            bits = sign;
        } else {
            uint32_t e = 127 - 1;
            uint32_t f = frac;
            while ((f & 0x400) == 0) {
                f <<= 1;
                e -= 1;
            }
            f &= 0x3ff;
            // Kept exactly as the reference writes it: the exponent starts at
            // 126, which scales f16 subnormals by 2^13 relative to IEEE.  A
            // drop-in must read the same values from the same file.
            bits = sign | (e << 23) | (f << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (frac << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (frac << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

int tensor_to_f32(const SafeTensorsFile &f, const TensorEntry &e, std::vector<float> *out) {
    size_t n = (size_t)e.numel();
    out->resize(n);
    const uint8_t *p = f.data(e);
    switch (e.dtype) {
        case DType::F32: memcpy(out->data(), p, n * 4); break;
        case DType::BF16:
            for (size_t i = 0; i < n; i++) {
                uint16_t b;
                memcpy(&b, p + 2 * i, 2);
                uint32_t u = (uint32_t)b << 16;
                memcpy(&(*out)[i], &u, 4);
            }
            break;
        case DType::F16:
            for (size_t i = 0; i < n; i++) {
                uint16_t h;
                memcpy(&h, p + 2 * i, 2);
                (*out)[i] = f16_to_f32(h);
            }
            break;
        default:
            return set_error(TMG_E_DTYPE, "unsupported dtype " + e.dtype_name + " for tensor " + e.name);
    }
    return TMG_OK;
}

// ---------------------------------------------------------------------------
// config.json
// ---------------------------------------------------------------------------

static int need_usize(const JsonValue &cfg, const char *key, uint32_t *out) {
    const JsonValue *v = cfg.get(key);
    unsigned long long u;
    if (!v || !v->as_u64(&u) || u > 0xFFFFFFFFull)
        return set_error(TMG_E_MISSING, std::string("config missing integer field `") + key + "`");
    *out = (uint32_t)u;
    return TMG_OK;
}

int config_load(const std::string &path, tmg_config *out) {
    std::ifstream in(path, std::ios::binary);
    if (!in) return set_error(TMG_E_IO, "reading config " + path);
    std::stringstream ss;
    ss << in.rdbuf();
    std::string text = ss.str();
    JsonValue cfg;
    std::string err;
    if (!json_parse(text.data(), text.size(), &cfg, &err) || cfg.kind != JsonValue::Object)
        return set_error(TMG_E_FORMAT, "parsing " + path + ": " + err);
    return config_from_json(cfg, out);
}

// ModelConfig::load's field rules (src/config.rs:112-172), which
// ModelConfig::from_json repeats for the config a TMB file embeds
// (src/config.rs:37-91).
int config_from_json(const JsonValue &cfg, tmg_config *out) {
    tmg_config c;
    memset(&c, 0, sizeof(c));
    int rc;
    if ((rc = need_usize(cfg, "hidden_size", &c.hidden_size))) return rc;
    if ((rc = need_usize(cfg, "num_attention_heads", &c.num_attention_heads))) return rc;
    unsigned long long u;
    const JsonValue *v = cfg.get("num_key_value_heads");
    c.num_key_value_heads = (v && v->as_u64(&u)) ? (uint32_t)u : c.num_attention_heads;
    v = cfg.get("head_dim");
    if (v && v->as_u64(&u)) {
        c.head_dim = (uint32_t)u;
    } else {
        if (c.num_attention_heads == 0) return set_error(TMG_E_INVALID, "num_attention_heads is 0");
        c.head_dim = c.hidden_size / c.num_attention_heads;
    }
    // rope_theta: top level, else rope_parameters.rope_theta, else 10000
    double d;
    c.rope_theta = 10000.0f;
    v = cfg.get("rope_theta");
    if (v && v->as_f64(&d)) {
        c.rope_theta = (float)d;
    } else if (const JsonValue *rp = cfg.get("rope_parameters")) {
        const JsonValue *rt = rp->get("rope_theta");
        if (rt && rt->as_f64(&d)) c.rope_theta = (float)d;
    }
    // eos_token_id: a number, a list (non-integers skipped), else none
    v = cfg.get("eos_token_id");
    if (v && v->kind == JsonValue::Number) {
        if (!v->as_u64(&u)) return set_error(TMG_E_FORMAT, "bad eos_token_id");
        c.eos_token_ids[c.n_eos++] = (uint32_t)u;
    } else if (v && v->kind == JsonValue::Array) {
        for (const auto &e : v->arr)
            if (e.as_u64(&u) && c.n_eos < 16) c.eos_token_ids[c.n_eos++] = (uint32_t)u;
    }
    if ((rc = need_usize(cfg, "num_hidden_layers", &c.num_hidden_layers))) return rc;
    if ((rc = need_usize(cfg, "intermediate_size", &c.intermediate_size))) return rc;
    v = cfg.get("rms_norm_eps");
    c.rms_norm_eps = (v && v->as_f64(&d)) ? (float)d : 1e-5f;
    if ((rc = need_usize(cfg, "vocab_size", &c.vocab_size))) return rc;
    v = cfg.get("bos_token_id");
    c.bos_token_id = (v && v->as_u64(&u)) ? (uint32_t)u : 0;
    c.tied_lm_head = 0;
    *out = c;
    return TMG_OK;
}

bool config_path_for_model(const std::string &model_path, std::string *out) {
    size_t slash = model_path.find_last_of('/');
    std::string dir = slash == std::string::npos ? "." : model_path.substr(0, slash);
    if (dir.empty()) dir = "/";
    std::string p = dir + "/config.json";
    struct stat st;
    if (stat(p.c_str(), &st) != 0) return false;
    *out = p;
    return true;
}

}  // namespace tmg

extern "C" int tmg_config_load(const char *path, tmg_config *out) {
    if (!path || !out) return tmg::set_error(TMG_E_INVALID, "null argument");
    tmg::clear_error();
    return tmg::config_load(path, out);
}
