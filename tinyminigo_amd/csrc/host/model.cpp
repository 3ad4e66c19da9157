// Model load, KV cache, decode step (captured as a hipGraph), prefill and
// the C ABI entry points of tmg.h.
#include "model.hpp"

#include <chrono>
#include <algorithm>
#include <memory>
#include <string>
#include <cmath>
#include <cstring>

namespace tmg {

#define TMG_HIP(expr)                                                                                       \
    do {                                                                                                    \
        hipError_t e_ = (expr);                                                                             \
        if (e_ != hipSuccess)                                                                               \
            return set_error(TMG_E_DEVICE, std::string("HIP error ") + hipGetErrorString(e_) + " in " #expr \
                                               " (" __FILE__ ":" + std::to_string(__LINE__) + ")");         \
    } while (0)

template <class T>
static int dev_alloc(tmg_model *m, T **p, size_t count) {
    void *q = nullptr;
    if (count == 0) count = 1;
    hipError_t e = hipMalloc(&q, count * sizeof(T));
    if (e != hipSuccess)
        return set_error(TMG_E_NOMEM, std::string("hipMalloc of ") + std::to_string(count * sizeof(T)) +
                                          " bytes failed: " + hipGetErrorString(e));
    m->allocs.push_back(q);
    *p = (T *)q;
    return TMG_OK;
}

int pinned(tmg_model *m, size_t bytes) {
    if (m->pin_bytes >= bytes) return TMG_OK;
    if (m->pin) (void)hipHostFree(m->pin);
    m->pin = nullptr;
    m->pin_bytes = 0;
    TMG_HIP(hipHostMalloc(&m->pin, bytes, hipHostMallocDefault));
    m->pin_bytes = bytes;
    return TMG_OK;
}

static void model_release(tmg_model *m) {
    if (!m) return;
    (void)hipSetDevice(m->device);
    if (m->stream) (void)hipStreamSynchronize(m->stream);
    for (void *p : m->allocs) (void)hipFree(p);
    if (m->pin) (void)hipHostFree(m->pin);
    if (m->stream) (void)hipStreamDestroy(m->stream);
    delete m;
}

// Rope::new + Rope::ensure (reference src/tensor.rs:1005-1023):
// inv_freq[i] = 1/theta^(2i/hd) with f32 powf; angle = pos * inv_freq[i];
// sin/cos with libm f32 -- the same calls the reference makes.
int ensure_rope(tmg_model *m, int npos) {
    if (npos <= m->rope_npos) return TMG_OK;
    const int half = m->hd / 2;
    int cap = m->rope_npos ? m->rope_npos : 64;
    while (cap < npos) cap *= 2;
    std::vector<float> inv(half), cs((size_t)cap * half), sn((size_t)cap * half);
    for (int i = 0; i < half; i++) inv[i] = 1.0f / powf(m->cfg.rope_theta, 2.0f * (float)i / (float)m->hd);
    for (int p = 0; p < cap; p++)
        for (int i = 0; i < half; i++) {
            float ang = (float)p * inv[i];
            sn[(size_t)p * half + i] = sinf(ang);
            cs[(size_t)p * half + i] = cosf(ang);
        }
    float *dc = nullptr, *ds = nullptr;
    int rc;
    if ((rc = dev_alloc(m, &dc, (size_t)cap * half)) || (rc = dev_alloc(m, &ds, (size_t)cap * half))) return rc;
    TMG_HIP(hipMemcpy(dc, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    TMG_HIP(hipMemcpy(ds, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
    // old tables stay allocated (graphs captured earlier may point at them)
    m->rope_cos = dc;
    m->rope_sin = ds;
    m->rope_npos = cap;
    return TMG_OK;
}

// ---------------------------------------------------------------------------
// load (reference load_model_safetensors, src/model.rs:181-244)
// ---------------------------------------------------------------------------

static int need(const SafeTensorsFile &f, const std::string &name, const std::vector<uint64_t> &shape,
                const TensorEntry **out) {
    const TensorEntry *e = f.find(name);
    if (!e) return set_error(TMG_E_MISSING, "missing tensor `" + name + "` in safetensors file");
    uint64_t want = 1;
    for (auto d : shape) want *= d;
    if (e->numel() != want) {
        std::string s;
        for (auto d : shape) s += (s.empty() ? "" : "x") + std::to_string(d);
        return set_error(TMG_E_INVALID, "tensor `" + name + "` has " + std::to_string(e->numel()) +
                                            " elements, expected " + s);
    }
    if (e->dtype == DType::Other)
        return set_error(TMG_E_DTYPE, "unsupported dtype " + e->dtype_name + " for tensor " + name);
    *out = e;
    return TMG_OK;
}

static int upload_f32(tmg_model *m, const SafeTensorsFile &f, const TensorEntry *e, float **dst) {
    std::vector<float> v;
    int rc = tensor_to_f32(f, *e, &v);
    if (rc) return rc;
    if ((rc = dev_alloc(m, dst, v.size()))) return rc;
    TMG_HIP(hipMemcpy(*dst, v.data(), v.size() * 4, hipMemcpyHostToDevice));
    return TMG_OK;
}

static int upload_raw(tmg_model *m, const void *src, size_t bytes, uint16_t **dst) {
    int rc;
    if ((rc = dev_alloc(m, dst, bytes / 2))) return rc;
    TMG_HIP(hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice));
    return TMG_OK;
}

static int upload_floats(tmg_model *m, const std::vector<float> &v, float **dst) {
    int rc;
    if ((rc = dev_alloc(m, dst, v.size()))) return rc;
    TMG_HIP(hipMemcpy(*dst, v.data(), v.size() * 4, hipMemcpyHostToDevice));
    return TMG_OK;
}

// Releases one allocation of the model before the model itself.
static void dev_free(tmg_model *m, void *p) {
    auto it = std::find(m->allocs.begin(), m->allocs.end(), p);
    if (it == m->allocs.end()) return;
    m->allocs.erase(it);
    (void)hipFree(p);
}

// Host-only phase: config.json + every tensor's presence, shape and dtype,
// so file errors surface before any device work (and without a GPU).
// A TMB1 file (reference load_model_tmb, src/model.rs:105-179) carries its
// config and is read through the same tensor interface.
static int validate_files(tmg_model *m, const std::string &path, SafeTensorsFile *f) {
    int rc;
    const bool tmb = is_tmb(path);
    if (tmb) {
        if ((rc = f->open_tmb(path, &m->cfg))) return rc;
    } else {
        std::string cpath;
        if (!config_path_for_model(path, &cpath))
            return set_error(TMG_E_MISSING, "config.json not found next to " + path);
        if ((rc = config_load(cpath, &m->cfg))) return rc;
    }
    m->from_tmb = tmb;
    const tmg_config &c = m->cfg;
    m->H = c.hidden_size;
    m->L = c.num_hidden_layers;
    m->nq = c.num_attention_heads;
    m->nkv = c.num_key_value_heads;
    m->hd = c.head_dim;
    m->I = c.intermediate_size;
    m->V = c.vocab_size;
    m->qd = m->nq * m->hd;
    m->kvd = m->nkv * m->hd;
    m->qkv_rows = m->qd + 2 * m->kvd;
    if (m->nkv == 0 || m->nq % m->nkv != 0)
        return set_error(TMG_E_INVALID, "num_attention_heads must be a multiple of num_key_value_heads");
    const int group = m->nq / m->nkv;
    if (group != 1 && group != 2 && group != 4 && group != 8)
        return set_error(TMG_E_INVALID, "GQA group size " + std::to_string(group) + " is not supported (1, 2, 4, 8)");
    if (m->hd != 16 && m->hd != 32 && m->hd != 64 && m->hd != 128 && m->hd != 256)
        return set_error(TMG_E_INVALID, "head_dim " + std::to_string(m->hd) + " is not supported (16..256, power of 2)");
    if (m->H % 32 || m->qd % 32 || m->I % 32 || m->H > 16384 || m->qd > 16384 || m->I > 16384)
        return set_error(TMG_E_INVALID, "hidden, q and intermediate sizes must be multiples of 32 and <= 16384");
    if (m->V == 0) return set_error(TMG_E_INVALID, "vocab_size is 0");
    if (!tmb && (rc = f->open(path))) return rc;
    const uint64_t H = m->H, I = m->I, V = m->V, qd = m->qd, kvd = m->kvd;
    const TensorEntry *e;
    if ((rc = need(*f, "model.embed_tokens.weight", {V, H}, &e))) return rc;
    // weight matrices: BF16 kept raw; F32 / F16 become f32 rows (WMat::F32,
    // src/model.rs:49-55); any other dtype is an error (need)
    for (int l = 0; l < m->L; l++) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        if ((rc = need(*f, p + "self_attn.q_proj.weight", {qd, H}, &e)) ||
            (rc = need(*f, p + "self_attn.k_proj.weight", {kvd, H}, &e)) ||
            (rc = need(*f, p + "self_attn.v_proj.weight", {kvd, H}, &e)) ||
            (rc = need(*f, p + "self_attn.o_proj.weight", {H, qd}, &e)) ||
            (rc = need(*f, p + "mlp.gate_proj.weight", {I, H}, &e)) ||
            (rc = need(*f, p + "mlp.up_proj.weight", {I, H}, &e)) ||
            (rc = need(*f, p + "mlp.down_proj.weight", {H, I}, &e)) ||
            (rc = need(*f, p + "input_layernorm.weight", {H}, &e)) ||
            (rc = need(*f, p + "post_attention_layernorm.weight", {H}, &e)))
            return rc;
    }
    if ((rc = need(*f, "model.norm.weight", {H}, &e))) return rc;
    if (f->find("lm_head.weight") && (rc = need(*f, "lm_head.weight", {V, H}, &e))) return rc;
    return TMG_OK;
}

// Device phase: upload into the HBM layout.
static int load_model(tmg_model *m, const SafeTensorsFile &f) {
    int rc;
    const int group = m->nq / m->nkv;
    const uint64_t H = m->H, I = m->I, V = m->V, qd = m->qd, kvd = m->kvd;

    // embedding: raw BF16 on the device, else f32 as the reference converts
    // it (an F32 table -- a TMB file's -- uploads as it lies in the file);
    // a tied lm_head streams the table as BF16, so then a table of BF16
    // values is narrowed back exactly (validate_files checked that)
    const TensorEntry *emb;
    if ((rc = need(f, "model.embed_tokens.weight", {V, H}, &emb))) return rc;
    const bool tied = f.find("lm_head.weight") == nullptr;
    if (emb->dtype == DType::BF16) {
        if ((rc = upload_raw(m, f.data(*emb), V * H * 2, &m->embed_bf16))) return rc;
    } else if (emb->dtype == DType::F32 && !tied) {
        if ((rc = dev_alloc(m, &m->embed_f32, V * H))) return rc;
        TMG_HIP(hipMemcpy(m->embed_f32, f.data(*emb), V * H * 4, hipMemcpyHostToDevice));
    } else {
        std::vector<float> v;
        if ((rc = tensor_to_f32(f, *emb, &v))) return rc;
        bool exact = true;
        std::vector<uint16_t> nb(v.size());
        for (size_t i = 0; i < v.size(); i++) {
            uint32_t u;
            memcpy(&u, &v[i], 4);
            exact = exact && (u & 0xFFFFu) == 0;
            nb[i] = (uint16_t)(u >> 16);
        }
        if (exact && tied) {
            if ((rc = upload_raw(m, nb.data(), nb.size() * 2, &m->embed_bf16))) return rc;
        } else {
            if ((rc = dev_alloc(m, &m->embed_f32, v.size()))) return rc;
            TMG_HIP(hipMemcpy(m->embed_f32, v.data(), v.size() * 4, hipMemcpyHostToDevice));
        }
    }

    const int half = m->hd / 2;
    std::vector<uint16_t> stage;
    std::vector<float> stagef;
    m->layers.resize(m->L);
    for (int l = 0; l < m->L; l++) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        const TensorEntry *wq, *wk, *wv, *wo, *wg, *wu, *wd, *n1, *n2;
        if ((rc = need(f, p + "self_attn.q_proj.weight", {qd, H}, &wq)) ||
            (rc = need(f, p + "self_attn.k_proj.weight", {kvd, H}, &wk)) ||
            (rc = need(f, p + "self_attn.v_proj.weight", {kvd, H}, &wv)) ||
            (rc = need(f, p + "self_attn.o_proj.weight", {H, qd}, &wo)) ||
            (rc = need(f, p + "mlp.gate_proj.weight", {I, H}, &wg)) ||
            (rc = need(f, p + "mlp.up_proj.weight", {I, H}, &wu)) ||
            (rc = need(f, p + "mlp.down_proj.weight", {H, I}, &wd)) ||
            (rc = need(f, p + "input_layernorm.weight", {H}, &n1)) ||
            (rc = need(f, p + "post_attention_layernorm.weight", {H}, &n2)))
            return rc;
        tmg_model::Layer &ly = m->layers[l];
        // A device matrix keeps raw BF16 rows when all its file tensors are
        // BF16 (WMat::BF16); otherwise it holds f32 rows (WMat::F32: F32 and
        // F16 tensors converted as the reference converts them, BF16 parts
        // widened exactly), in the same row order.
        auto bf16 = [](std::initializer_list<const TensorEntry *> es) {
            for (const TensorEntry *e : es)
                if (e->dtype != DType::BF16) return false;
            return true;
        };
        // QKV: logical rows [q; k; v]; physical row 2P = (head, j), 2P+1 = (head, j+hd/2)
        const int sec_rows[3] = {m->qd, m->kvd, m->kvd};
        if (bf16({wq, wk, wv})) {
            stage.resize((size_t)m->qkv_rows * H);
            const uint16_t *src[3] = {(const uint16_t *)f.data(*wq), (const uint16_t *)f.data(*wk),
                                      (const uint16_t *)f.data(*wv)};
            int P = 0;
            for (int sct = 0; sct < 3; sct++)
                for (int hh = 0; hh < sec_rows[sct] / m->hd; hh++)
                    for (int j = 0; j < half; j++, P++) {
                        memcpy(&stage[(size_t)(2 * P) * H], src[sct] + ((size_t)hh * m->hd + j) * H, H * 2);
                        memcpy(&stage[(size_t)(2 * P + 1) * H], src[sct] + ((size_t)hh * m->hd + j + half) * H,
                               H * 2);
                    }
            if ((rc = upload_raw(m, stage.data(), stage.size() * 2, &ly.qkv))) return rc;
        } else {
            std::vector<float> sf[3];
            if ((rc = tensor_to_f32(f, *wq, &sf[0])) || (rc = tensor_to_f32(f, *wk, &sf[1])) ||
                (rc = tensor_to_f32(f, *wv, &sf[2])))
                return rc;
            stagef.resize((size_t)m->qkv_rows * H);
            int P = 0;
            for (int sct = 0; sct < 3; sct++)
                for (int hh = 0; hh < sec_rows[sct] / m->hd; hh++)
                    for (int j = 0; j < half; j++, P++) {
                        memcpy(&stagef[(size_t)(2 * P) * H], sf[sct].data() + ((size_t)hh * m->hd + j) * H, H * 4);
                        memcpy(&stagef[(size_t)(2 * P + 1) * H],
                               sf[sct].data() + ((size_t)hh * m->hd + j + half) * H, H * 4);
                    }
            if ((rc = upload_floats(m, stagef, &ly.qkv_f))) return rc;
        }
        if (bf16({wo})) {
            if ((rc = upload_raw(m, f.data(*wo), H * qd * 2, &ly.o))) return rc;
        } else if ((rc = upload_f32(m, f, wo, &ly.o_f))) {
            return rc;
        }
        if (bf16({wg, wu})) {
            stage.resize((size_t)2 * I * H);
            const uint16_t *g = (const uint16_t *)f.data(*wg), *u = (const uint16_t *)f.data(*wu);
            for (uint64_t r = 0; r < I; r++) {
                memcpy(&stage[(2 * r) * H], g + r * H, H * 2);
                memcpy(&stage[(2 * r + 1) * H], u + r * H, H * 2);
            }
            if ((rc = upload_raw(m, stage.data(), stage.size() * 2, &ly.gu))) return rc;
        } else {
            std::vector<float> g, u;
            if ((rc = tensor_to_f32(f, *wg, &g)) || (rc = tensor_to_f32(f, *wu, &u))) return rc;
            stagef.resize((size_t)2 * I * H);
            for (uint64_t r = 0; r < I; r++) {
                memcpy(&stagef[(2 * r) * H], g.data() + r * H, H * 4);
                memcpy(&stagef[(2 * r + 1) * H], u.data() + r * H, H * 4);
            }
            if ((rc = upload_floats(m, stagef, &ly.gu_f))) return rc;
        }
        if (bf16({wd})) {
            if ((rc = upload_raw(m, f.data(*wd), H * I * 2, &ly.down))) return rc;
        } else if ((rc = upload_f32(m, f, wd, &ly.down_f))) {
            return rc;
        }
        if (ly.qkv_f || ly.o_f || ly.gu_f || ly.down_f) m->any_f32 = true;
        if ((rc = upload_f32(m, f, n1, &ly.in_norm)) || (rc = upload_f32(m, f, n2, &ly.post_norm))) return rc;
        if (m->i8) {
            // per-row quantization commutes with the row permutations above;
            // f32 rows are quantized from their f32 values (wmat_maybe_i8,
            // src/model.rs:69-72), their codes then kept as BF16 for prefill
            // and the f32 rows released
            struct {
                uint16_t **w;
                float **wf;
                int rows, in;
                int8_t **q8;
                float **sc;
            } mats[4] = {{&ly.qkv, &ly.qkv_f, m->qkv_rows, m->H, &ly.qkv8, &ly.qkv_s},
                         {&ly.o, &ly.o_f, m->H, m->qd, &ly.o8, &ly.o_s},
                         {&ly.gu, &ly.gu_f, 2 * m->I, m->H, &ly.gu8, &ly.gu_s},
                         {&ly.down, &ly.down_f, m->H, m->I, &ly.down8, &ly.down_s}};
            for (auto &mt : mats) {
                if ((rc = dev_alloc(m, mt.q8, (size_t)mt.rows * mt.in)) || (rc = dev_alloc(m, mt.sc, (size_t)mt.rows)))
                    return rc;
                if (*mt.wf) {
                    if ((rc = dev_alloc(m, mt.w, (size_t)mt.rows * mt.in))) return rc;
                    TMG_HIP(launch_quantize_i8_f32(*mt.wf, mt.rows, mt.in, *mt.q8, *mt.sc, *mt.w, m->stream));
                } else {
                    TMG_HIP(launch_quantize_i8(*mt.w, mt.rows, mt.in, *mt.q8, *mt.sc, true, m->stream));
                }
            }
            TMG_HIP(hipStreamSynchronize(m->stream));
            for (auto &mt : mats)
                if (*mt.wf) {
                    dev_free(m, *mt.wf);
                    *mt.wf = nullptr;
                }
        }
    }
    const TensorEntry *fn;
    if ((rc = need(f, "model.norm.weight", {H}, &fn)) || (rc = upload_f32(m, f, fn, &m->final_norm))) return rc;

    // lm_head: dedicated tensor if present, else tied to the embedding
    // (src/model.rs:230-233); tying reuses the raw BF16 table, which equals
    // the reference's f32 copy element for element.
    if (f.find("lm_head.weight")) {
        const TensorEntry *lm;
        if ((rc = need(f, "lm_head.weight", {V, H}, &lm))) return rc;
        if (lm->dtype == DType::BF16) {
            if ((rc = upload_raw(m, f.data(*lm), V * H * 2, &m->lm_head))) return rc;
        } else if ((rc = upload_f32(m, f, lm, &m->lm_head_f))) {
            return rc;
        }
        m->cfg.tied_lm_head = 0;
    } else {
        // WMat::F32(embed): the BF16 table when the file's values are BF16
        // values (exact), else the f32 table
        if (m->embed_bf16)
            m->lm_head = m->embed_bf16;
        else
            m->lm_head_f = m->embed_f32;
        m->cfg.tied_lm_head = 1;
    }
    if (m->lm_head_f) m->any_f32 = true;

    // decode scratch
    if ((rc = dev_alloc(m, &m->x, H)) || (rc = dev_alloc(m, &m->q, qd)) || (rc = dev_alloc(m, &m->attn_out, qd)) ||
        (rc = dev_alloc(m, &m->h, I)) || (rc = dev_alloc(m, &m->logits, V)))
        return rc;
    if ((rc = dev_alloc(m, &m->attn_part, (size_t)m->nkv * kMaxSplits * group * m->hd)) ||
        (rc = dev_alloc(m, &m->attn_ml, (size_t)m->nkv * kMaxSplits * group * 2)))
        return rc;
    m->argmax_nparts = gemv_blocks(m->V, m->H, m->lm_head_f != nullptr);
    if ((rc = dev_alloc(m, &m->argmax_part, (size_t)m->argmax_nparts))) return rc;
    if ((rc = ensure_rope(m, 64))) return rc;
    if ((rc = pinned(m, (size_t)std::max<uint64_t>(V * 4, 1 << 16)))) return rc;

    TMG_HIP(hipDeviceSynchronize());
    return TMG_OK;
}

// ---------------------------------------------------------------------------
// decode step (reference Model::forward_token, src/model.rs:392-491, plus the
// argmax of generate, src/model.rs:636-637)
// ---------------------------------------------------------------------------

bool LaunchRecorder::want(const char *name, double b) {
    names.push_back(name);
    bytes.push_back(b);
    return !none && (!only || strcmp(only, name) == 0);
}

// The split-K merge runs in the o_proj GEMV prologue when the splits are few
// (at most 8) and the attention output is at most 4096 wide: every o_proj
// workgroup re-reads the partials, which for the 4B shape (4096-wide output,
// 2560 rows, 16 rows per workgroup) makes o_proj 1.7 us slower but saves the
// 2.7 us merge kernel and its launch (sampled 4B 501 -> 518 tok/s).
static bool fused_merge(const tmg_model *m, const tmg_cache *c) {
    return c->attn_nsplit > 1 && c->attn_nsplit <= kFusedSplits && m->qd <= 4096;
}

int enqueue_decode_step(tmg_model *m, tmg_cache *c, LaunchRecorder *rec, int mode) {
    hipStream_t s = m->stream;
    const int H = m->H, I = m->I, qd = m->qd, kvd = m->kvd;
    const double n_ctx_est = (double)c->len + 1;
    // bytes per weight and per row scale of the layer matrices
    const double wb = m->i8 ? 1.0 : 2.0, sb = m->i8 ? 4.0 : 0.0;
    for (int l = 0; l < m->L; l++) {
        const tmg_model::Layer &ly = m->layers[l];
        float *kc = c->k + (size_t)l * c->max_pos * kvd;
        float *vc = c->v + (size_t)l * c->max_pos * kvd;

        GemvArgs qa{};
        qa.W = ly.qkv;
        qa.out = m->qkv_rows;
        qa.in = H;
        qa.x = m->x;
        qa.norm_w = ly.in_norm;
        qa.eps = m->cfg.rms_norm_eps;
        qa.rope_cos = m->rope_cos;
        qa.rope_sin = m->rope_sin;
        qa.pos = &c->st->pos;
        qa.hd = m->hd;
        qa.nq = m->nq;
        qa.nkv = m->nkv;
        qa.q_out = m->q;
        qa.k_cache = kc;
        qa.v_cache = vc;
        int pro = PRO_NORM;
        if (l == 0) {
            pro = PRO_EMBED_NORM;
            qa.token = &c->st->cur_token;
            qa.embed_bf16 = m->embed_bf16;
            qa.embed_f32 = m->embed_f32;
            qa.x_store = m->x;
        }
        qa.Wf = ly.qkv_f;
        if (m->i8) {
            qa.W8 = ly.qkv8;
            qa.wscale = ly.qkv_s;
        }
        if (!rec || rec->want("gemv_qkv_rope", (double)m->qkv_rows * (H * (ly.qkv_f ? 4.0 : wb) + sb) + H * 8.0 + (qd + 2 * kvd) * 4.0)) TMG_HIP(launch_gemv(pro, EPI_QKV, qa, s));

        AttnArgs aa{};
        aa.q = m->q;
        aa.k_cache = kc;
        aa.v_cache = vc;
        aa.nq = m->nq;
        aa.nkv = m->nkv;
        aa.hd = m->hd;
        aa.T = 1;
        aa.pos_dev = &c->st->pos;
        aa.scale = 1.0f / sqrtf((float)m->hd);
        aa.nsplit = c->attn_nsplit;
        aa.block = c->attn_block;
        aa.cap = (int)c->max_pos;
        aa.spec_splits = c->capture_spec_all ? c->attn_nsplit : 0;
        aa.part = m->attn_part;
        aa.part_ml = m->attn_ml;
        aa.out_f32 = c->attn_nsplit == 1 ? m->attn_out : nullptr;
        if (!rec || rec->want("attn_decode", 2.0 * n_ctx_est * kvd * 4 + 2.0 * qd * 4)) TMG_HIP(launch_attn(aa, s));
        const bool fused = fused_merge(m, c);
        if (c->attn_nsplit > 1 && !fused) {
            aa.out_f32 = m->attn_out;
            if (!rec || rec->want("attn_combine", 0.0)) TMG_HIP(launch_attn_combine(aa, s));
        }

        GemvArgs oa{};
        oa.W = ly.o;
        oa.out = H;
        oa.in = qd;
        oa.x = m->attn_out;
        oa.y = m->x;
        if (fused) {
            oa.part = m->attn_part;
            oa.part_ml = m->attn_ml;
            oa.pos = &c->st->pos;
            oa.nsplit = c->attn_nsplit;
            oa.attn_block = c->attn_block;
            oa.hd = m->hd;
            oa.group = m->nq / m->nkv;
        }
        oa.Wf = ly.o_f;
        if (m->i8) {
            oa.W8 = ly.o8;
            oa.wscale = ly.o_s;
        }
        if (!rec || rec->want("gemv_o_resid", (double)H * (qd * (ly.o_f ? 4.0 : wb) + sb) + qd * 4.0 + H * 8.0)) TMG_HIP(launch_gemv(fused ? PRO_ATTN_COMBINE : PRO_PLAIN, EPI_RESID, oa, s));

        GemvArgs ga{};
        ga.W = ly.gu;
        ga.out = 2 * I;
        ga.in = H;
        ga.x = m->x;
        ga.norm_w = ly.post_norm;
        ga.eps = m->cfg.rms_norm_eps;
        ga.y = m->h;
        ga.Wf = ly.gu_f;
        if (m->i8) {
            ga.W8 = ly.gu8;
            ga.wscale = ly.gu_s;
        }
        if (!rec || rec->want("gemv_gateup_swiglu", 2.0 * I * (H * (ly.gu_f ? 4.0 : wb) + sb) + H * 8.0 + I * 4.0)) TMG_HIP(launch_gemv(PRO_NORM, EPI_SWIGLU, ga, s));

        GemvArgs da{};
        da.W = ly.down;
        da.out = H;
        da.in = I;
        da.x = m->h;
        da.y = m->x;
        da.Wf = ly.down_f;
        if (m->i8) {
            da.W8 = ly.down8;
            da.wscale = ly.down_s;
        }
        if (!rec || rec->want("gemv_down_resid", (double)H * (I * (ly.down_f ? 4.0 : wb) + sb) + I * 4.0 + H * 8.0)) TMG_HIP(launch_gemv(PRO_PLAIN, EPI_RESID, da, s));
    }
    GemvArgs la{};
    la.W = m->lm_head;
    la.Wf = m->lm_head_f;
    la.out = m->V;
    la.in = H;
    la.x = m->x;
    la.norm_w = m->final_norm;
    la.eps = m->cfg.rms_norm_eps;
    la.y = m->logits;
    la.argmax_part = mode == SEL_ARGMAX ? m->argmax_part : nullptr;
    if (!rec || rec->want("gemv_lmhead_argmax", (double)m->V * H * (m->lm_head_f ? 4 : 2) + H * 8.0 + m->V * 4.0)) TMG_HIP(launch_gemv(PRO_NORM, EPI_LOGITS, la, s));
    int rc = TMG_OK;
    if (!rec || rec->want(mode == SEL_ARGMAX ? "finalize" : "sample", mode == SEL_ARGMAX ? 0.0 : m->V * 4.0)) rc = enqueue_select(m, c, mode, 1);
    return rc;
}

int enqueue_select(tmg_model *m, tmg_cache *c, int mode, int advance_pos) {
    if (mode == SEL_ARGMAX) {
        FinalizeArgs fa{c->st, c->history, advance_pos, m->V, m->argmax_part, m->argmax_nparts, (int)c->max_pos + 2};
        TMG_HIP(launch_finalize(fa, m->stream));
        return TMG_OK;
    }
    SampleArgs sa{};
    sa.logits = m->logits;
    sa.V = m->V;
    sa.st = c->st;
    sa.seen = c->seen;
    sa.seen_rw = c->seen;
    sa.cand = mode == SEL_FULL ? nullptr : c->cand;
    sa.scratch = c->gsc;
    sa.use_k = c->samp_use_k;
    sa.use_p = c->samp_use_p;
    sa.draws = c->draws;
    sa.n_draws = (int)c->max_pos + 2;
    sa.history = c->history;
    sa.hist_cap = (int)c->max_pos + 2;
    sa.greedy = mode == SEL_PENALTY_ARGMAX;
    sa.advance_pos = advance_pos;
    TMG_HIP(launch_sample(sa, m->stream));
    return TMG_OK;
}

int step_form(const tmg_cache *c, uint64_t pos) {
    // all splits active: ceil((pos + 1) / block) >= nsplit.  Where they are,
    // the first-block loads of splits kSpecSplits.. need not wait for the
    // position read (8K context: 15.5 -> 15.15 us per layer); on a long
    // cache at a short context they would stream every inactive split's
    // first block
    return c->attn_nsplit > kSpecSplits && pos + 1 > (uint64_t)(c->attn_nsplit - 1) * (uint64_t)c->attn_block;
}

int get_step_graph(tmg_model *m, tmg_cache *c, int mode, int form) {
    if (c->graphs[form][mode]) return TMG_OK;
    TMG_HIP(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    c->capture_spec_all = form == 1;
    int rc = enqueue_decode_step(m, c, nullptr, mode);
    c->capture_spec_all = false;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(m->stream, &g);
    if (rc) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    TMG_HIP(e);
    hipGraphExec_t ex = nullptr;
    e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        TMG_HIP(e);
    }
    c->graph_src[form][mode] = g;
    c->graphs[form][mode] = ex;
    return TMG_OK;
}

bool step_graphs_enabled() {
    // TMG_DECODE_GRAPH=0 launches each step's kernels one by one instead of
    // replaying the captured graph (for tools that cannot trace graph launches)
    static const bool on = [] {
        const char *e = getenv("TMG_DECODE_GRAPH");
        return !(e && e[0] == '0');
    }();
    return on;
}

int launch_step(tmg_model *m, tmg_cache *c, int mode, uint64_t pos) {
    const int form = step_form(c, pos);
    if (!step_graphs_enabled()) {
        c->capture_spec_all = form == 1;
        const int rc = enqueue_decode_step(m, c, nullptr, mode);
        c->capture_spec_all = false;
        return rc;
    }
    int rc = get_step_graph(m, c, mode, form);
    if (rc) return rc;
    TMG_HIP(hipGraphLaunch(c->graphs[form][mode], m->stream));
    return TMG_OK;
}

int set_state(tmg_model *m, tmg_cache *c, int token, bool reset_step) {
    // one small H2D write of the host-known fields; the step counter and the
    // argmax key are reset together with the position when asked
    DevState st{};
    st.pos = (int)c->len;
    st.cur_token = token;
    st.step = 0;
    st.argmax_key = kArgmaxInit;
    if (reset_step) {
        const size_t n = offsetof(DevState, temperature);
        memcpy(m->pin, &st, n);
        TMG_HIP(hipMemcpyAsync(c->st, m->pin, n, hipMemcpyHostToDevice, m->stream));
    } else {
        int v[2] = {st.pos, st.cur_token};
        memcpy(m->pin, v, sizeof(v));
        TMG_HIP(hipMemcpyAsync(c->st, m->pin, sizeof(v), hipMemcpyHostToDevice, m->stream));
    }
    return TMG_OK;
}

// ---------------------------------------------------------------------------
// prefill (reference Model::forward_seq, src/model.rs:503-590)
// ---------------------------------------------------------------------------

static int ensure_prefill(tmg_model *m, int T) {
    if (T <= m->pf_cap) return TMG_OK;
    int cap = std::max(T, 64);
    // earlier buffers are released lazily with the model
    int rc;
    if ((rc = dev_alloc(m, &m->pf_tokens, cap)) || (rc = dev_alloc(m, &m->pf_x, (size_t)cap * m->H)) ||
        (rc = dev_alloc(m, &m->pf_q, (size_t)cap * m->qd)) || (rc = dev_alloc(m, &m->pf_hi, (size_t)cap * m->H)) ||
        (rc = dev_alloc(m, &m->pf_lo, (size_t)cap * m->H)) || (rc = dev_alloc(m, &m->pf_ahi, (size_t)cap * m->qd)) ||
        (rc = dev_alloc(m, &m->pf_alo, (size_t)cap * m->qd)) || (rc = dev_alloc(m, &m->pf_hhi, (size_t)cap * m->I)) ||
        (rc = dev_alloc(m, &m->pf_hlo, (size_t)cap * m->I)) ||
        (rc = dev_alloc(m, &m->pf_nss, (size_t)cap * ((m->H + 63) / 64))))
        return rc;
    if (!m->pf_part) {
        const size_t nc = skinny_counters(std::max(std::max(m->qkv_rows, m->H), 2 * m->I));
        if ((rc = dev_alloc(m, &m->pf_part, kSkinnyPartFloats)) || (rc = dev_alloc(m, &m->pf_cnt, nc))) return rc;
        hipError_t e = hipMemset(m->pf_cnt, 0, nc * sizeof(unsigned));
        if (e != hipSuccess) return set_error(TMG_E_DEVICE, std::string("hipMemset: ") + hipGetErrorString(e));
    }
    m->pf_cap = cap;
    return TMG_OK;
}

// Split-bf16 KV scratch for cache rows [0, n) (n rounded up to 64).
static int ensure_kv_split(tmg_model *m, int n) {
    const int cap = (n + 63) / 64 * 64;
    if (cap <= m->kv_cap) return TMG_OK;
    int rc;
    const size_t sz = (size_t)cap * m->kvd;
    if ((rc = dev_alloc(m, &m->pf_kh, sz)) || (rc = dev_alloc(m, &m->pf_kl, sz)) || (rc = dev_alloc(m, &m->pf_vth, sz)) ||
        (rc = dev_alloc(m, &m->pf_vtl, sz)))
        return rc;
    m->kv_cap = cap;
    return TMG_OK;
}

// Runs the batched prefill; leaves the last token's logits in m->logits and
// the per-workgroup argmax keys in m->argmax_part.
int run_prefill(tmg_model *m, tmg_cache *c, const uint32_t *tokens, size_t n) {
    const int T = (int)n;
    const int H = m->H, I = m->I, qd = m->qd, kvd = m->kvd;
    hipStream_t s = m->stream;
    int rc;
    if ((rc = ensure_prefill(m, T))) return rc;
    if ((rc = ensure_rope(m, (int)c->len + T + 1))) return rc;
    if ((rc = pinned(m, (size_t)T * 4 + 64 + (size_t)m->V * 4))) return rc;
    memcpy(m->pin, tokens, (size_t)T * 4);
    TMG_HIP(hipMemcpyAsync(m->pf_tokens, m->pin, (size_t)T * 4, hipMemcpyHostToDevice, s));
    TMG_HIP(launch_embed_gather(m->pf_tokens, T, H, m->embed_bf16, m->embed_f32, m->pf_x, s));
    const int start = (int)c->len;
    const float eps = m->cfg.rms_norm_eps;
    // RMSNorm hand-off: the o_proj and down GEMMs write the next GEMM's
    // operand (new residual times the norm weight, split-bf16) and per-64-row
    // sums of squares, and QKV / gate-up apply the 1/rms scale in their
    // epilogues, instead of a separate normalization pass over the residual
    // (shapes permitting: hidden a multiple of 64, all four GEMMs on kernels
    // with the staged epilogue)
    // (f32 weight matrices run a per-element epilogue: no hand-off)
    bool f32_mats = false;
    for (const tmg_model::Layer &ly : m->layers) f32_mats = f32_mats || ly.qkv_f || ly.o_f || ly.gu_f || ly.down_f;
    const bool hand_off = !f32_mats && H % 256 == 0 && H / 64 <= kMaxNormGroups && gemm_stages_output(m->qkv_rows, T, H) &&
                          gemm_stages_output(H, T, qd) && gemm_stages_output(2 * I, T, H) &&
                          gemm_stages_output(H, T, I);
    auto norm_in = [&](GemmArgs &a) {  // consumer of a handed-off norm
        a.nss_in = m->pf_nss;
        a.ngroups = H / 64;
        a.nrm_eps = eps;
    };
    auto norm_out = [&](GemmArgs &a, const float *w) {  // producer
        a.nrm_w = w;
        a.nss = m->pf_nss;
        a.nx_hi = m->pf_hi;
        a.nx_lo = m->pf_lo;
    };
    for (int l = 0; l < m->L; l++) {
        const tmg_model::Layer &ly = m->layers[l];
        float *kc = c->k + (size_t)l * c->max_pos * kvd;
        float *vc = c->v + (size_t)l * c->max_pos * kvd;
        const bool in_handed = hand_off && l > 0;
        if (!in_handed) TMG_HIP(launch_rmsnorm_split(m->pf_x, ly.in_norm, eps, T, H, m->pf_hi, m->pf_lo, s));
        GemmArgs g{};
        g.W = ly.qkv;
        g.Wf = ly.qkv_f;
        g.Bhi = m->pf_hi;
        g.Blo = m->pf_lo;
        g.M = m->qkv_rows;
        g.N = T;
        g.K = H;
        g.rope_cos = m->rope_cos;
        g.rope_sin = m->rope_sin;
        g.start = start;
        g.hd = m->hd;
        g.nq = m->nq;
        g.nkv = m->nkv;
        g.q_out = m->pf_q;
        g.k_cache = kc;
        g.v_cache = vc;
        g.part = m->pf_part;
        g.cnt = m->pf_cnt;
        if (m->i8) g.wscale = ly.qkv_s;
        if (in_handed) norm_in(g);
        TMG_HIP(launch_gemm(GEPI_QKV, g, s));

        AttnArgs aa{};
        aa.q = m->pf_q;
        aa.k_cache = kc;
        aa.v_cache = vc;
        aa.nq = m->nq;
        aa.nkv = m->nkv;
        aa.hd = m->hd;
        aa.T = T;
        aa.start = start;
        aa.scale = 1.0f / sqrtf((float)m->hd);
        aa.nsplit = 1;
        // rows of short prompts: at four or more query heads per KV head the
        // 64-position chunk holds 237 VGPRs (one wavefront per SIMD);
        // 16-position chunks hold 99 (4B 128-token prefill 5.88 -> 5.83 ms;
        // at two heads per KV head 64 stays faster, 1B 1.63 against 1.64 ms)
        if (m->nq / m->nkv >= 4) aa.block = attn_chunk(m->hd, m->nq / m->nkv, kAttnThreads, kAttnBlockShort);
        aa.out_hi = m->pf_ahi;
        aa.out_lo = m->pf_alo;
        if (attn_prefill_supported(aa)) {
            if ((rc = ensure_kv_split(m, start + T))) return rc;
            KVSplitArgs ka{kc, vc, start + T, m->nkv, m->hd, m->pf_kh, m->pf_kl, m->pf_vth, m->pf_vtl, m->kv_cap};
            TMG_HIP(launch_kv_split(ka, s));
            aa.kh = m->pf_kh;
            aa.kl = m->pf_kl;
            aa.vth = m->pf_vth;
            aa.vtl = m->pf_vtl;
            aa.vt_pitch = m->kv_cap;
            TMG_HIP(launch_attn_prefill(aa, s));
        } else {
            TMG_HIP(launch_attn(aa, s));
        }

        GemmArgs o{};
        o.W = ly.o;
        o.Wf = ly.o_f;
        o.Bhi = m->pf_ahi;
        o.Blo = m->pf_alo;
        o.M = H;
        o.N = T;
        o.K = qd;
        o.y = m->pf_x;
        o.part = m->pf_part;
        o.cnt = m->pf_cnt;
        if (m->i8) o.wscale = ly.o_s;
        if (hand_off) norm_out(o, ly.post_norm);
        TMG_HIP(launch_gemm(GEPI_RESID, o, s));

        if (!hand_off) TMG_HIP(launch_rmsnorm_split(m->pf_x, ly.post_norm, eps, T, H, m->pf_hi, m->pf_lo, s));
        GemmArgs gu{};
        gu.W = ly.gu;
        gu.Wf = ly.gu_f;
        gu.Bhi = m->pf_hi;
        gu.Blo = m->pf_lo;
        gu.M = 2 * I;
        gu.N = T;
        gu.K = H;
        gu.h_hi = m->pf_hhi;
        gu.h_lo = m->pf_hlo;
        gu.part = m->pf_part;
        gu.cnt = m->pf_cnt;
        if (m->i8) gu.wscale = ly.gu_s;
        if (hand_off) norm_in(gu);
        TMG_HIP(launch_gemm(GEPI_SWIGLU, gu, s));

        GemmArgs d{};
        d.W = ly.down;
        d.Wf = ly.down_f;
        d.Bhi = m->pf_hhi;
        d.Blo = m->pf_hlo;
        d.M = H;
        d.N = T;
        d.K = I;
        d.y = m->pf_x;
        d.part = m->pf_part;
        d.cnt = m->pf_cnt;
        if (m->i8) d.wscale = ly.down_s;
        if (hand_off && l + 1 < m->L) norm_out(d, m->layers[l + 1].in_norm);
        TMG_HIP(launch_gemm(GEPI_RESID, d, s));
    }
    // final norm of the last row (batch association) + lm_head + argmax
    GemvArgs la{};
    la.W = m->lm_head;
    la.Wf = m->lm_head_f;
    la.out = m->V;
    la.in = H;
    la.x = m->pf_x + (size_t)(T - 1) * H;
    la.norm_w = m->final_norm;
    la.eps = m->cfg.rms_norm_eps;
    la.y = m->logits;
    la.argmax_part = m->argmax_part;
    TMG_HIP(launch_gemv(PRO_NORM_BATCH, EPI_LOGITS, la, s));
    c->len += (uint32_t)T;
    // the device position follows the host mirror after a prefill
    memcpy((char *)m->pin + ((size_t)T * 4 + 63) / 64 * 64, &c->len, 4);
    TMG_HIP(hipMemcpyAsync(&c->st->pos, (char *)m->pin + ((size_t)T * 4 + 63) / 64 * 64, 4, hipMemcpyHostToDevice, s));
    return TMG_OK;
}

}  // namespace tmg

using namespace tmg;

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

extern "C" int tmg_model_load(const char *path, int device, tmg_model **out) {
    clear_error();
    if (!path || !out) return set_error(TMG_E_INVALID, "null argument");
    *out = nullptr;
    tmg_model *m = new tmg_model();
    SafeTensorsFile f;
    int rc = validate_files(m, path, &f);
    if (rc) {
        delete m;
        return rc;
    }
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess || ndev == 0) {
        delete m;
        return set_error(TMG_E_DEVICE, "no HIP device available");
    }
    if (device < 0 || device >= ndev) {
        delete m;
        return set_error(TMG_E_INVALID, "device index out of range");
    }
    m->device = device;
    {
        // the reference's gate: std::env::var("TMG_I8") == "1" (src/model.rs:61);
        // a TMB file always loads its BF16 views (load_model_tmb has no int8 path)
        const char *e = getenv("TMG_I8");
        m->i8 = e && strcmp(e, "1") == 0 && !m->from_tmb;
    }
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&m->stream, hipStreamNonBlocking) != hipSuccess) {
        model_release(m);
        return set_error(TMG_E_DEVICE, "cannot create a HIP stream on the device");
    }
    rc = load_model(m, f);
    if (rc) {
        std::string msg = tmg_last_error();
        model_release(m);
        return set_error(rc, msg);
    }
    *out = m;
    return TMG_OK;
}

extern "C" void tmg_model_free(tmg_model *m) {
    if (!m) return;
    {
        std::lock_guard<std::mutex> lk(m->life_mu);
        if (m->live_caches > 0) {
            m->free_requested = true;  // released by the last tmg_cache_free
            return;
        }
    }
    model_release(m);
}

extern "C" int tmg_model_config(const tmg_model *m, tmg_config *out) {
    if (!m || !out) return set_error(TMG_E_INVALID, "null argument");
    *out = m->cfg;
    return TMG_OK;
}

extern "C" int tmg_cache_new(tmg_model *m, uint32_t max_pos, tmg_cache **out) {
    clear_error();
    if (!m || !out || max_pos == 0) return set_error(TMG_E_INVALID, "bad argument to tmg_cache_new");
    *out = nullptr;
    (void)hipSetDevice(m->device);
    {
        std::lock_guard<std::mutex> lk(m->life_mu);
        if (m->free_requested) return set_error(TMG_E_INVALID, "model handle already freed");
        m->live_caches++;
    }
    tmg_cache *c = new tmg_cache();
    c->model = m;
    c->max_pos = max_pos;
    // Short caches deal the context to at most kFusedSplits splits in small
    // blocks: at 64-320 positions (1B) 5-8 workgroups per KV head of 16-40
    // positions each instead of 2-5 of 64, the merge still fused into o_proj.
    if (max_pos <= (uint32_t)kShortAttnCache) {
        c->attn_block = attn_chunk(m->hd, m->nq / m->nkv, kAttnThreads, kAttnBlockShort);
        c->attn_nsplit = (int)std::min<uint32_t>(kFusedSplits, (max_pos + c->attn_block - 1) / c->attn_block);
    } else {
        c->attn_block = kAttnBlockLong;
        c->attn_nsplit = (int)std::min<uint32_t>(kMaxSplits, (max_pos + kAttnBlockLong - 1) / kAttnBlockLong);
    }
    const size_t n = (size_t)m->L * max_pos * m->kvd;
    int rc = TMG_OK;
    void *k = nullptr, *v = nullptr, *st = nullptr, *hist = nullptr;
    if (hipMalloc(&k, n * 4) != hipSuccess || hipMalloc(&v, n * 4) != hipSuccess ||
        hipMalloc(&st, sizeof(DevState)) != hipSuccess ||
        hipHostMalloc(&hist, ((size_t)max_pos + 2) * 4, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess)
        rc = set_error(TMG_E_NOMEM, "KV cache allocation of " + std::to_string(2 * n * 4) + " bytes failed");
    c->k = (float *)k;
    c->v = (float *)v;
    c->st = (DevState *)st;
    c->history = (int *)hist;
    const size_t seen_words = ((size_t)m->V + 31) / 32;
    const size_t nslices = ((size_t)m->V + kSampleSlice - 1) / kSampleSlice;
    void *seen = nullptr, *cand = nullptr, *gsc = nullptr, *draws = nullptr;
    if (!rc && (hipMalloc(&seen, seen_words * 4) != hipSuccess ||
                hipMalloc(&cand, nslices * kSampleMaxK * 8) != hipSuccess ||
                hipMalloc(&gsc, kSampleScratchBytes(m->V)) != hipSuccess ||
                hipMalloc(&draws, ((size_t)max_pos + 2) * 4) != hipSuccess))
        rc = set_error(TMG_E_NOMEM, "sampler buffer allocation failed");
    c->seen = (unsigned *)seen;
    c->cand = (unsigned long long *)cand;
    c->gsc = (float *)gsc;
    c->draws = (float *)draws;
    if (!rc && (hipMemset(c->draws, 0, ((size_t)max_pos + 2) * 4) != hipSuccess ||
                hipMemset(c->gsc, 0, kSampleScratchBytes(m->V)) != hipSuccess))
        rc = set_error(TMG_E_DEVICE, "hipMemset failed");
    if (!rc && hipMemset(c->seen, 0, seen_words * 4) != hipSuccess) rc = set_error(TMG_E_DEVICE, "hipMemset failed");
    if (!rc) {
        DevState init{};
        init.argmax_key = kArgmaxInit;
        init.temperature = 0.0f;
        init.top_p = 1.0f;
        init.penalty = 1.0f;
        if (hipMemcpy(c->st, &init, sizeof(init), hipMemcpyHostToDevice) != hipSuccess)
            rc = set_error(TMG_E_DEVICE, "state upload failed");
    }
    if (!rc) rc = ensure_rope(m, (int)max_pos + 1);
    if (!rc) rc = set_state(m, c, 0, true);
    if (!rc && hipStreamSynchronize(m->stream) != hipSuccess) rc = set_error(TMG_E_DEVICE, "stream sync failed");
    if (rc) {
        tmg_cache_free(c);
        return rc;
    }
    *out = c;
    return TMG_OK;
}

extern "C" void tmg_cache_free(tmg_cache *c) {
    if (!c) return;
    (void)hipSetDevice(c->model->device);
    (void)hipStreamSynchronize(c->model->stream);
    for (int f = 0; f < 2; f++)
        for (int i = 0; i < 4; i++) {
            if (c->graphs[f][i]) (void)hipGraphExecDestroy(c->graphs[f][i]);
            if (c->graph_src[f][i]) (void)hipGraphDestroy(c->graph_src[f][i]);
        }
    (void)hipFree(c->seen);
    (void)hipFree(c->cand);
    (void)hipFree(c->gsc);
    (void)hipFree(c->draws);
    (void)hipFree(c->k);
    (void)hipFree(c->v);
    (void)hipFree(c->st);
    (void)hipHostFree(c->history);
    tmg_model *m = c->model;
    delete c;
    bool release;
    {
        std::lock_guard<std::mutex> lk(m->life_mu);
        release = --m->live_caches == 0 && m->free_requested;
    }
    if (release) model_release(m);
}

extern "C" int tmg_cache_len(const tmg_cache *c, uint32_t layer, uint32_t *len) {
    if (!c || !len) return set_error(TMG_E_INVALID, "null argument");
    if (layer >= (uint32_t)c->model->L) return set_error(TMG_E_INVALID, "layer index out of range");
    *len = c->len;
    return TMG_OK;
}

extern "C" int tmg_cache_reset(tmg_cache *c) {
    if (!c) return set_error(TMG_E_INVALID, "null argument");
    (void)hipSetDevice(c->model->device);
    c->len = 0;
    int rc = set_state(c->model, c, 0, true);
    if (rc) return rc;
    TMG_HIP(hipStreamSynchronize(c->model->stream));
    return TMG_OK;
}

extern "C" int tmg_cache_read(const tmg_cache *c, uint32_t layer, float *keys, float *values) {
    if (!c) return set_error(TMG_E_INVALID, "null argument");
    tmg_model *m = c->model;
    if (layer >= (uint32_t)m->L) return set_error(TMG_E_INVALID, "layer index out of range");
    (void)hipSetDevice(m->device);
    TMG_HIP(hipStreamSynchronize(m->stream));
    const size_t off = (size_t)layer * c->max_pos * m->kvd, bytes = (size_t)c->len * m->kvd * 4;
    if (keys && bytes) TMG_HIP(hipMemcpy(keys, c->k + off, bytes, hipMemcpyDeviceToHost));
    if (values && bytes) TMG_HIP(hipMemcpy(values, c->v + off, bytes, hipMemcpyDeviceToHost));
    return TMG_OK;
}

static int fetch_logits(tmg_model *m, float *logits) {
    if (logits) {
        TMG_HIP(hipMemcpyAsync(m->pin, m->logits, (size_t)m->V * 4, hipMemcpyDeviceToHost, m->stream));
        TMG_HIP(hipStreamSynchronize(m->stream));
        memcpy(logits, m->pin, (size_t)m->V * 4);
    } else {
        TMG_HIP(hipStreamSynchronize(m->stream));
    }
    return TMG_OK;
}

extern "C" int tmg_forward_token(tmg_model *m, tmg_cache *c, uint32_t token, float *logits) {
    clear_error();
    if (!m || !c || c->model != m) return set_error(TMG_E_INVALID, "bad model/cache handle");
    if (token >= (uint32_t)m->V) return set_error(TMG_E_INVALID, "token id " + std::to_string(token) + " out of range");
    if (c->len >= c->max_pos) return set_error(TMG_E_CAPACITY, "KV cache full (max_pos " + std::to_string(c->max_pos) + ")");
    (void)hipSetDevice(m->device);
    int rc;
    if ((rc = set_state(m, c, (int)token, false))) return rc;
    if ((rc = launch_step(m, c, SEL_ARGMAX, c->len))) return rc;
    c->len += 1;
    return fetch_logits(m, logits);
}

extern "C" int tmg_forward_seq(tmg_model *m, tmg_cache *c, const uint32_t *tokens, size_t n, float *last_logits) {
    clear_error();
    if (!m || !c || c->model != m || (!tokens && n)) return set_error(TMG_E_INVALID, "bad argument");
    if (n == 0) return set_error(TMG_E_EMPTY, "empty prompt");
    for (size_t i = 0; i < n; i++)
        if (tokens[i] >= (uint32_t)m->V) return set_error(TMG_E_INVALID, "token id out of range");
    if ((uint64_t)c->len + n > c->max_pos) return set_error(TMG_E_CAPACITY, "KV cache full");
    (void)hipSetDevice(m->device);
    int rc = run_prefill(m, c, tokens, n);
    if (rc) return rc;
    return fetch_logits(m, last_logits);
}

extern "C" int tmg_prefill(tmg_model *m, tmg_cache *c, const uint32_t *tokens, size_t n, float *last_logits) {
    if (n == 0) return set_error(TMG_E_EMPTY, "empty prompt");
    return tmg_forward_seq(m, c, tokens, n, last_logits);
}

extern "C" int tmg_gemv_bf16(const uint16_t *w, const float *x, float *y, uint32_t out, uint32_t in, void *stream) {
    if (!w || !x || !y || out == 0 || in == 0) return set_error(TMG_E_INVALID, "bad argument to tmg_gemv_bf16");
    if (in % 8 != 0 || in > 16384) return set_error(TMG_E_INVALID, "in must be a multiple of 8 and <= 16384");
    if (((uintptr_t)w & 15) || ((uintptr_t)x & 15)) return set_error(TMG_E_INVALID, "W and x must be 16-byte aligned");
    GemvArgs a{};
    a.W = w;
    a.out = (int)out;
    a.in = (int)in;
    a.x = x;
    a.y = y;
    TMG_HIP(launch_gemv(PRO_PLAIN, EPI_STORE, a, (hipStream_t)stream));
    return TMG_OK;
}

extern "C" int tmg_gemv_f32(const float *w, const float *x, float *y, uint32_t out, uint32_t in, void *stream) {
    if (!w || !x || !y || out == 0 || in == 0) return set_error(TMG_E_INVALID, "bad argument to tmg_gemv_f32");
    if (in % 8 != 0 || in > 16384) return set_error(TMG_E_INVALID, "in must be a multiple of 8 and <= 16384");
    if (((uintptr_t)w & 15) || ((uintptr_t)x & 15)) return set_error(TMG_E_INVALID, "W and x must be 16-byte aligned");
    GemvArgs a{};
    a.Wf = w;
    a.out = (int)out;
    a.in = (int)in;
    a.x = x;
    a.y = y;
    TMG_HIP(launch_gemv(PRO_PLAIN, EPI_STORE, a, (hipStream_t)stream));
    return TMG_OK;
}

extern "C" int tmg_gemv_i8(const int8_t *q, const float *scale, const float *x, float *y, uint32_t out, uint32_t in,
                           void *stream) {
    if (!q || !scale || !x || !y || out == 0 || in == 0) return set_error(TMG_E_INVALID, "bad argument to tmg_gemv_i8");
    if (in % 8 != 0 || in > 16384) return set_error(TMG_E_INVALID, "in must be a multiple of 8 and <= 16384");
    if (((uintptr_t)q & 7) || ((uintptr_t)x & 15) || ((uintptr_t)scale & 3))
        return set_error(TMG_E_INVALID, "q must be 8-byte, x 16-byte and scale 4-byte aligned");
    GemvArgs a{};
    a.W8 = q;
    a.wscale = scale;
    a.out = (int)out;
    a.in = (int)in;
    a.x = x;
    a.y = y;
    TMG_HIP(launch_gemv(PRO_PLAIN, EPI_STORE, a, (hipStream_t)stream));
    return TMG_OK;
}

extern "C" int tmg_quantize_i8(const uint16_t *w, uint32_t rows, uint32_t in, int8_t *q, float *scale, void *stream) {
    if (!w || !q || !scale || rows == 0 || in == 0) return set_error(TMG_E_INVALID, "bad argument to tmg_quantize_i8");
    if (in % 8 != 0 || rows > 0x7fffffffu || in > 0x7fffffffu)
        return set_error(TMG_E_INVALID, "in must be a multiple of 8");
    if (((uintptr_t)w & 15) || ((uintptr_t)q & 7) || ((uintptr_t)scale & 3))
        return set_error(TMG_E_INVALID, "w must be 16-byte, q 8-byte and scale 4-byte aligned");
    // rewrite = false: w is only read
    TMG_HIP(launch_quantize_i8(const_cast<uint16_t *>(w), (int)rows, (int)in, q, scale, false, (hipStream_t)stream));
    return TMG_OK;
}

extern "C" int tmg_decode_greedy(tmg_model *m, tmg_cache *c, uint32_t token, uint32_t n_steps, uint32_t *tokens_out,
                                 float *ms) {
    clear_error();
    if (!m || !c || c->model != m) return set_error(TMG_E_INVALID, "bad model/cache handle");
    if (token >= (uint32_t)m->V) return set_error(TMG_E_INVALID, "token id out of range");
    if ((uint64_t)c->len + n_steps > c->max_pos) return set_error(TMG_E_CAPACITY, "KV cache full");
    (void)hipSetDevice(m->device);
    int rc;
    if ((rc = set_state(m, c, (int)token, true))) return rc;
    // the step graphs (the forms of the first and the last step) are
    // captured before the first timing event
    if (step_graphs_enabled() && n_steps > 0 &&
        ((rc = get_step_graph(m, c, SEL_ARGMAX, step_form(c, c->len))) ||
         (rc = get_step_graph(m, c, SEL_ARGMAX, step_form(c, (uint64_t)c->len + n_steps - 1)))))
        return rc;
    EventPair ev;
    TMG_HIP(ev.create());
    TMG_HIP(hipEventRecord(ev.e0, m->stream));
    for (uint32_t i = 0; i < n_steps; i++)
        if ((rc = launch_step(m, c, SEL_ARGMAX, (uint64_t)c->len + i))) return rc;
    TMG_HIP(hipEventRecord(ev.e1, m->stream));
    TMG_HIP(hipEventSynchronize(ev.e1));
    float el = 0.f;
    TMG_HIP(hipEventElapsedTime(&el, ev.e0, ev.e1));
    c->len += n_steps;
    if (ms) *ms = el;
    if (tokens_out && n_steps) memcpy(tokens_out, (const void *)c->history, (size_t)n_steps * 4);
    return TMG_OK;
}

extern "C" int tmg_profile_decode_step(tmg_model *m, tmg_cache *c, uint32_t token, tmg_kernel_record *records,
                                       size_t cap, size_t *n_records) {
    clear_error();
    if (!m || !c || c->model != m) return set_error(TMG_E_INVALID, "bad model/cache handle");
    if (token >= (uint32_t)m->V) return set_error(TMG_E_INVALID, "token id out of range");
    if (c->len >= c->max_pos) return set_error(TMG_E_CAPACITY, "KV cache full");
    (void)hipSetDevice(m->device);
    int rc;
    // the kernels of one step, in launch order
    FormGuard form(c);
    LaunchRecorder all;
    all.none = true;
    if ((rc = enqueue_decode_step(m, c, &all, SEL_ARGMAX))) return rc;
    std::vector<std::string> kinds;
    for (auto &n : all.names)
        if (std::find(kinds.begin(), kinds.end(), n) == kinds.end()) kinds.push_back(n);
    // each kind: its launches of one step captured as a graph, replayed back
    // to back between two events (kernels abut as in the step graph)
    constexpr int kReps = 8;
    size_t nrec = 0;
    EventPair ev;
    TMG_HIP(ev.create());
    hipEvent_t e0 = ev.e0, e1 = ev.e1;
    // TMG_DECODE_GRAPH=0: the same launches enqueued one by one (profilers
    // that do not follow graph launches)
    const bool use_graph = step_graphs_enabled();
    for (auto &kind : kinds) {
        if ((rc = set_state(m, c, (int)token, true))) break;
        int count = 0;  // launches of this kind in one step
        double bytes = 0.0;
        for (size_t i = 0; i < all.names.size(); i++)
            if (all.names[i] == kind) {
                count++;
                bytes = all.bytes[i];
            }
        // kinds launched once or a few times per step are repeated so that one
        // replay holds at least as many launches as a per-layer kind
        const int inner = std::max(1, m->L / std::max(count, 1));
        auto enqueue = [&]() -> int {
            int r = TMG_OK;
            for (int i = 0; i < inner && !r; i++) {
                LaunchRecorder one;
                one.only = kind.c_str();
                r = enqueue_decode_step(m, c, &one, SEL_ARGMAX);
            }
            return r;
        };
        hipGraphExec_t ex = nullptr;
        if (use_graph) {
            TMG_HIP(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
            rc = enqueue();
            hipGraph_t g = nullptr;
            hipError_t e = hipStreamEndCapture(m->stream, &g);
            if (!rc && e == hipSuccess) e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
            if (g) (void)hipGraphDestroy(g);
            if (rc) break;
            TMG_HIP(e);
        }
        // destroys the replay graph on every path out of this iteration,
        // after the replays queued on the stream
        struct ExecGuard {
            hipGraphExec_t &x;
            hipStream_t s;
            ~ExecGuard() {
                if (x) {
                    (void)hipStreamSynchronize(s);
                    (void)hipGraphExecDestroy(x);
                }
                x = nullptr;
            }
        } guard{ex, m->stream};
        auto replay = [&]() -> int {
            if (use_graph)
                return hipGraphLaunch(ex, m->stream) == hipSuccess ? TMG_OK
                                                                   : set_error(TMG_E_DEVICE, "graph launch failed");
            return enqueue();
        };
        float el = 0.f;
        if (!(rc = replay())) {  // warm
            TMG_HIP(hipEventRecord(e0, m->stream));
            for (int r = 0; r < kReps && !rc; r++) rc = replay();
            TMG_HIP(hipEventRecord(e1, m->stream));
            TMG_HIP(hipEventSynchronize(e1));
            TMG_HIP(hipEventElapsedTime(&el, e0, e1));
        }
        if (rc) break;
        if (nrec < cap && records) {
            tmg_kernel_record r{};
            snprintf(r.name, sizeof(r.name), "%s", kind.c_str());
            r.bytes = bytes;
            r.ms = el / (float)(kReps * inner * count);
            r.launches = count;
            records[nrec] = r;
        }
        nrec++;
    }
    // the replays touched only scratch, the KV row at the current position
    // (rewritten by the next step) and the step state, restored here
    if (!rc) rc = set_state(m, c, (int)token, true);
    if (!rc && hipStreamSynchronize(m->stream) != hipSuccess) rc = set_error(TMG_E_DEVICE, "stream sync failed");
    if (n_records) *n_records = std::min(nrec, cap);
    return rc;
}
