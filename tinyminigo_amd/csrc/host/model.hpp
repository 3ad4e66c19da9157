// Device-resident model and KV cache.
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <mutex>
#include <vector>

#include "../kernels/kernels.hpp"
#include "common.hpp"

struct tmg_model {
    tmg_config cfg{};
    int device = 0;
    hipStream_t stream = nullptr;
    int H = 0, L = 0, nq = 0, nkv = 0, hd = 0, I = 0, V = 0, qd = 0, kvd = 0, qkv_rows = 0;

    struct Layer {
        uint16_t *qkv = nullptr;   // [qkv_rows, H]: rows (j, j+hd/2) of every q/k/v head adjacent
        uint16_t *o = nullptr;     // [H, qd]
        uint16_t *gu = nullptr;    // [2I, H]: gate row p at 2p, up row p at 2p+1
        uint16_t *down = nullptr;  // [H, I]
        float *in_norm = nullptr, *post_norm = nullptr;  // [H]
        // int8 mode: the same four matrices as int8 rows plus f32 row scales
        // (then qkv/o/gu/down above hold the int8 codes as BF16, for prefill)
        int8_t *qkv8 = nullptr, *o8 = nullptr, *gu8 = nullptr, *down8 = nullptr;
        float *qkv_s = nullptr, *o_s = nullptr, *gu_s = nullptr, *down_s = nullptr;
        // f32 rows in the same order instead of the BF16 ones (WMat::F32: a
        // matrix whose file tensors are not all BF16, src/model.rs:49-55);
        // then the BF16 pointer is null
        float *qkv_f = nullptr, *o_f = nullptr, *gu_f = nullptr, *down_f = nullptr;
    };
    // int8 weight-only mode (TMG_I8=1 at load, reference src/model.rs:57-76)
    bool i8 = false;
    // loaded from a TMB1 file
    bool from_tmb = false;
    std::vector<Layer> layers;
    float *final_norm = nullptr;
    uint16_t *embed_bf16 = nullptr;  // [V, H] when the file stores BF16
    float *embed_f32 = nullptr;      // [V, H] otherwise (converted like the reference)
    uint16_t *lm_head = nullptr;     // [V, H]; the embedding when tied
    float *lm_head_f = nullptr;      // f32 lm_head instead (F32/F16 tensor, or tied to an f32 table)
    bool any_f32 = false;            // some layer matrix or the lm_head has f32 rows

    // RoPE cos/sin tables [npos][hd/2], built on the host with libm exactly
    // like the reference's Rope (src/tensor.rs:1005-1023) and uploaded.
    float *rope_cos = nullptr, *rope_sin = nullptr;
    int rope_npos = 0;

    // decode scratch
    float *x = nullptr, *q = nullptr, *attn_out = nullptr, *h = nullptr, *logits = nullptr;
    float *attn_part = nullptr, *attn_ml = nullptr;  // split-K partials (up to kMaxSplits)
    unsigned long long *argmax_part = nullptr;       // per-workgroup argmax keys of the lm_head
    int argmax_nparts = 0;

    // prefill scratch, grown on demand
    int pf_cap = 0;
    int *pf_tokens = nullptr;
    float *pf_x = nullptr, *pf_q = nullptr;
    uint16_t *pf_hi = nullptr, *pf_lo = nullptr, *pf_ahi = nullptr, *pf_alo = nullptr, *pf_hhi = nullptr,
             *pf_hlo = nullptr;
    // split-K partial tiles and arrival counters of the short-prompt GEMM
    float *pf_part = nullptr;
    float *pf_nss = nullptr;  // per-64-row sums of squares of the residual handed to the next GEMM
    unsigned *pf_cnt = nullptr;
    // split-bf16 KV rows for the MFMA prefill attention (rows [0, kv_cap))
    int kv_cap = 0;
    uint16_t *pf_kh = nullptr, *pf_kl = nullptr, *pf_vth = nullptr, *pf_vtl = nullptr;

    // pinned host staging
    void *pin = nullptr;
    size_t pin_bytes = 0;

    std::vector<void *> allocs;

    // Caches created on this model and not yet freed.  tmg_model_free with
    // live caches only marks the model; the last tmg_cache_free releases it
    // (a cache uses the model's stream, device and weights until it is freed).
    // Both fields change under life_mu, so frees on different threads
    // release the model exactly once.
    std::mutex life_mu;
    int live_caches = 0;
    bool free_requested = false;
};

struct tmg_cache {
    tmg_model *model = nullptr;
    uint32_t max_pos = 0;
    float *k = nullptr, *v = nullptr;  // [L][max_pos][kvd]
    tmg::DevState *st = nullptr;       // device
    // generated ids, max_pos + 2 entries, in coherent pinned host memory that
    // the kernels write directly (the host reads a token as soon as the step
    // that wrote it has completed; no copy per step)
    int *history = nullptr;
    uint32_t len = 0;                  // host mirror of st->pos
    int attn_nsplit = 1;               // split-K width of decode attention for this cache
    int attn_block = tmg::kAttnBlockLong;  // positions per block of its split partition
    unsigned *seen = nullptr;          // bitmap of generated ids (repetition penalty)
    unsigned long long *cand = nullptr;  // sampler candidates
    float *draws = nullptr;              // [max_pos + 2] uniform draw per step (sampling)
    float *gsc = nullptr;                // kSampleScratchBytes(V) of the whole-vocabulary sampler
    int samp_use_k = 0, samp_use_p = 0;  // the running generate call's top-k / nucleus
    // one captured step graph per token-selection mode (tmg::SelectMode) and
    // attention form: [1] where every split is active (long contexts of
    // caches with more than kSpecSplits splits), every split loads its first
    // block before the position read; [0] otherwise
    hipGraphExec_t graphs[2][4] = {};
    hipGraph_t graph_src[2][4] = {};
    bool capture_spec_all = false;  // set while [1] is being captured
};

namespace tmg {

// Decode attention: the context is dealt to the splits in blocks of
// attn_block positions; a cache of max_pos rows uses up to
// ceil(max_pos / attn_block) splits (at most kMaxSplits).  Up to kFusedSplits
// the merge runs in the o_proj prologue, above in attn_combine_kernel.
constexpr int kMaxSplits = 32;
// Sequences per tmg_generate_batch call (the short-prompt GEMM takes up to
// 255 token rows; the bound keeps the per-call KV allocation in view).
constexpr int kMaxBatch = 128;

// Launch filter used by tmg_profile_decode_step: every kernel of the step is
// announced with its name and algorithmic bytes; when `only` is set, just the
// kernels of that name are launched (to time them back to back in a graph).
struct LaunchRecorder {
    const char *only = nullptr;
    bool none = false;  // announce only, launch nothing
    std::vector<std::string> names;
    std::vector<double> bytes;
    bool want(const char *name, double b);
};

// How a step turns logits into the next token.
// Two timing events, destroyed on every return path.
struct EventPair {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t create() {
        hipError_t e = hipEventCreate(&e0);
        return e == hipSuccess ? hipEventCreate(&e1) : e;
    }
    ~EventPair() {
        if (e0) (void)hipEventDestroy(e0);
        if (e1) (void)hipEventDestroy(e1);
    }
};

enum SelectMode {
    SEL_ARGMAX = 0,          // greedy, argmax fused into the lm_head GEMV
    SEL_PENALTY_ARGMAX = 1,  // greedy after the repetition penalty
    SEL_TOPK = 2,            // temperature sampling with 0 < top_k <= kSampleMaxK
    SEL_FULL = 3,            // temperature sampling, any other top_k / top_p
};

int enqueue_decode_step(tmg_model *m, tmg_cache *c, LaunchRecorder *rec, int mode);
int enqueue_select(tmg_model *m, tmg_cache *c, int mode, int advance_pos);
// The attention form of a step writing position pos (1: every split active
// on a cache with more than kSpecSplits splits).
int step_form(const tmg_cache *c, uint64_t pos);
int get_step_graph(tmg_model *m, tmg_cache *c, int mode, int form);
// For its lifetime, steps enqueued directly (measurement captures) take the
// attention form of a step at the cache's position.
struct FormGuard {
    tmg_cache *c;
    explicit FormGuard(tmg_cache *c_) : c(c_) { c->capture_spec_all = step_form(c, c->len) == 1; }
    ~FormGuard() { c->capture_spec_all = false; }
    FormGuard(const FormGuard &) = delete;
    FormGuard &operator=(const FormGuard &) = delete;
};
// One decode step writing position pos on the model's stream: the cache's
// captured graph for `mode` and the step's attention form, or
// (TMG_DECODE_GRAPH=0) the same kernels launched one by one.
bool step_graphs_enabled();
int launch_step(tmg_model *m, tmg_cache *c, int mode, uint64_t pos);
int set_state(tmg_model *m, tmg_cache *c, int token, bool reset_step);
int run_prefill(tmg_model *m, tmg_cache *c, const uint32_t *tokens, size_t n);
int ensure_rope(tmg_model *m, int npos);
int pinned(tmg_model *m, size_t bytes);

}  // namespace tmg
