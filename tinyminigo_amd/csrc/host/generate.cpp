// generate (reference src/model.rs:614-663) on the device-resident step.
//
// The reference loop is: prefill -> for each of max_tokens: (penalty) ->
// argmax or sample -> on_token -> push -> EOS check -> forward_token.  Here
// the selection runs on the GPU at the end of every captured step graph, so
// the host only reads back the chosen id (4 bytes) for on_token and the EOS
// check.  Up to kWindow steps are enqueued ahead of the host: every step's
// input token is produced on the device by the previous step, so running
// ahead computes exactly what the host would have submitted.  Steps enqueued
// past an EOS only touch generate's private KV cache, which is discarded,
// as the reference discards its own (src/model.rs:620-621).
#include <chrono>
#include <cstring>
#include <vector>

#include "model.hpp"

namespace tmg {
namespace {

constexpr int kWindow = 4;

struct CacheGuard {
    tmg_cache *c = nullptr;
    ~CacheGuard() { tmg_cache_free(c); }
};

struct EventRing {
    std::vector<hipEvent_t> ev;
    ~EventRing() {
        for (auto e : ev) (void)hipEventDestroy(e);
    }
};

}  // namespace
}  // namespace tmg

using namespace tmg;

#define TMG_HIPG(expr)                                                                                     \
    do {                                                                                                   \
        hipError_t e_ = (expr);                                                                            \
        if (e_ != hipSuccess) return set_error(TMG_E_DEVICE, std::string("HIP error ") + hipGetErrorString(e_) + " in " #expr); \
    } while (0)

extern "C" int tmg_generate(tmg_model *m, const uint32_t *prompt, size_t n_prompt, const tmg_gen_params *p,
                            tmg_on_token_fn on_token, void *user, uint32_t *out_tokens, size_t out_cap, size_t *n_out,
                            float *first_logits, float *prefill_secs) {
    clear_error();
    if (n_out) *n_out = 0;
    if (!m || !p || (!prompt && n_prompt)) return set_error(TMG_E_INVALID, "bad argument to tmg_generate");
    if (n_prompt == 0) return set_error(TMG_E_EMPTY, "empty prompt");
    if (!out_tokens || out_cap < p->max_tokens) return set_error(TMG_E_INVALID, "out_tokens capacity below max_tokens");
    for (size_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= (uint32_t)m->V) return set_error(TMG_E_INVALID, "prompt token id out of range");

    // token-selection mode (src/model.rs:632-646; top_k is effective only when
    // 0 < k < vocab, src/tensor.rs:1172)
    const bool greedy = p->temperature <= 0.0f;
    const bool use_k = p->top_k > 0 && p->top_k < (uint32_t)m->V;
    int mode;
    if (greedy) {
        mode = p->repetition_penalty != 1.0f ? SEL_PENALTY_ARGMAX : SEL_ARGMAX;
    } else {
        // small k: per-slice candidate lists; no k or a larger one: threshold
        // searches over the whole vocabulary
        mode = use_k && p->top_k <= (uint32_t)kSampleMaxK ? SEL_TOPK : SEL_FULL;
    }
    if ((size_t)m->V > (size_t)kSampleMaxVocab && mode != SEL_ARGMAX)
        return set_error(TMG_E_INVALID, "vocabulary too large for the device sampler");

    (void)hipSetDevice(m->device);
    CacheGuard cg;
    const size_t max_pos = n_prompt + (size_t)p->max_tokens + 1;
    if (max_pos > 0x7fffffff) return set_error(TMG_E_INVALID, "sequence too long");
    int rc = tmg_cache_new(m, (uint32_t)max_pos, &cg.c);
    if (rc) return rc;
    tmg_cache *c = cg.c;

    // sampling parameters live in the device state read by the sampler
    DevState st{};
    st.pos = 0;
    st.cur_token = 0;
    st.step = 0;
    st.argmax_key = kArgmaxInit;
    st.temperature = p->temperature;
    st.top_k = use_k ? (int)p->top_k : 0;
    st.top_p = p->top_p;
    st.penalty = p->repetition_penalty;
    TMG_HIPG(hipMemcpy(c->st, &st, sizeof(st), hipMemcpyHostToDevice));
    c->samp_use_k = use_k;
    c->samp_use_p = p->top_p < 1.0f;
    if (!greedy && p->max_tokens > 0) {
        // the reference's StdRng::seed_from_u64(seed) stream: one
        // StandardUniform f32 per sampled step (src/model.rs:629,
        // src/tensor.rs:1204)
        std::vector<float> draws(p->max_tokens);
        stdrng_uniform(p->seed, draws.size(), draws.data());
        TMG_HIPG(hipMemcpy(c->draws, draws.data(), draws.size() * 4, hipMemcpyHostToDevice));
    }
    // step j writes position n_prompt + j: the graphs of the first and the
    // last step's attention forms
    if (step_graphs_enabled() &&
        ((rc = get_step_graph(m, c, mode, step_form(c, n_prompt))) ||
         (p->max_tokens > 0 && (rc = get_step_graph(m, c, mode, step_form(c, n_prompt + p->max_tokens - 1))))))
        return rc;

    // prefill (timed like the reference, src/model.rs:622-624)
    auto t0 = std::chrono::steady_clock::now();
    if ((rc = run_prefill(m, c, prompt, n_prompt))) return rc;
    TMG_HIPG(hipStreamSynchronize(m->stream));
    auto t1 = std::chrono::steady_clock::now();
    if (prefill_secs) *prefill_secs = std::chrono::duration<float>(t1 - t0).count();
    if (first_logits) {
        TMG_HIPG(hipMemcpy(first_logits, m->logits, (size_t)m->V * 4, hipMemcpyDeviceToHost));
    }

    const size_t max_tokens = p->max_tokens;
    if (max_tokens == 0) return TMG_OK;
    // the kernels write each id into c->history (coherent pinned host memory)
    const volatile int *host_tok = c->history;
    EventRing ring;
    ring.ev.resize(kWindow + 1);
    for (auto &e : ring.ev) TMG_HIPG(hipEventCreateWithFlags(&e, hipEventDisableTiming));

    // token 0 comes from the prefill logits (src/model.rs:623-646)
    if ((rc = enqueue_select(m, c, mode, 0))) return rc;
    TMG_HIPG(hipEventRecord(ring.ev[0], m->stream));

    size_t enq = 0;  // forward steps enqueued; step j consumes token j and yields token j+1
    size_t produced = 0;
    for (size_t i = 0; i < max_tokens; i++) {
        while (enq < max_tokens && enq < i + kWindow) {
            if ((rc = launch_step(m, c, mode, n_prompt + enq))) return rc;
            TMG_HIPG(hipEventRecord(ring.ev[(enq + 1) % (kWindow + 1)], m->stream));
            enq++;
        }
        TMG_HIPG(hipEventSynchronize(ring.ev[i % (kWindow + 1)]));
        const uint32_t tok = (uint32_t)host_tok[i];
        out_tokens[i] = tok;
        produced = i + 1;
        if (on_token) on_token(tok, user);
        bool eos = false;
        for (uint32_t e = 0; e < m->cfg.n_eos; e++)
            if (m->cfg.eos_token_ids[e] == tok) eos = true;
        if (eos) break;
    }
    TMG_HIPG(hipStreamSynchronize(m->stream));
    if (n_out) *n_out = produced;
    return TMG_OK;
}
