// tmg_profile_step_floor: the decode step next to its floor on the same
// device, cache and position (measurement only; no counterpart in the
// reference).  The step is captured as the decode loop captures it; its
// kernel nodes, read back from the captured graph in chain order, give each
// launch's grid, and the launch record gives its algorithmic bytes.  The
// floor chain replaces every launch by a streaming phase (floor.hip) with
// the same grid and the same bytes (to whole 4-KiB blocks per workgroup),
// all of a workgroup's loads in flight at once, read from a weight slab of its
// own that is larger than the last-level cache, so each replay streams from
// HBM as the step does.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <string>
#include <vector>

#include "model.hpp"

namespace tmg {
namespace {

#define TMG_HIPF(expr)                                                                                      \
    do {                                                                                                    \
        hipError_t e_ = (expr);                                                                             \
        if (e_ != hipSuccess)                                                                               \
            return set_error(TMG_E_DEVICE, std::string("HIP error ") + hipGetErrorString(e_) + " in " #expr \
                                               " (" __FILE__ ":" + std::to_string(__LINE__) + ")");         \
    } while (0)

constexpr int kReps = 8;          // timed replays of each graph
constexpr int kEmptyLaunches = 240;
constexpr size_t kBlockBytes = 4096;
constexpr int kMaxNb = 32;        // blocks per chunk of a streaming phase

struct Phase {
    std::string name;
    double bytes = 0.0;  // algorithmic bytes of the kernel it stands for
    int nwg = 0, nb = 0, nchunk = 0;
    size_t off = 0;      // into the weight slab
    size_t floor_bytes() const { return (size_t)nwg * nb * nchunk * kBlockBytes; }
};

// Device buffers and graphs of one call, released on every path out.
struct Scope {
    std::vector<void *> mem;
    std::vector<hipGraph_t> graphs;
    std::vector<hipGraphExec_t> execs;
    ~Scope() {
        // replays enqueued before an early return finish before their
        // graphs and buffers go
        if (!mem.empty() || !execs.empty()) (void)hipDeviceSynchronize();
        for (auto x : execs) (void)hipGraphExecDestroy(x);
        for (auto g : graphs) (void)hipGraphDestroy(g);
        for (auto p : mem) (void)hipFree(p);
    }
};

int alloc(Scope &sc, void **p, size_t bytes) {
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess)
        return set_error(TMG_E_NOMEM, std::string("hipMalloc of ") + std::to_string(bytes) +
                                          " bytes failed: " + hipGetErrorString(e));
    sc.mem.push_back(*p);
    return TMG_OK;
}

// Captures what `enqueue` launches on the model's stream into an
// instantiated graph (kept in sc); `graph_out` receives the graph itself.
template <class F>
int capture(tmg_model *m, Scope &sc, F &&enqueue, hipGraphExec_t *ex, hipGraph_t *graph_out = nullptr) {
    TMG_HIPF(hipStreamBeginCapture(m->stream, hipStreamCaptureModeThreadLocal));
    const int rc = enqueue();
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(m->stream, &g);
    if (g) sc.graphs.push_back(g);
    if (rc) return rc;
    TMG_HIPF(e);
    TMG_HIPF(hipGraphInstantiate(ex, g, nullptr, nullptr, 0));
    sc.execs.push_back(*ex);
    if (graph_out) *graph_out = g;
    return TMG_OK;
}

// Average ms of one replay of ex over kReps back-to-back replays (after one
// untimed replay); `before` runs before each replay is enqueued.
template <class F>
int time_replays(tmg_model *m, hipGraphExec_t ex, F &&before, float *ms) {
    EventPair ev;
    TMG_HIPF(ev.create());
    int rc;
    if ((rc = before())) return rc;
    TMG_HIPF(hipGraphLaunch(ex, m->stream));
    TMG_HIPF(hipEventRecord(ev.e0, m->stream));
    for (int r = 0; r < kReps; r++) {
        if ((rc = before())) return rc;
        TMG_HIPF(hipGraphLaunch(ex, m->stream));
    }
    TMG_HIPF(hipEventRecord(ev.e1, m->stream));
    TMG_HIPF(hipEventSynchronize(ev.e1));
    float el = 0.0f;
    TMG_HIPF(hipEventElapsedTime(&el, ev.e0, ev.e1));
    *ms = el / kReps;
    return TMG_OK;
}

// The kernel nodes of a captured single-stream graph, in chain order.
int chain_kernels(hipGraph_t g, std::vector<hipKernelNodeParams> *out) {
    size_t nr = 0;
    TMG_HIPF(hipGraphGetRootNodes(g, nullptr, &nr));
    if (nr != 1) return set_error(TMG_E_DEVICE, "captured step is not a single chain");
    hipGraphNode_t cur = nullptr;
    TMG_HIPF(hipGraphGetRootNodes(g, &cur, &nr));
    while (cur) {
        hipGraphNodeType ty;
        TMG_HIPF(hipGraphNodeGetType(cur, &ty));
        if (ty != hipGraphNodeTypeKernel) return set_error(TMG_E_DEVICE, "captured step holds a non-kernel node");
        hipKernelNodeParams kp{};
        TMG_HIPF(hipGraphKernelNodeGetParams(cur, &kp));
        out->push_back(kp);
        size_t nd = 0;
        TMG_HIPF(hipGraphNodeGetDependentNodes(cur, nullptr, &nd));
        if (nd > 1) return set_error(TMG_E_DEVICE, "captured step is not a single chain");
        hipGraphNode_t next = nullptr;
        if (nd == 1) TMG_HIPF(hipGraphNodeGetDependentNodes(cur, &next, &nd));
        cur = next;
    }
    return TMG_OK;
}

}  // namespace
}  // namespace tmg

using namespace tmg;

extern "C" int tmg_profile_step_floor(tmg_model *m, tmg_cache *c, uint32_t token, tmg_floor_record *records,
                                      size_t cap, size_t *n_records, float *step_ms, float *floor_ms,
                                      float *empty_ms) {
    clear_error();
    if (n_records) *n_records = 0;
    if (!m || !c || c->model != m) return set_error(TMG_E_INVALID, "bad model/cache handle");
    if (token >= (uint32_t)m->V) return set_error(TMG_E_INVALID, "token id out of range");
    // every replay of the step advances the position by one
    if ((size_t)c->len + kReps + 1 >= c->max_pos) return set_error(TMG_E_CAPACITY, "KV cache too short for the replays");
    (void)hipSetDevice(m->device);
    int rc;
    Scope sc;

    // the step as the decode loop captures it (greedy selection, the
    // attention form of a step at the cache's position)
    FormGuard form(c);
    if ((rc = set_state(m, c, (int)token, true))) return rc;
    LaunchRecorder rec;
    hipGraphExec_t step_ex = nullptr;
    hipGraph_t step_g = nullptr;
    if ((rc = capture(m, sc, [&] { return enqueue_decode_step(m, c, &rec, SEL_ARGMAX); }, &step_ex, &step_g)))
        return rc;
    std::vector<hipKernelNodeParams> nodes;
    if ((rc = chain_kernels(step_g, &nodes))) return rc;
    if (nodes.size() != rec.names.size())
        return set_error(TMG_E_DEVICE, "captured step and launch record disagree (" + std::to_string(nodes.size()) +
                                           " kernels, " + std::to_string(rec.names.size()) + " records)");
    // consecutive steps from the cache's position, as the decode loop runs
    // them; the rows they append lie past the cache's length
    float t_step = 0.0f;
    rc = time_replays(m, step_ex, [] { return TMG_OK; }, &t_step);
    const int rs = set_state(m, c, (int)token, true);
    if (rc || rs) return rc ? rc : rs;

    // one streaming phase per launch, with its grid and bytes
    std::vector<Phase> ph(nodes.size());
    size_t slab = 0;
    int max_wg = 2048;
    for (size_t i = 0; i < nodes.size(); i++) {
        const dim3 g = nodes[i].gridDim;
        Phase &p = ph[i];
        p.name = rec.names[i];
        p.bytes = rec.bytes[i];
        p.nwg = (int)(g.x * g.y * g.z);
        // the launch's bytes to the nearest whole block per workgroup (a
        // GEMV workgroup's rows are whole blocks; the activation and output
        // bytes in the algorithmic count add a fraction of one)
        const double per_wg = p.bytes / std::max(p.nwg, 1);
        const int nblk = std::max(1, (int)std::lround(per_wg / (double)kBlockBytes));
        p.nchunk = (nblk + kMaxNb - 1) / kMaxNb;
        p.nb = (nblk + p.nchunk - 1) / p.nchunk;
        p.off = slab;
        slab += p.floor_bytes();
        max_wg = std::max(max_wg, p.nwg);
    }
    void *w = nullptr, *act0 = nullptr, *buf[2] = {nullptr, nullptr};
    if ((rc = alloc(sc, &w, slab)) || (rc = alloc(sc, &act0, 2048 * 4)) ||
        (rc = alloc(sc, &buf[0], (size_t)max_wg * 4)) || (rc = alloc(sc, &buf[1], (size_t)max_wg * 4)))
        return rc;
    TMG_HIPF(hipMemsetAsync(w, 0, slab, m->stream));
    TMG_HIPF(hipMemsetAsync(act0, 0, 2048 * 4, m->stream));
    TMG_HIPF(hipMemsetAsync(buf[0], 0, (size_t)max_wg * 4, m->stream));
    TMG_HIPF(hipMemsetAsync(buf[1], 0, (size_t)max_wg * 4, m->stream));
    TMG_HIPF(hipStreamSynchronize(m->stream));

    // phases in order; phase k of the sequence reads the output of phase k-1
    auto launch_seq = [&](const std::vector<size_t> &idx) -> int {
        for (size_t k = 0; k < idx.size(); k++) {
            const Phase &p = ph[idx[k]];
            const float *act = k == 0 ? (const float *)act0 : (const float *)buf[(k - 1) & 1];
            TMG_HIPF(launch_stream_phase((const char *)w + p.off, p.nwg, p.nb, p.nchunk, act, (float *)buf[k & 1],
                                         m->stream));
        }
        return TMG_OK;
    };
    auto nothing = [] { return TMG_OK; };

    std::vector<size_t> all(ph.size());
    for (size_t i = 0; i < ph.size(); i++) all[i] = i;
    hipGraphExec_t floor_ex = nullptr;
    if ((rc = capture(m, sc, [&] { return launch_seq(all); }, &floor_ex))) return rc;
    float t_floor = 0.0f;
    if ((rc = time_replays(m, floor_ex, nothing, &t_floor))) return rc;

    // each kind's phases back to back (repeated like tmg_profile_decode_step
    // repeats a kind launched a few times per step)
    std::vector<std::string> kinds;
    for (auto &p : ph)
        if (std::find(kinds.begin(), kinds.end(), p.name) == kinds.end()) kinds.push_back(p.name);
    size_t nrec = 0;
    for (auto &kind : kinds) {
        std::vector<size_t> one;
        for (size_t i = 0; i < ph.size(); i++)
            if (ph[i].name == kind) one.push_back(i);
        const int count = (int)one.size();
        const int inner = std::max(1, m->L / count);
        std::vector<size_t> seq;
        for (int r = 0; r < inner; r++) seq.insert(seq.end(), one.begin(), one.end());
        hipGraphExec_t ex = nullptr;
        if ((rc = capture(m, sc, [&] { return launch_seq(seq); }, &ex))) return rc;
        float t = 0.0f;
        if ((rc = time_replays(m, ex, nothing, &t))) return rc;
        if (records && nrec < cap) {
            const Phase &p = ph[one[0]];
            tmg_floor_record r{};
            snprintf(r.name, sizeof(r.name), "%s", kind.c_str());
            r.bytes = p.bytes;
            r.floor_bytes = (double)p.floor_bytes();
            r.floor_ms = t / (float)seq.size();
            r.launches = (uint32_t)count;
            r.workgroups = (uint32_t)p.nwg;
            records[nrec] = r;
        }
        nrec++;
    }

    // the launch cost alone: empty 256-workgroup kernels back to back
    hipGraphExec_t empty_ex = nullptr;
    if ((rc = capture(m, sc, [&]() -> int {
             for (int i = 0; i < kEmptyLaunches; i++) TMG_HIPF(launch_empty(256, m->stream));
             return TMG_OK;
         }, &empty_ex)))
        return rc;
    float t_empty = 0.0f;
    if ((rc = time_replays(m, empty_ex, nothing, &t_empty))) return rc;

    if (step_ms) *step_ms = t_step;
    if (floor_ms) *floor_ms = t_floor;
    if (empty_ms) *empty_ms = t_empty / kEmptyLaunches;
    if (n_records) *n_records = std::min(nrec, cap);
    TMG_HIPF(hipStreamSynchronize(m->stream));
    return TMG_OK;
}

extern "C" int tmg_profile_stream(size_t bytes, uint32_t wg_kib, int device, float *us, size_t *bytes_read) {
    clear_error();
    if (bytes == 0 || wg_kib < 4 || wg_kib > 4 * kMaxNb || wg_kib % 4)
        return set_error(TMG_E_INVALID, "tmg_profile_stream: bytes > 0 and wg_kib a multiple of 4 in [4, 128]");
    if (hipSetDevice(device) != hipSuccess) return set_error(TMG_E_DEVICE, "no such device");
    const int nb = (int)(wg_kib / 4);
    const size_t wg_bytes = (size_t)nb * kBlockBytes;
    const size_t nwg = (bytes + wg_bytes - 1) / wg_bytes;
    if (nwg > (size_t)1 << 24) return set_error(TMG_E_INVALID, "tmg_profile_stream: too many workgroups");
    const size_t each = nwg * wg_bytes;
    // enough copies that a replay streams more than the last-level cache
    // holds several times over: none is still cached when its turn comes
    const size_t ncopy = std::max<size_t>(4, ((size_t)1 << 30) / each + 1);
    int rc;
    Scope sc;
    hipStream_t s = nullptr;
    TMG_HIPF(hipStreamCreate(&s));
    struct StreamGuard {
        hipStream_t s;
        ~StreamGuard() { (void)hipStreamDestroy(s); }
    } sg{s};
    void *w = nullptr, *act = nullptr, *out = nullptr;
    const size_t nout = std::max<size_t>(nwg, 2048);
    if ((rc = alloc(sc, &w, ncopy * each)) || (rc = alloc(sc, &act, 2048 * 4)) || (rc = alloc(sc, &out, nout * 4)))
        return rc;
    TMG_HIPF(hipMemsetAsync(w, 0, ncopy * each, s));
    TMG_HIPF(hipMemsetAsync(act, 0, 2048 * 4, s));
    TMG_HIPF(hipStreamSynchronize(s));
    hipGraphExec_t ex = nullptr;
    {
        TMG_HIPF(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        hipError_t le = hipSuccess;
        for (size_t i = 0; i < ncopy && le == hipSuccess; i++)
            le = launch_stream_phase((const char *)w + i * each, (int)nwg, nb, 1, (const float *)act, (float *)out, s);
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamEndCapture(s, &g);
        if (g) sc.graphs.push_back(g);
        TMG_HIPF(le);
        TMG_HIPF(e);
        TMG_HIPF(hipGraphInstantiate(&ex, g, nullptr, nullptr, 0));
        sc.execs.push_back(ex);
    }
    EventPair ev;
    TMG_HIPF(ev.create());
    const int reps = (int)std::max<size_t>(3, 2000 / ncopy);
    TMG_HIPF(hipGraphLaunch(ex, s));
    TMG_HIPF(hipEventRecord(ev.e0, s));
    for (int r = 0; r < reps; r++) TMG_HIPF(hipGraphLaunch(ex, s));
    TMG_HIPF(hipEventRecord(ev.e1, s));
    TMG_HIPF(hipEventSynchronize(ev.e1));
    float el = 0.0f;
    TMG_HIPF(hipEventElapsedTime(&el, ev.e0, ev.e1));
    if (us) *us = el * 1e3f / (float)(reps * ncopy);
    if (bytes_read) *bytes_read = each;
    return TMG_OK;
}
