#!/usr/bin/env python3
"""Decode/prefill benchmark of the TinyMiniGo decode path on one MI355X.

Workload (default): the 1B-class MiniCPM5-shaped synthetic model (hidden
2048, 24 layers, 16/8 heads, head_dim 128, SwiGLU 6144, vocab 73448, untied
lm_head, BF16 N(0, 0.02) weights from seed 3), a 64-token prompt (seed 4),
batched prefill, then greedy decode.  A step is one decode token: the whole
forward_token (24 layers + lm_head) plus the argmax that picks the next id,
replayed from a captured hipGraph with inputs resident in HBM.

    python bench.py [--gpus 1] [--steps 256] [--warmup 16]

Prints ONE JSON line.  `value` = decode tokens/s over the timed steps;
`roofline` = the dominant kernel's algorithmic HBM bytes per launch over its
average launch time (its launches of one step replayed back to back from a
graph between HIP events on the model's stream); `cpu_baseline` = the
CPU oracle (C restatement of the reference Rust path, reference threading)
timed on this host on a bounded sample of the same decode.
"""
import argparse
import json
import os
import platform
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
METRIC = "decode tok/s + % HBM roofline (1B-class bf16, 1 MI355X); prefill tok/s"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(path, prompt, seconds, long_wl=None, gpu_model=None, gpu_cache=None, sampled=None, i8=False):
    """The oracle (the C restatement of the reference CPU path) decoding the
    same model on this host's cores: a prefill of the prompt, then decode
    steps until about `seconds` have passed (at most 256).  For the 8k
    workload the 8192-token CPU prefill (about ten minutes of single-threaded
    attention) is replaced by the device's KV cache copied into the oracle's,
    so the timed steps are CPU decode steps at that context.  With `sampled`
    each step applies the penalty and the reference's sampler; with `i8` the
    oracle runs the reference's int8 weight-only path (TMG_I8=1)."""
    from oracle import oracle as O
    m = O.OracleModel.load(path, i8=i8)
    cache = m.new_cache()
    if long_wl is not None:
        n0 = gpu_cache.total_len()
        for layer in range(long_wl.num_hidden_layers):
            cache.push_rows(layer, gpu_cache.keys_flat(layer), gpu_cache.values_flat(layer))
        logits = m.forward_token(int(prompt[-1]), cache)
        prefill_s = None
        what = f"decode at context {n0 + 1}+ (KV cache of the device prefill copied in)"
    else:
        t0 = time.perf_counter()
        logits = m.prefill(prompt, cache)
        prefill_s = time.perf_counter() - t0
        what = f"after a {len(prompt)}-token prefill ({len(prompt) / prefill_s:.1f} prefill tok/s)"
    generated = []
    n, t0 = 0, time.perf_counter()

    def pick(lg):
        if sampled is None:
            return int(O.argmax(lg))
        if generated:
            lg = O.apply_repetition_penalty(lg, generated, sampled["repetition_penalty"])
        return O.sample(lg, sampled["temperature"], sampled["top_k"], sampled["top_p"], 0.5).token

    tok = pick(logits)
    while True:
        generated.append(tok)
        logits = m.forward_token(tok, cache)
        tok = pick(logits)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 256:
            break
    threads = max(1, O.lib.om_num_threads() // 4)
    mode = "sampled (penalty + top-k/top-p sampler)" if sampled else "greedy"
    return {
        "value": round(n / el, 3), "unit": "tok/s", "cores": threads, "kind": "port",
        "sample": (f"oracle (C restatement of the reference CPU path{', int8 weights' if i8 else ''}, GEMV on "
                   f"max(1,ncores/4)={threads} threads of "
                   f"{os.cpu_count()} on '{cpu_model()}', AVX2={bool(O.lib.om_uses_avx2())}): {n} {mode} decode "
                   f"steps {what}"),
        "prefill_tok_s": round(len(prompt) / prefill_s, 2) if prefill_s else None,
    }


C1_SHAPES = [(2048, 2048), (6144, 2048), (2048, 6144), (73448, 2048)]
MALL_BYTES = 256 << 20  # MI355X last-level (Infinity) cache


# workgroup sizes (KiB per workgroup) the streaming floor is taken over
STREAM_WG_KIB = (8, 12, 16, 24, 32, 48, 64, 96)


def gemv_sweep(T):
    """matmul_w (src/tensor.rs:315-338) at the decode GEMV shapes through the
    kernel-level entry point tmg_gemv_bf16.  W BF16 N(0, 0.02) and x N(0, 1)
    from seed 2.  HBM-cold: the launches of one replay rotate over enough
    copies of W (>= 1 GiB) that none is still in the last-level cache;
    MALL-hot: the same number of launches on one copy.  Bytes per launch =
    2*out*in + 4*in + 4*out; each figure is the per-launch average over
    graph replays (HIP events on the launch stream).  Beside each shape, the
    streaming floor of its weight bytes (tmg_profile_stream, the best of
    STREAM_WG_KIB)."""
    import numpy as np

    from tinyminigo_amd import hip as H
    stream = H.Stream()
    res = []
    for out, inp in C1_SHAPES:
        w = T.synth_normal_bf16(2, f"w{out}x{inp}", out * inp, 0.02)
        x = T.synth_normal_f32(2, f"x{inp}", inp, 1.0)
        wbytes = w.nbytes
        ncopy = max(4, min(128, -(-(4 * MALL_BYTES) // wbytes)))
        w0 = H.DeviceBuffer.from_array(w)
        ws = [w0] + [H.DeviceBuffer(wbytes) for _ in range(ncopy - 1)]
        for b in ws[1:]:
            H.copy_device(b, w0, wbytes)
        xd, yd = H.DeviceBuffer.from_array(x), H.DeviceBuffer(out * 4)
        H.synchronize()
        nbytes = 2 * out * inp + 4 * inp + 4 * out
        row = {"shape": f"{out}x{inp}", "bytes": nbytes, "copies": ncopy}
        # max-abs error of the device result against the oracle's matmul_w
        # (the reference's 8-lane dot order), computed before any timing
        from oracle import oracle as O
        T.gemv_bf16(w0.addr, xd.addr, yd.addr, out, inp, stream.addr)
        stream.synchronize()
        y = yd.to_array(np.float32, out)
        ref = O.matmul_w(x, w, out, inp)
        row["max_abs_err"] = float(np.abs(y.astype(np.float64) - ref.astype(np.float64)).max())
        for kind, pick in (("cold", lambda i: ws[i]), ("hot", lambda i: w0)):
            g = H.Graph(stream, lambda st: [T.gemv_bf16(pick(i).addr, xd.addr, yd.addr, out, inp, st.addr)
                                            for i in range(ncopy)])
            g.launch()
            stream.synchronize()
            reps = max(3, 2000 // ncopy)
            tm = H.Timer(stream)
            tm.start()
            for _ in range(reps):
                g.launch()
            us = tm.stop() * 1e3 / (reps * ncopy)
            row[f"{kind}_us"] = round(us, 3)
            row[f"{kind}_GB_s"] = round(nbytes / (us * 1e-6) / 1e9, 1)
            del g
        del ws, w0, xd, yd
        # the floor: a kernel that only streams the same weight bytes,
        # HBM-cold, at the best of several workgroup sizes
        fl = min((T.profile_stream(wbytes, kib)[0], kib) for kib in STREAM_WG_KIB)
        row["stream_floor_us"], row["stream_floor_wg_kib"] = round(fl[0], 3), fl[1]
        row["cold_above_floor_us"] = round(row["cold_us"] - fl[0], 3)
        res.append(row)
        log(f"gemv {out}x{inp}: cold {row['cold_us']} us ({row['cold_GB_s']} GB/s), "
            f"hot {row['hot_us']} us ({row['hot_GB_s']} GB/s), streaming floor {fl[0]:.3f} us, "
            f"max abs err vs oracle {row['max_abs_err']:.2e}")
    return res


TRAFFIC_FILES = {w: os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f)
                 for w, f in (("bf16", "decode_1b_gemv_traffic.md"), ("i8", "decode_1b_i8_gemv_traffic.md"))}


def summary_line(path, tag, kernel):
    """The `tag: kernel=... key=value ...` line of a committed profile summary
    for `kernel`, as a dict, or None."""
    try:
        for line in open(path):
            if line.startswith(tag + ":"):
                f = dict(kv.split("=", 1) for kv in line.split(":", 1)[1].split())
                if f.get("kernel") == kernel:
                    return f
    except OSError:
        pass
    return None


def pmc_traffic(kernel, weights="bf16"):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC
    summary (FETCH_SIZE + WRITE_SIZE, scaled by a copy kernel of known size)
    and the commit of the tree it was measured on; (None, None) when the
    summary has no line for it."""
    f = summary_line(TRAFFIC_FILES[weights], "traffic-bytes-per-launch", kernel)
    return (int(f["bytes"]), f.get("tree")) if f else (None, None)


STATS_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "decode_1b_kernel_stats.md")


def rocprof_avg(kernel):
    """The rocprofv3 --kernel-trace --stats average duration (us) of `kernel`
    in the committed 1B decode summary, and its tree; (None, None) if absent."""
    f = summary_line(STATS_FILE, "rocprof-avg-us", kernel)
    return (float(f["us"]), f.get("tree")) if f else (None, None)


SAMPLED = dict(temperature=0.8, top_k=50, top_p=0.9, repetition_penalty=1.1, seed=42)


def kernel_table(m, cache, tok, reps=3):
    """Per-kernel-kind timing of one decode step at the cache's position:
    {name: (launches per step, algorithmic bytes per launch, ms per launch)}."""
    import numpy as np
    per = {}
    for _ in range(reps):
        for name, nbytes, ms, launches in m.profile_decode_step(tok, cache):
            per.setdefault(name, [launches, nbytes, []])[2].append(ms)
    return {k: (v[0], v[1], float(np.median(v[2]))) for k, v in per.items()}


def step_floor(m, tok, cache, per, step_bytes):
    """tmg_profile_step_floor at the cache's position: the greedy step
    replayed from its graph, and the same launch chain with every kernel
    replaced by a streaming phase of its grid and bytes (weights and one
    dependent activation load, nothing else).  Per kind: the real kernel's
    graph-replay time (tmg_profile_decode_step, `per`) beside its phase's."""
    f = m.profile_step_floor(tok, cache)
    kinds = {}
    for name, nbytes, fbytes, fms, launches, nwg in f["kinds"]:
        real = per.get(name)
        kinds[name] = {"launches": launches, "workgroups": nwg, "bytes": nbytes, "phase_bytes": fbytes,
                       "phase_us": round(fms * 1e3, 3), "real_us": round(real[2] * 1e3, 3) if real else None,
                       "above_phase_us": round((real[2] - fms) * 1e3, 3) if real else None}
    step_us, floor_us = f["step_ms"] * 1e3, f["floor_ms"] * 1e3
    log(f"step floor: step {step_us:.1f} us, streaming chain {floor_us:.1f} us, empty launch "
        f"{f['empty_launch_ms'] * 1e3:.3f} us")
    return {"step_us": round(step_us, 2), "floor_us": round(floor_us, 2),
            "empty_launch_us": round(f["empty_launch_ms"] * 1e3, 3),
            "step_hbm_frac": round(step_bytes / (step_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "floor_hbm_frac": round(step_bytes / (floor_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "kinds": kinds}


def extra_long_context(T, W, m, sync, with_floor=True):
    """The long-context workload (C3) on the already loaded 1B model: an
    8192-token prefill, then 128 greedy decode steps from the captured step
    graph (warmed on the same cache, which is reset and refilled before the
    timed steps).  Reports the step rate, the KV share of the step bytes, the
    decode attention kernel's rate at that context and, with_floor, the step
    next to its streaming floor at the final position."""
    import numpy as np
    wl = W.LONG_CTX
    prompt = [int(t) for t in wl.prompt()]
    P, K = wl.prompt_len, wl.gen_tokens
    c = T.KvCache(m, P + K + 24)  # + the step-floor replays
    sync()
    t = time.perf_counter()
    lg = m.forward_seq(prompt, c)
    sync()
    first_prefill_s = time.perf_counter() - t
    first = int(np.argmax(lg))
    m.decode_greedy(first, 4, c)
    c.reset()
    # the timed prefill: the first one also grew the model's prefill scratch
    # to 8192 tokens (device allocations, once per model)
    sync()
    t = time.perf_counter()
    m.forward_seq(prompt, c, want_logits=False)
    sync()
    prefill_s = time.perf_counter() - t
    t = time.perf_counter()
    toks, ev_ms = m.decode_greedy(first, K, c)
    sync()
    wall = time.perf_counter() - t
    ms_step = wall * 1e3 / K
    n_ctx = P + (K + 1) / 2.0
    step_bytes = wl.decode_bytes(int(round(n_ctx)))
    per = kernel_table(m, c, int(toks[-1]))
    attn = per.get("attn_decode")
    floor = step_floor(m, int(toks[-1]), c, per, step_bytes) if with_floor else None
    c.close()
    log(f"8k: prefill {prefill_s * 1e3:.1f} ms (first, with scratch allocation: {first_prefill_s * 1e3:.1f} ms), "
        f"decode {ms_step:.4f} ms/step")
    return {
        "workload": f"{wl.name}: {P}-token prompt, batched prefill, {K} greedy decode steps",
        "ms_per_step": round(ms_step, 4), "tok_s": round(K / wall, 1), "decode_ms_events": round(ev_ms, 3),
        "step_hbm": {"bytes_per_token": step_bytes, "kv_bytes_per_token": wl.kv_bytes(int(round(n_ctx))),
                     "n_ctx_avg": n_ctx, "frac": round(step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "attn_decode": ({"avg_us": round(attn[2] * 1e3, 2), "bytes_per_launch": attn[1],
                         "GB_s": round(attn[1] / (attn[2] * 1e-3) / 1e9, 1)} if attn else None),
        "prefill_ms": round(prefill_s * 1e3, 2), "prefill_tok_s": round(P / prefill_s, 1),
        "prefill_tflops": round(wl.prefill_flops(P) / prefill_s / 1e12, 1),
        "first_prefill_ms": round(first_prefill_s * 1e3, 2),
        "step_floor": floor,
    }


def generate_setup_secs(T, m, prompt, samp, sync, reps=5):
    """Median time generate spends outside its prefill when it produces no
    token: the KV cache's allocation, the sampling state's upload, the step
    graph's capture and the cache's release (max_tokens = 0 returns right
    after the prefill)."""
    import numpy as np
    out = []
    for _ in range(reps):
        sync()
        t = time.perf_counter()
        g = T.generate(m, prompt, T.GenParams(max_tokens=0, **samp))
        out.append(time.perf_counter() - t - g.prefill_secs)
    return float(np.median(out))


def extra_four_b(T, W, model_dir, sync):
    """The 4B sampled workload (C4): 128-token prompt, 256 tokens with
    T=0.8, top-k 50, top-p 0.9, penalty 1.1, seed 42 through generate (the
    product path: device sampling, one id per step to the host), rate as the
    reference's main.rs reports it, (n - 1) / (elapsed - prefill)."""
    wl = W.FOUR_B
    path = W.ensure_model(wl, model_dir)
    m = T.Model.load(path)
    prompt = [int(t) for t in wl.prompt()]
    K = wl.gen_tokens
    T.generate(m, prompt, T.GenParams(max_tokens=16, **SAMPLED))
    sync()
    setup_s = generate_setup_secs(T, m, prompt, SAMPLED, sync)
    t = time.perf_counter()
    gen = T.generate(m, prompt, T.GenParams(max_tokens=K, **SAMPLED))
    wall_all = time.perf_counter() - t
    wall = wall_all - gen.prefill_secs
    n = len(gen.tokens) - 1
    ms_tok = wall * 1e3 / n
    n_ctx = wl.prompt_len + (K + 1) / 2.0
    step_bytes = wl.decode_bytes(int(round(n_ctx)))
    m.close()
    log(f"4b: {n / wall:.1f} tok/s through generate, {ms_tok:.4f} ms/token")
    return {
        "workload": f"{wl.name}: {wl.prompt_len}-token prompt, {K} sampled tokens (T=0.8, top-k 50, top-p 0.9, "
                    f"penalty 1.1, seed 42) through generate",
        "ms_per_token": round(ms_tok, 4), "tok_s": round(n / wall, 1),
        "prefill_ms": round(gen.prefill_secs * 1e3, 2),
        # the decode window holds the call's set-up (KV cache allocation, the
        # step graph's capture), as the reference's elapsed holds its own;
        # measured alone, and the rate without it
        "setup_ms": round(setup_s * 1e3, 3), "tok_s_excl_setup": round(n / (wall - setup_s), 1),
        "step_hbm": {"bytes_per_token": step_bytes, "n_ctx_avg": n_ctx,
                     "frac": round(step_bytes / (ms_tok * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
    }


def bench_batch(args, T, W, wl, m, load_s):
    """B prompts of the workload's length (prompt seeds s, s+1, ...), K greedy
    decode steps each through tmg_generate_batch; the device time of the
    batched steps (HIP events around the graph replays) gives the aggregate
    rate.  Step bytes: the weights once + every sequence's KV at its mean
    context."""
    from tinyminigo_amd.model import synth_tokens
    B, P = args.batch, wl.prompt_len
    K = args.steps if args.steps is not None else wl.gen_tokens
    prompts = [[int(t) for t in synth_tokens(wl.prompt_seed + i, P, wl.vocab_size)] for i in range(B)]
    T.generate_batch(m, prompts, min(K, args.warmup) + 1)
    out, ms = T.generate_batch(m, prompts, K + 1)
    ms_per_step = ms / K
    n_ctx_avg = P + (K + 1) / 2.0
    step_bytes = wl.weight_bytes() + B * (wl.kv_bytes(int(round(n_ctx_avg))) + wl.misc_bytes())
    gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"batch {B}: {K} steps in {ms:.1f} ms -> {B * K / (ms * 1e-3):.0f} tok/s aggregate")
    print(json.dumps({
        "metric": METRIC + " [batched decode]",
        "value": round(B * K / (ms * 1e-3), 1), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{wl.name}: {B} prompts of {P} tokens, {K} greedy decode steps each, batched",
                   "global_batch": B, "seq_len": P + K, "parallelism": "none (1 GPU)"},
        "load_s": round(load_s, 3),
        "roofline": {"bound": "hbm", "kernel": "batched decode step (all kernels)", "achieved": round(gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_step": step_bytes},
        "per_sequence_tok_s": round(K / (ms * 1e-3), 1),
        "cpu_baseline": None,
    }), flush=True)


def bench_prefill(args, T, wl, m, prompt, sync):
    """Prefill only (no decode step, so no graph launch): the workload's
    prompt through forward_seq on fresh caches, --prefill-reps times; the
    line reports the median.  For profiling the prefill kernels."""
    import numpy as np
    P = len(prompt)
    pf = []
    for _ in range(max(1, args.prefill_reps)):
        c = T.KvCache(m, P + 8)
        sync()
        t = time.perf_counter()
        m.forward_seq(prompt, c, want_logits=False)
        sync()
        pf.append(time.perf_counter() - t)
        c.close()
    s = float(np.median(pf))
    flops = wl.prefill_flops(P)
    log(f"prefill {P} tokens: {s * 1e3:.2f} ms ({flops / s / 1e12:.1f} TFLOP/s algorithmic)")
    print(json.dumps({
        "metric": METRIC + " [prefill only]", "value": round(P / s, 1), "unit": "tok/s", "n_gpus": 1,
        "steps": len(pf), "warmup": 0, "ms_per_step": round(s * 1e3, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"{wl.name}: {P}-token prompt, batched prefill", "global_batch": 1, "seq_len": P,
                   "parallelism": "none (1 GPU)"},
        "prefill_tflops": round(flops / s / 1e12, 2), "prefill_flops": flops, "cpu_baseline": None,
    }), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=["1b", "4b", "8k"], default="1b",
                    help="1b: 64-token prompt + 256 greedy steps (default); 4b: 128-token prompt + 256 sampled "
                         "tokens (T=0.8, top-k 50, top-p 0.9, penalty 1.1, seed 42); 8k: the 1b model after an "
                         "8192-token prefill, 128 greedy steps")
    ap.add_argument("--steps", type=int, default=None, help="decode steps (default: the workload's)")
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prefill-reps", type=int, default=5)
    ap.add_argument("--profile-steps", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-sweep", action="store_true", help="skip the GEMV shape sweep")
    ap.add_argument("--no-floor", action="store_true",
                    help="skip the step-floor measurement (tmg_profile_step_floor)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="time only the prefill of the workload's prompt (no decode, no graph launches)")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the long-context (8192-token) and 4B sampled workloads reported beside the 1b line")
    ap.add_argument("--weights", choices=["bf16", "i8"], default="bf16",
                    help="i8: load with TMG_I8=1, the reference's int8 weight-only mode (per-row int8 q/k/v/o/"
                         "gate/up/down, BF16 lm_head); the CPU baseline then times the oracle's int8 path")
    ap.add_argument("--batch", type=int, default=1,
                    help="B > 1: greedy decode of B prompts at once (tmg_generate_batch); value = aggregate "
                         "decode tok/s over the B sequences")
    ap.add_argument("--format", choices=["safetensors", "tmb"], default="safetensors",
                    help="tmb: repack the model into a TMB1 file once (the reference's --repack) and load that")
    ap.add_argument("--temperature", type=float, default=None,
                    help="sample through generate with these parameters (the rest default to the 4b workload's: "
                         "T=0.8, top-k 50, top-p 0.9, penalty 1.1, seed 42); top-k 0 or above 64 and top-p < 1 "
                         "without top-k take the whole-vocabulary sampler")
    ap.add_argument("--top-k", type=int, default=None)
    ap.add_argument("--top-p", type=float, default=None)
    ap.add_argument("--repetition-penalty", type=float, default=None)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only copy MIB MiB device to device (hipMemcpy; ROCclr's copyBuffer kernel), twice: "
                         "the known-size dispatch that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--model-dir", default=os.environ.get("TMG_MODEL_DIR",
                                                           os.path.join(tempfile.gettempdir(), "tmg_models")))
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: the decode path runs on a single MI355X "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration > 0:
        from tinyminigo_amd import hip as H
        nbytes = args.copy_calibration << 20
        src, dst = H.DeviceBuffer(nbytes), H.DeviceBuffer(nbytes)
        src.fill_byte(1)
        for _ in range(2):
            H.copy_device(dst, src, nbytes)
        H.synchronize()
        src.close()
        dst.close()
        log(f"copied {args.copy_calibration} MiB device to device twice ({nbytes} B read and written per copy)")
        return None

    import numpy as np

    import tinyminigo_amd as T
    from tinyminigo_amd import workloads as W
    # torch is not imported: a second HIP runtime in the process would leave
    # one of the two without a device; synchronize through libtmg's runtime
    from tinyminigo_amd.hip import synchronize as sync

    wl = {"1b": W.ONE_B, "4b": W.FOUR_B, "8k": W.LONG_CTX}[args.workload]
    samp = dict(SAMPLED) if args.workload == "4b" else None
    over = {k: v for k, v in (("temperature", args.temperature), ("top_k", args.top_k), ("top_p", args.top_p),
                              ("repetition_penalty", args.repetition_penalty)) if v is not None}
    if over:
        samp = dict(SAMPLED if samp is None else samp, **over)
    sampled = samp is not None and samp["temperature"] > 0
    t0 = time.perf_counter()
    path = W.ensure_model(wl, args.model_dir)
    log(f"model ready at {path} ({time.perf_counter() - t0:.1f}s)")
    prompt = [int(t) for t in wl.prompt()]
    K = args.steps if args.steps is not None else wl.gen_tokens
    Wm = args.warmup
    P = wl.prompt_len
    i8 = args.weights == "i8"
    if i8:
        os.environ["TMG_I8"] = "1"  # read by tmg_model_load, as the reference reads it at load
    else:
        os.environ.pop("TMG_I8", None)
    load_path = path
    if args.format == "tmb":
        load_path = os.path.splitext(path)[0] + ".tmb"
        if not os.path.exists(load_path) or os.path.getmtime(load_path) < os.path.getmtime(path):
            T.repack_tmb(path, load_path + ".part")
            os.replace(load_path + ".part", load_path)
    t0 = time.perf_counter()
    m = T.Model.load(load_path)
    sync()
    load_s = time.perf_counter() - t0
    log(f"model loaded ({args.weights} weights, {args.format}) in {load_s:.2f} s")

    if args.batch > 1:
        return bench_batch(args, T, W, wl, m, load_s)
    if args.prefill_only:
        return bench_prefill(args, T, wl, m, prompt, sync)

    # prefill tok/s: median over repetitions on fresh caches (one for 8k)
    pf = []
    for _ in range(1 if args.workload == "8k" else args.prefill_reps):
        c = T.KvCache(m, P + 8)
        sync()
        t = time.perf_counter()
        m.forward_seq(prompt, c, want_logits=False)
        sync()
        pf.append(time.perf_counter() - t)
        c.close()
    prefill_s = float(np.median(pf))
    log(f"prefill {P} tokens: {prefill_s * 1e3:.2f} ms")

    cap = P + max(K, Wm) + args.profile_steps + 18  # + the step-floor replays
    gen, setup_s = None, None
    if sampled:
        # the product path: generate (prefill, device sampling, one id per
        # step to the host); decode tok/s as the reference's main.rs reports
        # it, (n - 1) / (elapsed - prefill)
        T.generate(m, prompt, T.GenParams(max_tokens=Wm, **samp))
        sync()
        setup_s = generate_setup_secs(T, m, prompt, samp, sync)
        t = time.perf_counter()
        gen = T.generate(m, prompt, T.GenParams(max_tokens=K, **samp))
        wall_all = time.perf_counter() - t
        wall = wall_all - gen.prefill_secs
        K_timed = len(gen.tokens) - 1
        ev_ms = None
        log(f"generate {len(gen.tokens)} sampled tokens: {wall_all * 1e3:.1f} ms incl. prefill "
            f"{gen.prefill_secs * 1e3:.1f} ms and set-up {setup_s * 1e3:.2f} ms -> {K_timed / wall:.1f} tok/s")
        cache = T.KvCache(m, cap)
        logits = m.forward_seq(prompt, cache)
        toks = [int(np.argmax(logits))]
    else:
        # warmup on the timed cache itself (its step graph is captured there
        # and kept across the reset), then the prompt again and the timed steps
        cache = T.KvCache(m, cap)
        logits = m.forward_seq(prompt, cache)
        first = int(np.argmax(logits))
        m.decode_greedy(first, max(Wm, 1), cache)
        cache.reset()
        m.forward_seq(prompt, cache, want_logits=False)
        sync()
        t = time.perf_counter()
        toks, ev_ms = m.decode_greedy(first, K, cache)
        sync()
        wall = time.perf_counter() - t
        K_timed = K
        log(f"decode {K} steps: {wall * 1e3:.1f} ms wall, {ev_ms:.1f} ms events -> {K / wall:.1f} tok/s")
    ms_per_step = wall * 1e3 / K_timed
    n_ctx_avg = P + (K + 1) / 2.0
    step_bytes = wl.decode_bytes(int(round(n_ctx_avg)), i8)

    # per-kernel timing: each kernel kind's launches of one step replayed back
    # to back from a graph between HIP events on the library's stream
    per = {}
    tok = int(toks[-1])
    for _ in range(args.profile_steps):
        for name, nbytes, ms, launches in m.profile_decode_step(tok, cache):
            d = per.setdefault(name, [launches, nbytes, []])
            d[2].append(ms)
    per = {k: (v[0], v[1], float(np.median(v[2]))) for k, v in per.items()}
    step_kern_ms = sum(n * ms for n, _, ms in per.values())
    # dominant kernel: largest share of the step's kernel time
    name, (n_launch, nbytes, kern_ms) = max(per.items(), key=lambda kv: kv[1][0] * kv[1][2])
    achieved = nbytes / (kern_ms * 1e-3) / 1e9
    step_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    kernels = {k: {"launches": n, "avg_us": round(ms * 1e3, 2),
                   "GB_s": round(b / (ms * 1e-3) / 1e9, 1) if b else None,
                   "share": round(n * ms / step_kern_ms, 3)} for k, (n, b, ms) in per.items()}
    traffic, traffic_tree = pmc_traffic(name, args.weights) if args.workload == "1b" else (None, None)
    rp_us, rp_tree = rocprof_avg(name) if args.workload == "1b" and not i8 else (None, None)

    sweep = None if (args.no_sweep or args.workload != "1b" or i8) else gemv_sweep(T)

    # the step next to its floor (graph replays; skipped when the step's
    # kernels are launched one by one, as under the profiler)
    floor = None
    if args.workload in ("1b", "4b") and not i8 and not args.no_floor and os.environ.get("TMG_DECODE_GRAPH", "1") != "0":
        floor = step_floor(m, tok, cache, per, step_bytes)

    # the other two model workloads, reported beside the headline (1b line only)
    extras = {} if setup_s is None else {"generate_setup_ms": round(setup_s * 1e3, 3)}
    if args.workload == "1b" and not i8 and not sampled and not args.no_extras:
        extras["c3_long_context"] = extra_long_context(
            T, W, m, sync, with_floor=not args.no_floor and os.environ.get("TMG_DECODE_GRAPH", "1") != "0")

    cpu = None
    if not args.no_cpu:
        log("timing the CPU baseline")
        cpu = cpu_baseline(path, prompt, args.cpu_seconds, wl if args.workload == "8k" else None,
                           m if args.workload == "8k" else None, cache if args.workload == "8k" else None,
                           samp if sampled else None, i8)

    if args.workload == "1b" and not i8 and not sampled and not args.no_extras:
        extras["c4_four_b_sampled"] = extra_four_b(T, W, args.model_dir, sync)

    kind = (f"{K} sampled tokens (T={samp['temperature']:g}, top-k {samp['top_k']}, top-p {samp['top_p']:g}, "
             f"penalty {samp['repetition_penalty']:g}, seed {samp['seed']}) through generate"
            if sampled else f"{K} greedy decode steps")
    out = {
        "metric": METRIC,
        "value": round(K_timed / wall, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K_timed,
        "warmup": Wm,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8" if i8 else "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"{wl.name}: {P}-token prompt, batched prefill, {kind}",
            "model": "MiniCPM5-shaped Llama (random init)", "hidden": wl.hidden_size,
            "layers": wl.num_hidden_layers, "heads": wl.num_attention_heads, "kv_heads": wl.num_key_value_heads,
            "head_dim": wl.head_dim, "intermediate": wl.intermediate_size, "vocab": wl.vocab_size,
            "global_batch": 1, "seq_len": P + K, "parallelism": "none (1 GPU)",
            "arith": ("int8 layer weights with f32 row scales (TMG_I8=1), activations quantized per GEMV to int8, "
                      "exact int32 dots; BF16 lm_head; f32 KV cache" if i8 else
                      "BF16 weights, f32 activations/accumulation, f32 KV cache"),
        },
        "load_s": round(load_s, 3),
        "format": args.format,
        "prefill_tok_s": round(P / prefill_s, 1),
        "prefill_ms": round(prefill_s * 1e3, 3),
        "prefill_tflops": round(wl.prefill_flops(P) / prefill_s / 1e12, 2),
        "decode_ms_events": round(ev_ms, 3) if ev_ms is not None else None,
        "step_hbm": {"bytes_per_token": step_bytes, "kv_bytes_per_token": wl.kv_bytes(int(round(n_ctx_avg))),
                     "n_ctx_avg": n_ctx_avg, "achieved_GB_s": round(step_gbs, 1),
                     "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "kernel": name, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_per_launch": nbytes, "avg_launch_us": round(kern_ms * 1e3, 3),
                     "launches_per_step": n_launch, "traffic_tree": traffic_tree,
                     # the same kernel's rocprofv3 average (eager launches) in the
                     # committed summary, and the fraction of peak it gives
                     "rocprof_avg_us": rp_us, "rocprof_tree": rp_tree,
                     "frac_rocprof": round(nbytes / (rp_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if rp_us else None},
        "kernels": kernels,
        "step_floor": floor,
        "gemv_sweep": sweep,
        **extras,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
