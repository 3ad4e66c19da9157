"""Writes tests/golden/long_context_8k.npz: the oracle's results for the
long-context workload (the 1B MiniCPM5-shaped model, weights seed 3, an
8192-id prompt from seed 5, then 128 greedy tokens).

    python tests/golden/make_long_context.py [--threads N]

The oracle runs with N threads for the batched GEMM and, for attention_batch,
the head-parallel split (each (token, head) row is computed by the same code
in the same order, so the result is bit-identical to the single-threaded
reference order; om_set_attn_threads).  About 10-20 minutes on 8 cores.

Stored (small enough to commit):
  prompt_seed, prompt_len, n_gen      the workload
  ids                                 the 128 greedy ids generate returns
  last_idx, last_val                  every 16th prefill last-token logit
  top_ids, top_val                    the 64 largest prefill logits (desc.)
  step_top_ids, step_top_val          top-8 ids (descending) and their logits
                                      of the logits each greedy id was chosen
                                      from (128 x 8)
  step_idx, step_val                  every 16th logit (ids last_idx) at the
                                      decode steps step_idx: the logits
                                      forward_token returns after feeding
                                      ids[step - 1] (step 0 is the prefill)
  kv_pos                              sampled cache positions
  k0, v0, k23, v23                    layers 0 and 23, K/V rows at kv_pos
  kv_sum, kv_sumsq                    per layer f64 sum / sum of squares of
                                      all 8192 prefill K and V rows [L, 2]
"""
import argparse
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from tinyminigo_amd import workloads as W  # noqa: E402

KV_POS = [0, 1, 63, 64, 1000, 4095, 4096, 6001, 8190, 8191]
# decode steps whose logits are stored in full (every 16th id)
STEP_IDX = [1, 31, 63, 127]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--model-dir", default=os.environ.get("TMG_MODEL_DIR") or os.path.join(tempfile.gettempdir(),
                                                                                             "tmg_models"))
    args = ap.parse_args()
    wl = W.LONG_CTX
    path = W.ensure_model(W.ONE_B, args.model_dir)
    O.set_num_threads(args.threads)
    O.set_attn_threads(args.threads)
    m = O.OracleModel.load(path)
    prompt = [int(t) for t in wl.prompt()]
    assert len(prompt) == 8192
    L = m.config.num_hidden_layers
    t0 = time.time()
    cache = m.new_cache()
    # the oracle's prefill state is kept beside the model (not in the
    # repository), so a rerun resumes at the decode steps
    state = os.path.join(os.path.dirname(path), f"oracle_prefill_seed{wl.prompt_seed}_{len(prompt)}.npz")
    if os.path.exists(state):
        st = np.load(state)
        for layer in range(L):
            cache.push_rows(layer, st[f"k{layer}"], st[f"v{layer}"])
        logits = st["logits"]
        print(f"[long-context] prefill state loaded from {state}", flush=True)
    else:
        logits = m.forward_seq(prompt, cache)
        print(f"[long-context] prefill {len(prompt)} tokens: {time.time() - t0:.1f} s", flush=True)
        arrays = {"logits": logits}
        for layer in range(L):
            arrays[f"k{layer}"] = cache.keys_flat(layer)
            arrays[f"v{layer}"] = cache.values_flat(layer)
        np.savez(state + ".part.npz", **arrays)
        os.replace(state + ".part.npz", state)
    kv_sum = np.zeros((L, 2), np.float64)
    kv_sumsq = np.zeros((L, 2), np.float64)
    rows = {}
    kvd = m.config.num_key_value_heads * m.config.head_dim
    for layer in range(L):
        k = cache.keys_flat(layer).astype(np.float64)
        v = cache.values_flat(layer).astype(np.float64)
        kv_sum[layer] = k.sum(), v.sum()
        kv_sumsq[layer] = (k * k).sum(), (v * v).sum()
        if layer in (0, L - 1):
            kk, vv = k.reshape(-1, kvd), v.reshape(-1, kvd)
            rows[layer] = (kk[KV_POS].astype(np.float32), vv[KV_POS].astype(np.float32))
    order = np.argsort(-logits, kind="stable")
    # the greedy continuation, as generate runs it (first id from the prefill
    # logits, src/model.rs:623-646); reuse the filled cache
    ids, step_top, step_top_val, step_val = [], [], [], []
    lg = logits
    t1 = time.time()
    for i in range(wl.gen_tokens):
        nxt = O.argmax(lg)
        ids.append(nxt)
        top8 = np.argsort(-lg, kind="stable")[:8]
        step_top.append(top8)
        step_top_val.append(lg[top8].astype(np.float32))
        if i in STEP_IDX:
            step_val.append(lg[::16].astype(np.float32))
        if i + 1 < wl.gen_tokens:
            lg = m.forward_token(nxt, cache)
    print(f"[long-context] {wl.gen_tokens} greedy ids: {time.time() - t1:.1f} s", flush=True)
    out = os.path.join(HERE, "long_context_8k.npz")
    np.savez_compressed(
        out, prompt_seed=wl.prompt_seed, prompt_len=len(prompt), n_gen=wl.gen_tokens,
        ids=np.array(ids, np.uint32), last_idx=np.arange(0, logits.size, 16, dtype=np.uint32),
        last_val=logits[::16].astype(np.float32), top_ids=order[:64].astype(np.uint32),
        top_val=logits[order[:64]].astype(np.float32), step_top_ids=np.array(step_top, np.uint32),
        step_top_val=np.array(step_top_val, np.float32), step_idx=np.array(STEP_IDX, np.uint32),
        step_val=np.array(step_val, np.float32),
        kv_pos=np.array(KV_POS, np.uint32), k0=rows[0][0], v0=rows[0][1], k23=rows[L - 1][0], v23=rows[L - 1][1],
        kv_sum=kv_sum, kv_sumsq=kv_sumsq)
    print(f"[long-context] wrote {out} ({os.path.getsize(out)} bytes)", flush=True)


if __name__ == "__main__":
    main()
