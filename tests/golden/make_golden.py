"""Writes the golden fixtures under tests/golden from the oracle.

    python tests/golden/make_golden.py

tiny_llama.json   C0: the synthetic tiny Llama (hidden 64, 2 layers, 4/2
                  heads, head_dim 16, I 128, V 1024, tied lm_head, weights
                  seed 0), its 16-id prompt (seed 1), 40 greedy ids, and per
                  step the first 16 logits, the top-8 (id, logit) pairs and
                  the float64 sum of all logits.
tiny_llama.npz    C0 prefill last-token logits [1024] and the prefill KV
                  cache of layer 1 [16, 32] (keys, values).
gemv_small.npz    a 64x128 BF16 GEMV (W seed 2 stream "w", x seed 2 stream
                  "x") with the oracle's output.

The oracle itself is pinned by the known-answer, brute-force and textbook
tests; these fixtures freeze its outputs so any later change to it, to the
synthetic generator or to the loaders shows up as a diff.
"""
import hashlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from tinyminigo_amd import synth_normal_bf16, synth_normal_f32  # noqa: E402
from tinyminigo_amd import workloads as W  # noqa: E402


def main():
    root = tempfile.mkdtemp(prefix="tmg_golden_")
    path = W.ensure_model(W.TINY, root)
    m = O.OracleModel.load(path)
    prompt = [int(t) for t in W.TINY.prompt()]
    g = O.generate(m, prompt, W.TINY.gen_tokens)
    # per-step logits by replaying the ids token by token after the prefill
    cache = m.new_cache()
    first = m.forward_seq(prompt, cache)
    kv = (cache.keys_flat(1).reshape(len(prompt), -1), cache.values_flat(1).reshape(len(prompt), -1))
    steps = []
    logits = first
    for t in g.tokens:
        top = np.argsort(-logits, kind="stable")[:8]
        steps.append({"first16": [float(v) for v in logits[:16]],
                      "top8": [[int(i), float(logits[i])] for i in top],
                      "sum": float(np.sum(logits.astype(np.float64)))})
        logits = m.forward_token(t, cache)
    fx = {
        "workload": W.TINY.name,
        "model_sha256": hashlib.sha256(open(path, "rb").read()).hexdigest(),
        "prompt": prompt,
        "greedy_tokens": g.tokens,
        "steps": steps,
    }
    with open(os.path.join(HERE, "tiny_llama.json"), "w") as f:
        json.dump(fx, f, indent=1)
    np.savez(os.path.join(HERE, "tiny_llama.npz"), prefill_logits=first, keys_l1=kv[0], values_l1=kv[1])

    w = synth_normal_bf16(2, "w", 64 * 128, 0.02)
    x = synth_normal_f32(2, "x", 128, 1.0)
    y = O.matmul_w(x, w, 64, 128)
    np.savez(os.path.join(HERE, "gemv_small.npz"), w=w, x=x, y=y)
    print("wrote fixtures; tokens:", g.tokens[:8], "...")


if __name__ == "__main__":
    main()
