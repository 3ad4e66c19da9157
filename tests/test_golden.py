"""The oracle against the committed golden fixtures (tests/golden)."""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def fx():
    return json.load(open(os.path.join(GOLD, "tiny_llama.json")))


def test_tiny_llama_prefill_and_greedy(tiny_path, fx):
    m = O.OracleModel.load(tiny_path)
    z = np.load(os.path.join(GOLD, "tiny_llama.npz"))
    cache = m.new_cache()
    logits = m.forward_seq(fx["prompt"], cache)
    assert np.array_equal(logits, z["prefill_logits"])
    assert np.array_equal(cache.keys_flat(1).reshape(z["keys_l1"].shape), z["keys_l1"])
    assert np.array_equal(cache.values_flat(1).reshape(z["values_l1"].shape), z["values_l1"])
    g = O.generate(m, fx["prompt"], len(fx["greedy_tokens"]))
    assert g.tokens == fx["greedy_tokens"]
    for i, (t, st) in enumerate(zip(fx["greedy_tokens"], fx["steps"])):
        assert [float(v) for v in logits[:16]] == st["first16"], f"step {i}"
        assert [[int(a), float(b)] for a, b in st["top8"]] == [[int(j), float(logits[j])] for j, _ in st["top8"]]
        assert abs(float(np.sum(logits.astype(np.float64))) - st["sum"]) == 0.0
        logits = m.forward_token(t, cache)


def test_gemv_small():
    z = np.load(os.path.join(GOLD, "gemv_small.npz"))
    assert np.array_equal(O.matmul_w(z["x"], z["w"], 64, 128), z["y"])
