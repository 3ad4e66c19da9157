"""Model-level pins of the oracle on the tiny synthetic Llama: agreement with
an independent float64 textbook decoder, and the reference's own invariants
(forward_seq ~ forward_token, tests/diff_debug.rs:10-40; first generated
token = argmax of the prefill logits, src/model.rs:623-646)."""
import numpy as np
import pytest

from oracle import oracle as O
from textbook import TextbookLlama
from tinyminigo_amd import workloads as W


@pytest.fixture(scope="module")
def tiny(tiny_path):
    m = O.OracleModel.load(tiny_path)
    tb = TextbookLlama(m.config, O.load_safetensors(tiny_path))
    return m, tb


def test_oracle_matches_float64_textbook(tiny):
    m, tb = tiny
    prompt = list(W.TINY.prompt())
    g = O.generate(m, prompt, 12)
    seq = prompt + g.tokens
    ref = tb.logits_all(seq)
    scale = np.abs(ref).max()
    assert np.abs(g.logits_first_step - ref[len(prompt) - 1]).max() < 2e-6 * scale
    cache = m.new_cache()
    for i, t in enumerate(seq):
        l = m.forward_token(t, cache)
        assert np.abs(l - ref[i]).max() < 2e-6 * scale, f"position {i}"


def test_textbook_catches_planted_mistakes(tiny):
    # a dropped residual term or a swapped RoPE pairing must show up far above
    # the tolerance used above
    m, tb = tiny
    prompt = list(W.TINY.prompt())
    ref = tb.logits_all(prompt)[-1]
    scale = np.abs(ref).max()
    d0 = tb.layers[0]["d"].copy()
    tb.layers[0]["d"][:] = 0.0
    bad = tb.logits_all(prompt)[-1]
    tb.layers[0]["d"][:] = d0
    assert np.abs(bad - ref).max() > 1e-3 * scale
    half = tb.hd // 2
    orig = tb.rope
    tb.rope = lambda x, pos: orig(np.concatenate([x[..., 1::2], x[..., ::2]], axis=-1), pos)
    bad = tb.logits_all(prompt)[-1]
    tb.rope = orig
    assert np.abs(bad - ref).max() > 1e-4 * scale
    assert half > 0


def test_forward_seq_matches_forward_token(tiny):
    m, _ = tiny
    prompt = list(W.TINY.prompt())
    c1 = m.new_cache()
    for t in prompt:
        a = m.forward_token(t, c1)
    c2 = m.new_cache()
    b = m.forward_seq(prompt, c2)
    # reference bound 1e-2 (tests/diff_debug.rs:39); the restatement differs
    # only in the RMSNorm association, so it sits far below that
    assert np.abs(a - b).max() < 1e-5
    for l in range(m.config.num_hidden_layers):
        assert c1.len(l) == c2.len(l) == len(prompt)
        assert np.abs(c1.keys_flat(l) - c2.keys_flat(l)).max() < 1e-5


def test_generate_first_token_is_prefill_argmax(tiny):
    m, _ = tiny
    prompt = list(W.TINY.prompt())
    g = O.generate(m, prompt, 3)
    assert g.tokens[0] == int(np.argmax(g.logits_first_step))
    with pytest.raises(O.OracleError, match="empty prompt"):
        O.generate(m, [], 3)


def test_kv_cache_push_and_len():
    # src/model.rs:784-797
    c = O.OracleCache(3, 2)
    assert c.total_len() == 0
    c.push(1, [0.1, 0.2], [0.3, 0.4])
    assert c.len(1) == 1 and c.len(0) == 0 and c.total_len() == 0
    c.push(0, [0.1, 0.2], [0.3, 0.4])
    assert c.len(0) == 1 and c.total_len() == 1
    c.reset()
    assert c.total_len() == 0
    with pytest.raises(O.OracleError, match="kv row width"):
        c.push(0, [0.1], [0.2])


def test_kv_cache_push_rows_equals_row_pushes():
    rng = np.random.default_rng(5)
    k = rng.standard_normal(6 * 4).astype(np.float32)
    v = rng.standard_normal(6 * 4).astype(np.float32)
    a, b = O.OracleCache(2, 4), O.OracleCache(2, 4)
    a.push_rows(1, k, v)
    for i in range(6):
        b.push(1, k[4 * i:4 * i + 4], v[4 * i:4 * i + 4])
    assert a.len(1) == b.len(1) == 6
    assert np.array_equal(a.keys_flat(1), b.keys_flat(1)) and np.array_equal(a.values_flat(1), b.values_flat(1))
    with pytest.raises(O.OracleError, match="kv row width"):
        a.push_rows(0, k[:5], v[:5])
