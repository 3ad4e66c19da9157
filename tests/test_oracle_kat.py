"""Known-answer tests that pin the oracle, ported from the reference's own
unit tests (src/tensor.rs:1215-1364, src/config.rs:187-225,
src/safetensors_loader.rs:177-226), plus brute-force and closed-form checks
chosen so that a plausible slip (dropped term, wrong pairing, swapped
association) fails one of them."""
import json
import math
import os
import struct

import numpy as np
import pytest

from oracle import oracle as O


def approx(a, b, tol):
    assert abs(a - b) < tol, f"a={a} b={b}"


def bf16_bits(x):
    """round-to-nearest-even f32 -> BF16 bits (test-side helper)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


# --- src/tensor.rs:1223-1240 -------------------------------------------------

def test_matmul_identity():
    w = bf16_bits([1.0, 0.0, 0.0, 1.0])
    assert list(O.matmul_w([3.0, -4.0], w, 2, 2)) == [3.0, -4.0]


def test_matmul_linear_weights():
    # HF nn.Linear: y = x W^T with W [out, in]: out0 = 1+2, out1 = 3+4
    w = bf16_bits([1.0, 2.0, 3.0, 4.0])
    assert list(O.matmul_w([1.0, 1.0], w, 2, 2)) == [3.0, 7.0]


def test_dot_bf16_brute_force_and_lane_order():
    rng = np.random.default_rng(5)
    for n in (8, 16, 64, 67, 2048):
        a = rng.standard_normal(n).astype(np.float32)
        w = bf16_bits(rng.standard_normal(n) * 0.02)
        wf = (w.astype(np.uint32) << 16).view(np.float32)
        exact = float(np.dot(a.astype(np.float64), wf.astype(np.float64)))
        got = O.dot_bf16(a, w)
        assert abs(got - exact) <= 1e-6 * (np.abs(a.astype(np.float64) * wf).sum() + 1e-30)
        # the 8-lane FMA + ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7)) order, restated
        lanes = [np.float32(0)] * 8
        for i in range(n // 8):
            for j in range(8):
                lanes[j] = np.float32(np.float64(a[8 * i + j]) * np.float64(wf[8 * i + j]) + np.float64(lanes[j]))
        s = np.float32(np.float32(np.float32(lanes[0] + lanes[4]) + np.float32(lanes[2] + lanes[6])) +
                       np.float32(np.float32(lanes[1] + lanes[5]) + np.float32(lanes[3] + lanes[7])))
        for i in range(n // 8 * 8, n):
            s = np.float32(s + np.float32(a[i] * wf[i]))
        assert np.float32(got) == s


def test_matmul_batch_equals_per_row_dot():
    # src/tensor.rs:734-738: the tiled GEMM is bit-identical to dot_bf16 per element
    rng = np.random.default_rng(6)
    T, out, inp = 7, 13, 40
    x = rng.standard_normal(T * inp).astype(np.float32)
    w = bf16_bits(rng.standard_normal(out * inp) * 0.02)
    y = O.matmul_batch_w(x, w, out, inp, T).reshape(T, out)
    for t in range(T):
        for o in range(out):
            assert y[t, o] == np.float32(O.dot_bf16(x[t * inp:(t + 1) * inp], w[o * inp:(o + 1) * inp]))


# --- src/tensor.rs:1243-1259 -------------------------------------------------

def test_rms_norm_known():
    y = O.rms_norm([3.0, 4.0], [1.0, 1.0], 0.0)
    inv = 1.0 / math.sqrt(12.5)
    approx(y[0], 3.0 * inv, 1e-6)
    approx(y[1], 4.0 * inv, 1e-6)


def test_rms_norm_weighted():
    y = O.rms_norm([3.0, 4.0], [2.0, 0.5], 1e-6)
    inv = 1.0 / math.sqrt(12.5 + 1e-6)
    approx(y[0], 3.0 * inv * 2.0, 1e-6)
    approx(y[1], 4.0 * inv * 0.5, 1e-6)


def test_rms_norm_associations_differ_only_in_rounding():
    # decode (v*inv)*w vs prefill v*(inv*w) (src/tensor.rs:951 vs :975)
    rng = np.random.default_rng(7)
    x = rng.standard_normal(64).astype(np.float32)
    w = rng.standard_normal(64).astype(np.float32)
    a = O.rms_norm(x, w, 1e-5)
    b = O.rms_norm_batch(x, w, 1e-5, 64)
    assert np.max(np.abs(a - b)) < 1e-6 * np.max(np.abs(a))
    inv = np.float32(1.0) / np.sqrt(np.float32(np.sum(x.astype(np.float64) ** 2) / 64) + np.float32(1e-5))
    assert np.allclose(a, x * inv * w, rtol=1e-5)


# --- src/tensor.rs:1262-1292 -------------------------------------------------

def test_rope_preserves_norm():
    v = np.arange(8, dtype=np.float32) * 0.5 - 1.75
    r = O.rope_rotate(v, 17, 5000000.0)
    approx(float(np.sum(v * v)), float(np.sum(r * r)), 1e-4)


def test_rope_zero_pos_identity():
    assert list(O.rope_rotate([1.0, 2.0, 3.0, 4.0], 0, 10000.0)) == [1.0, 2.0, 3.0, 4.0]


def test_rope_matches_reference_pairing():
    # rotate_half: pairs (i, i+half); pos=1, theta=1e4, d=4 -> angles 1 and 0.01
    v = O.rope_rotate([1.0, 0.0, 0.0, 1.0], 1, 10000.0)
    approx(v[0], math.cos(1.0), 1e-5)
    approx(v[2], math.sin(1.0), 1e-5)
    approx(v[1], -math.sin(0.01), 1e-5)
    approx(v[3], math.cos(0.01), 1e-5)


def test_rope_table_matches_rotate_and_closed_form():
    hd, theta = 16, 10000.0
    cos, sin = O.rope_table(hd, theta, 40)
    for pos in (0, 1, 7, 39):
        for i in range(hd // 2):
            ang = pos / theta ** (2 * i / hd)
            approx(cos[pos, i], math.cos(ang), 2e-6 * max(1.0, pos))
            approx(sin[pos, i], math.sin(ang), 2e-6 * max(1.0, pos))


# --- src/tensor.rs:1295-1333 -------------------------------------------------

def test_silu_known():
    approx(O.silu([0.0])[0], 0.0, 1e-6)
    approx(O.silu([1.0])[0], 1.0 / (1.0 + math.exp(-1.0)), 1e-6)


def test_softmax_sums_to_one():
    p = O.softmax([1.0, 2.0, 3.0])
    approx(float(p.sum()), 1.0, 1e-6)
    assert p[2] > p[1] > p[0]
    e = np.exp(np.array([1.0, 2.0, 3.0]) - 3.0)
    assert np.allclose(p, e / e.sum(), rtol=1e-6)


def test_argmax_basic_and_ties():
    assert O.argmax([0.1, 3.0, 2.0]) == 1
    assert O.argmax([2.0, 2.0]) == 0
    assert O.argmax([-np.inf, -np.inf]) == 0
    assert O.argmax([np.nan, 1.0, np.nan]) == 1


def test_argmax_edge_values():
    # `v > best` from (0, -inf) (src/tensor.rs:1063-1073): -0.0 == +0.0, so
    # the first zero wins; +inf is taken once; NaN never; empty -> 0
    assert O.argmax([-0.0, 0.0]) == 0
    assert O.argmax([0.0, -0.0]) == 0
    assert O.argmax([-1.0, -0.0, 0.0]) == 1
    assert O.argmax([1.0, np.inf, np.inf]) == 1
    assert O.argmax([np.nan, np.inf]) == 1
    assert O.argmax([np.nan, -np.inf, np.nan]) == 0
    assert O.argmax([-np.inf, -3.0, -np.inf]) == 1
    assert O.argmax([]) == 0
    assert O.argmax([1e-45, 0.0]) == 0 and O.argmax([0.0, 1e-45]) == 1


def test_attention_row_shapes():
    q = [1.0, 0.0]
    keys = [1.0, 0.0, 0.0, 1.0]
    vals = [1.0, 2.0, 3.0, 4.0]
    out = O.attention_row(q, keys, vals, 2, 1.0 / math.sqrt(2.0))
    p = O.softmax([1.0 / math.sqrt(2.0), 0.0])
    approx(out[0], p[0] * 1.0 + p[1] * 3.0, 1e-5)
    approx(out[1], p[0] * 2.0 + p[1] * 4.0, 1e-5)


def test_attention_batch_single_position_returns_v_and_matches_brute_force():
    rng = np.random.default_rng(8)
    nq, nkv, hd, T = 4, 2, 8, 5
    q = rng.standard_normal(T * nq * hd).astype(np.float32)
    k = rng.standard_normal(T * nkv * hd).astype(np.float32)
    v = rng.standard_normal(T * nkv * hd).astype(np.float32)
    out = O.attention_batch(q, k, v, nq, nkv, hd, 0).reshape(T, nq, hd)
    # n_ctx = 1 for token 0: the output is v of that KV head
    for h in range(nq):
        assert np.allclose(out[0, h], v.reshape(T, nkv, hd)[0, h // 2], atol=1e-7)
    # brute force in f64 with the GQA head mapping kv = h // group
    q3, k3, v3 = q.reshape(T, nq, hd), k.reshape(T, nkv, hd), v.reshape(T, nkv, hd)
    for t in range(T):
        for h in range(nq):
            s = k3[:t + 1, h // 2].astype(np.float64) @ q3[t, h] / math.sqrt(hd)
            p = np.exp(s - s.max())
            p /= p.sum()
            assert np.allclose(out[t, h], p @ v3[:t + 1, h // 2], atol=2e-6)


def test_repetition_penalty_applied():
    l = O.apply_repetition_penalty([2.0, -2.0, 1.0], [0, 1], 2.0)
    assert list(l) == [1.0, -4.0, 1.0]
    # a set, not a multiset: a repeated id is penalized once
    l = O.apply_repetition_penalty([2.0, -2.0, 1.0], [0, 0, 0], 2.0)
    assert list(l) == [1.0, -2.0, 1.0]
    assert list(O.apply_repetition_penalty([2.0, -2.0], [0, 1], 1.0)) == [2.0, -2.0]


# --- src/tensor.rs:1336-1364 (sampling invariants) ---------------------------

def test_greedy_sample_is_argmax():
    assert O.sample([0.1, 5.0, 3.0], 0.0, 0, 1.0, 0.3).token == 1


def test_temperature_sample_peaked():
    # "strongly peaked -> should pick 4 most of the time": the walk is in id
    # order, so every draw above the first four probabilities (~0.0337) picks 4
    logits = [0.1, 0.2, 0.3, 0.4, 5.0]
    for r in (0.05, 0.5, 0.9, 0.999):
        assert O.sample(logits, 1.0, 0, 1.0, r).token == 4
    assert O.sample(logits, 1.0, 0, 1.0, 0.0).token == 0


def test_top_k_restricts_candidates():
    logits = [0.0, 5.0, 1.0, 4.0, 2.0]
    for r in np.linspace(0, 0.999, 50):
        tr = O.sample(logits, 1.0, 2, 1.0, float(r))
        assert tr.token in (1, 3)
        assert list(tr.cand_ids) == [1, 3]


def test_sample_inverse_cdf_closed_form():
    # k=0: candidates in id order; the draw walks cumulative probabilities
    logits = np.log(np.array([0.1, 0.2, 0.3, 0.4], np.float64)).astype(np.float32)
    for r, want in ((0.05, 0), (0.15, 1), (0.35, 2), (0.65, 3), (0.999, 3)):
        assert O.sample(logits, 1.0, 0, 1.0, r).token == want
    # nucleus p=0.5 keeps {3 (0.4), 2 (0.3)}; renormalized 4/7, 3/7 walked in id order
    tr = O.sample(logits, 1.0, 0, 0.5, 0.5)
    assert np.allclose(tr.cand_probs, [0, 0, 3 / 7, 4 / 7], atol=1e-6)
    assert tr.token == 3
    assert O.sample(logits, 1.0, 0, 0.5, 0.2).token == 2


# --- src/config.rs:187-225 ---------------------------------------------------

TINY_RANDOM_MINICPM5 = {
    "architectures": ["LlamaForCausalLM"], "bos_token_id": 0, "eos_token_id": [1, 130073], "head_dim": 32,
    "hidden_size": 16, "intermediate_size": 64, "model_type": "llama", "num_attention_heads": 16,
    "num_hidden_layers": 2, "num_key_value_heads": 2, "rms_norm_eps": 1e-06,
    "rope_parameters": {"rope_theta": 5000000.0, "rope_type": "default"}, "tie_word_embeddings": False,
    "vocab_size": 130560,
}


def test_parses_tiny_random_minicpm5_config(tmp_path):
    p = tmp_path / "config.json"
    p.write_text(json.dumps(TINY_RANDOM_MINICPM5))
    c = O.load_config(str(p))
    assert (c.hidden_size, c.num_hidden_layers, c.num_attention_heads, c.num_key_value_heads) == (16, 2, 16, 2)
    assert (c.head_dim, c.intermediate_size, c.vocab_size) == (32, 64, 130560)
    assert c.rms_norm_eps == np.float32(1e-6)
    assert c.rope_theta == 5_000_000.0
    assert c.eos_token_ids == [1, 130073]
    assert c.bos_token_id == 0
    assert c.num_attention_heads // c.num_key_value_heads == 8


def test_config_defaults(tmp_path):
    p = tmp_path / "config.json"
    p.write_text(json.dumps({"hidden_size": 64, "num_attention_heads": 4, "num_hidden_layers": 1,
                             "intermediate_size": 8, "vocab_size": 10, "eos_token_id": 7}))
    c = O.load_config(str(p))
    assert c.num_key_value_heads == 4 and c.head_dim == 16
    assert c.rope_theta == 10000.0 and c.rms_norm_eps == np.float32(1e-5)
    assert c.eos_token_ids == [7]
    p.write_text(json.dumps({"hidden_size": 64}))
    with pytest.raises(O.OracleError, match="num_attention_heads"):
        O.load_config(str(p))


# --- src/safetensors_loader.rs:177-226 ----------------------------------------

def test_f16_and_bf16_conversions():
    assert O.f16_to_f32(np.array([0x3C00], np.uint16))[0] == 1.0
    assert O.f16_to_f32(np.array([0x0000], np.uint16))[0] == 0.0
    assert O.f16_to_f32(np.array([0xBC00], np.uint16))[0] == -1.0
    assert O.bf16_to_f32(np.array([0x3F80], np.uint16))[0] == 1.0
    assert O.bf16_to_f32(np.array([0x0000], np.uint16))[0] == 0.0


def _write_st(path, tensors):
    hdr, blobs, off = {}, [], 0
    for name, (dt, shape, raw) in tensors.items():
        hdr[name] = {"dtype": dt, "shape": shape, "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(hdr).encode()
    h += b" " * ((8 - (8 + len(h)) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"".join(blobs))


def test_safetensors_roundtrip(tmp_path):
    p = str(tmp_path / "t.safetensors")
    _write_st(p, {"w": ("F32", [2, 2], np.array([1, 2, 3, 4], np.float32).tobytes()),
                  "b": ("BF16", [2], np.array([0x3F80, 0xC000], np.uint16).tobytes())})
    t = O.load_safetensors(p)
    assert t["w"].shape == [2, 2] and list(t["w"].data) == [1.0, 2.0, 3.0, 4.0]
    assert t["b"].dtype == "BF16" and list(t["b"].data) == [0x3F80, 0xC000]


def test_safetensors_errors(tmp_path):
    p = str(tmp_path / "bad.safetensors")
    _write_st(p, {"x": ("I64", [1], np.zeros(1, np.int64).tobytes())})
    with pytest.raises(O.OracleError, match="unsupported dtype"):
        O.load_safetensors(p)
    with open(p, "wb") as f:
        f.write(struct.pack("<Q", 1000) + b"{}")
    with pytest.raises(O.OracleError, match="truncated"):
        O.load_safetensors(p)
