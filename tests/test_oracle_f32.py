"""Pins of the oracle's WMat::F32 path (F32 / F16 weight matrices, converted
to f32 at load: src/model.rs:49-55, src/safetensors_loader.rs:103-147):
matmul_w_into's f32 arm (src/tensor.rs:387-420) against exact float64 sums,
the batched GEMM against the per-element dot it equals (src/tensor.rs:734-738),
an F32 file of BF16 values against the BF16 model bit for bit (the reference
notes the two dots are bit-identical, src/tensor.rs:38-41), and whole models
against the independent float64 textbook decoder."""
import numpy as np
import pytest

from conftest import model_root
from f32models import variant
from oracle import oracle as O
from textbook import TextbookLlama
from tinyminigo_amd import workloads as W


def test_matmul_w_f32_against_float64():
    rng = np.random.default_rng(3)
    for out, inp in ((100, 136), (7, 8), (513, 64), (64, 2056)):
        w = rng.standard_normal((out, inp)).astype(np.float32)
        x = rng.standard_normal(inp).astype(np.float32)
        y = O.matmul_w_f32(x, w, out, inp)
        exact = w.astype(np.float64) @ x.astype(np.float64)
        mag = np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64))
        assert np.all(np.abs(y - exact) <= 2e-6 * mag)
        # threaded or not, every row is dot(x, w_o)
        assert np.array_equal(y, np.array([O.dot(x, w[o]) for o in range(out)], np.float32))


def test_matmul_batch_w_f32_is_dot_per_element():
    rng = np.random.default_rng(4)
    out, inp, T = 70, 136, 5
    w = rng.standard_normal((out, inp)).astype(np.float32)
    x = rng.standard_normal((T, inp)).astype(np.float32)
    y = O.matmul_batch_w_f32(x, w, out, inp, T).reshape(T, out)
    want = np.array([[O.dot(x[t], w[o]) for o in range(out)] for t in range(T)], np.float32)
    assert np.array_equal(y, want)


def test_planted_transpose_is_caught():
    # a transposed operand fails the float64 bound above
    rng = np.random.default_rng(5)
    n = 64
    w = rng.standard_normal((n, n)).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    y = O.matmul_w_f32(x, np.ascontiguousarray(w.T), n, n)
    exact = w.astype(np.float64) @ x.astype(np.float64)
    assert np.abs(y - exact).max() > 1e-2


@pytest.fixture(scope="module")
def untied_path():
    import dataclasses
    wl = dataclasses.replace(W.TINY, name="tiny-llama-untied-s11", tied_lm_head=False, weight_seed=11,
                             rope_theta=500.0, rms_norm_eps=1e-5)
    return W.ensure_model(wl, model_root())


def test_f32_file_of_bf16_values_equals_bf16_model(untied_path):
    a = O.OracleModel.load(untied_path)
    b = O.OracleModel.load(variant(untied_path, model_root(), "f32_exact"))
    ids = [int(t) for t in W.TINY.prompt()]
    ca, cb = a.new_cache(), b.new_cache()
    assert np.array_equal(a.forward_seq(ids, ca), b.forward_seq(ids, cb))
    for t in (3, 77, 500):
        assert np.array_equal(a.forward_token(t, ca), b.forward_token(t, cb))


@pytest.mark.parametrize("kind", ["f32", "f16", "mixed"])
def test_f32_models_against_float64_textbook(untied_path, kind):
    p = variant(untied_path, model_root(), kind)
    m = O.OracleModel.load(p)
    tensors = O.load_safetensors(p)
    if kind != "mixed":
        want = "F32" if kind == "f32" else "F16"
        assert tensors["model.layers.0.self_attn.q_proj.weight"].dtype == want
        assert tensors["lm_head.weight"].dtype == want
    tb = TextbookLlama(m.config, tensors)
    prompt = [int(t) for t in W.TINY.prompt()]
    g = O.generate(m, prompt, 8)
    seq = prompt + g.tokens
    ref = tb.logits_all(seq)
    scale = np.abs(ref).max()
    assert np.abs(g.logits_first_step - ref[len(prompt) - 1]).max() < 2e-6 * scale
    cache = m.new_cache()
    for i, t in enumerate(seq):
        lg = m.forward_token(t, cache)
        assert np.abs(lg - ref[i]).max() < 2e-6 * scale, f"{kind} position {i}"
    # the perturbation matters: the BF16 source gives different logits
    base = O.OracleModel.load(untied_path)
    assert np.abs(base.forward_seq(prompt, base.new_cache()) - g.logits_first_step).max() > 1e-6 * scale


def test_tied_f32_embedding_against_float64_textbook(tiny_path):
    p = variant(tiny_path, model_root(), "tied_f32")
    m = O.OracleModel.load(p)
    tensors = O.load_safetensors(p)
    assert "lm_head.weight" not in tensors and tensors["model.embed_tokens.weight"].dtype == "F32"
    tb = TextbookLlama(m.config, tensors)
    prompt = [int(t) for t in W.TINY.prompt()]
    ref = tb.logits_all(prompt)
    lg = m.forward_seq(prompt, m.new_cache())
    assert np.abs(lg - ref[-1]).max() < 2e-6 * np.abs(ref).max()


def test_i8_from_f32_quantizes_the_f32_values(untied_path):
    # wmat_maybe_i8 (src/model.rs:60-76): an F32 matrix is quantized from its
    # f32 values; the int8 model's prefill equals the textbook with those
    # quantized weights (no activation quantization in the batched path)
    p = variant(untied_path, model_root(), "f32")
    m = O.OracleModel.load(p, i8=True)
    tensors = O.load_safetensors(p)
    tb = TextbookLlama(m.config, tensors, i8=True)
    prompt = [int(t) for t in W.TINY.prompt()]
    ref = tb.logits_all(prompt)
    lg = m.forward_seq(prompt, m.new_cache())
    assert np.abs(lg - ref[-1]).max() < 2e-6 * np.abs(ref).max()
