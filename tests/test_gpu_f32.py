"""F32 / F16 weight matrices on the GPU (WMat::F32: the reference converts
such tensors to f32 at load, src/model.rs:49-55, and multiplies them with
`dot`, src/tensor.rs:58-74 and 387-420): the f32-row decode GEMV, the fp32
MFMA prefill GEMM and the loader, against the oracle's f32 path on the same
files.  Tolerances are the decode path's (logits within 2e-3 abs + 1e-3 rel,
greedy ids identical)."""
import dataclasses

import numpy as np
import pytest

from conftest import model_root
from f32models import variant

pytestmark = pytest.mark.gpu

ABS_TOL, REL_TOL = 2e-3, 1e-3


def close_logits(a, b, what=""):
    d = np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))
    lim = ABS_TOL + REL_TOL * np.abs(np.asarray(b, np.float64))
    assert np.all(d <= lim), f"{what}: max abs diff {d.max():.3e}"
    return float(d.max())


@pytest.fixture(scope="module")
def T():
    import tinyminigo_amd as T
    return T


@pytest.fixture(scope="module")
def O():
    from oracle import oracle as O
    return O


@pytest.fixture(scope="module")
def W():
    from tinyminigo_amd import workloads as W
    return W


@pytest.fixture(scope="module")
def untied_path(W):
    wl = dataclasses.replace(W.TINY, name="tiny-llama-untied-s11", tied_lm_head=False, weight_seed=11,
                             rope_theta=500.0, rms_norm_eps=1e-5)
    return W.ensure_model(wl, model_root())


@pytest.mark.parametrize("out,inp", [(2048, 2048), (6144, 2048), (2048, 6144), (24, 64), (100, 136), (8, 10240),
                                     (1, 8), (2560, 4096), (16, 2056)])
def test_gemv_f32_vs_oracle(T, O, out, inp):
    from tinyminigo_amd.hip import DeviceBuffer, synchronize
    print(f"gemv f32 {out}x{inp}", flush=True)
    rng = np.random.default_rng(out * 7 + inp)
    w = (rng.standard_normal((out, inp)) * 0.02).astype(np.float32)
    x = rng.standard_normal(inp).astype(np.float32)
    want = O.matmul_w_f32(x, w, out, inp)
    wd, xd = DeviceBuffer.from_array(w), DeviceBuffer.from_array(x)
    yd = DeviceBuffer(out * 4)
    yd.fill_byte(0xFF)  # NaN pattern: every row must be written
    T.gemv_f32(wd.addr, xd.addr, yd.addr, out, inp)
    synchronize()
    got = yd.to_array(np.float32, out)
    exact = w.astype(np.float64) @ x.astype(np.float64)
    mag = np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(got - exact) <= 2e-6 * mag + 1e-30)
    assert np.abs(got - want).max() <= 1e-4


def test_gemv_f32_partial_chunk_inf_weight(T, O):
    # the clamped copies a partial last chunk loads must add nothing
    from tinyminigo_amd.hip import DeviceBuffer, synchronize
    out, inp = 16, 2056
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((out, inp)) * 0.02).astype(np.float32)
    w[:, inp - 1] = np.inf
    x = rng.standard_normal(inp).astype(np.float32)
    x[inp - 1] = 1.0
    wd, xd, yd = DeviceBuffer.from_array(w), DeviceBuffer.from_array(x), DeviceBuffer(out * 4)
    T.gemv_f32(wd.addr, xd.addr, yd.addr, out, inp)
    synchronize()
    got = yd.to_array(np.float32, out)
    assert np.all(np.isposinf(got)), got
    assert np.all(np.isposinf(O.matmul_w_f32(x, w, out, inp)))


def _check_model(T, O, path, n_prompt=20, n_steps=24, what=""):
    g, o = T.Model.load(path), O.OracleModel.load(path)
    V = g.config.vocab_size
    ids = [int(t) for t in T.synth_tokens(31, n_prompt + n_steps, V)]
    gc, oc = T.KvCache(g, n_prompt + n_steps + 8), o.new_cache()
    close_logits(g.forward_seq(ids[:n_prompt], gc), o.forward_seq(ids[:n_prompt], oc), f"{what} prefill")
    for i, t in enumerate(ids[n_prompt:]):
        close_logits(g.forward_token(t, gc), o.forward_token(t, oc), f"{what} decode {i}")
    for layer in range(g.config.num_hidden_layers):
        assert np.abs(gc.keys_flat(layer) - oc.keys_flat(layer)).max() < 1e-4
        assert np.abs(gc.values_flat(layer) - oc.values_flat(layer)).max() < 1e-4
    prompt = ids[:n_prompt]
    want = O.generate(o, prompt, 24).tokens
    assert T.generate(g, prompt, T.GenParams(max_tokens=24)).tokens == want, what
    return g


@pytest.mark.parametrize("kind", ["f32", "f16", "mixed", "f32_exact"])
def test_f32_models_vs_oracle(T, O, untied_path, kind):
    print(f"f32 model {kind}", flush=True)
    _check_model(T, O, variant(untied_path, model_root(), kind), what=kind)


def test_f32_file_of_bf16_values_matches_bf16_model(T, untied_path):
    # the f32 rows hold the BF16 values exactly, so the logits agree with the
    # BF16 model to the f32 summation order
    a = T.Model.load(untied_path)
    b = T.Model.load(variant(untied_path, model_root(), "f32_exact"))
    ids = [int(t) for t in T.synth_tokens(33, 24, a.config.vocab_size)]
    ca, cb = T.KvCache(a, 40), T.KvCache(b, 40)
    la, lb = a.forward_seq(ids[:16], ca), b.forward_seq(ids[:16], cb)
    assert np.abs(la - lb).max() < 1e-4
    for t in ids[16:]:
        assert np.abs(a.forward_token(t, ca) - b.forward_token(t, cb)).max() < 1e-4


def test_tied_f32_embedding_vs_oracle(T, O, tiny_path):
    print("tied f32 embedding", flush=True)
    g = _check_model(T, O, variant(tiny_path, model_root(), "tied_f32"), what="tied f32")
    assert g.config.tied_lm_head


def test_f32_long_prompt_and_wide_heads(T, O, W):
    # hidden 2048, head_dim 128 (the 1B shapes, 2 layers, vocab 1024): a
    # 300-token prompt takes the fp32-MFMA GEMM at K = 2048 and 6144 and the
    # MFMA prefill attention; decode the f32-row GEMVs at one and three chunks
    wl = dataclasses.replace(W.ONE_B, name="mid-h2048-l2-v1024", num_hidden_layers=2, vocab_size=1024,
                             weight_seed=17)
    p = variant(W.ensure_model(wl, model_root()), model_root(), "f32")
    print("f32 mid model", flush=True)
    _check_model(T, O, p, n_prompt=300, n_steps=8, what="mid f32")


def test_i8_from_f32_vs_oracle(T, O, untied_path, monkeypatch):
    # TMG_I8=1 quantizes an F32 matrix from its f32 values (src/model.rs:69-72)
    p = variant(untied_path, model_root(), "f32")
    monkeypatch.setenv("TMG_I8", "1")
    g = T.Model.load(p)
    o = O.OracleModel.load(p, i8=True)
    ids = [int(t) for t in T.synth_tokens(35, 28, g.config.vocab_size)]
    gc, oc = T.KvCache(g, 40), o.new_cache()
    close_logits(g.forward_seq(ids[:16], gc), o.forward_seq(ids[:16], oc), "i8 prefill")
    for i, t in enumerate(ids[16:]):
        close_logits(g.forward_token(t, gc), o.forward_token(t, oc), f"i8 decode {i}")
    prompt = ids[:16]
    assert T.generate(g, prompt, T.GenParams(max_tokens=16)).tokens == O.generate(o, prompt, 16).tokens


def test_batch_rejects_f32_models(T, untied_path):
    g = T.Model.load(variant(untied_path, model_root(), "f32"))
    with pytest.raises(T.TmgError, match="f32 weight matrices"):
        T.generate_batch(g, [[1, 2], [3]], 4)
