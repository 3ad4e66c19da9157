"""GPU side of the TMB1 format (reference src/tmb.rs, load_model_tmb at
src/model.rs:105-179): a model loaded from a TMB file -- written by the
library or by the oracle's restatement of write_tmb -- holds the same bits
in HBM as the one loaded from safetensors, so every logit, cache row and
token matches bit for bit.  TMG_I8 does not apply to TMB files (the
reference's TMB loader has no int8 path)."""
import os
import time

import numpy as np
import pytest

from conftest import model_root

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def T():
    import tinyminigo_amd as T
    return T


@pytest.fixture(scope="module")
def W():
    from tinyminigo_amd import workloads as W
    return W


def _untied(W):
    import dataclasses
    return W.ensure_model(dataclasses.replace(W.TINY, name="tiny-llama-untied-s11", tied_lm_head=False,
                                              weight_seed=11, rope_theta=500.0, rms_norm_eps=1e-5), model_root())


def _same_run(T, a, b, vocab, n_decode=20):
    ids = [int(t) for t in T.synth_tokens(51, 16 + n_decode, vocab)]
    ca, cb = T.KvCache(a, 64), T.KvCache(b, 64)
    assert np.array_equal(a.forward_seq(ids[:16], ca), b.forward_seq(ids[:16], cb))
    for t in ids[16:]:
        assert np.array_equal(a.forward_token(t, ca), b.forward_token(t, cb))
    for layer in (0, 1):
        assert np.array_equal(ca.keys_flat(layer), cb.keys_flat(layer))
        assert np.array_equal(ca.values_flat(layer), cb.values_flat(layer))


@pytest.mark.parametrize("which", ["tied", "untied"])
@pytest.mark.parametrize("writer", ["library", "oracle"])
def test_tmb_model_is_bitwise_the_safetensors_model(T, W, tiny_path, tmp_path, which, writer):
    src = tiny_path if which == "tied" else _untied(W)
    dst = str(tmp_path / "m.tmb")
    if writer == "library":
        T.repack_tmb(src, dst)
    else:
        from oracle import tmb as OT
        OT.write_tmb(src, dst)
    print(f"tmb {which} {writer}", flush=True)
    a, b = T.Model.load(src), T.Model.load(dst)
    ca, cb = a.config, b.config
    assert (ca.hidden_size, ca.num_hidden_layers, ca.vocab_size, ca.tied_lm_head) == \
        (cb.hidden_size, cb.num_hidden_layers, cb.vocab_size, cb.tied_lm_head)
    assert cb.eos_token_ids == []
    _same_run(T, a, b, ca.vocab_size)
    prompt = [int(t) for t in T.synth_tokens(52, 12, ca.vocab_size)]
    assert T.generate(a, prompt, T.GenParams(max_tokens=24)).tokens == \
        T.generate(b, prompt, T.GenParams(max_tokens=24)).tokens


def test_tmb_ignores_int8_mode(T, W, tmp_path):
    src = _untied(W)
    dst = str(tmp_path / "m.tmb")
    T.repack_tmb(src, dst)
    old = os.environ.get("TMG_I8")
    os.environ["TMG_I8"] = "1"
    try:
        b = T.Model.load(dst)
        q = T.Model.load(src)
    finally:
        if old is None:
            del os.environ["TMG_I8"]
        else:
            os.environ["TMG_I8"] = old
    a = T.Model.load(src)
    _same_run(T, a, b, a.config.vocab_size, n_decode=4)
    ids = [int(t) for t in T.synth_tokens(53, 16, a.config.vocab_size)]
    assert not np.array_equal(q.forward_seq(ids, T.KvCache(q, 32)), b.forward_seq(ids, T.KvCache(b, 32)))


def test_one_b_from_tmb(T, W, tmp_path):
    src = W.ensure_model(W.ONE_B, model_root())
    dst = str(tmp_path / "1b.tmb")
    t0 = time.perf_counter()
    T.repack_tmb(src, dst)
    t_repack = time.perf_counter() - t0
    times = {}
    for name, path in (("safetensors", src), ("tmb", dst), ("safetensors2", src), ("tmb2", dst)):
        t0 = time.perf_counter()
        m = T.Model.load(path)
        times[name] = time.perf_counter() - t0
        if name == "safetensors2":
            a = m
        elif name == "tmb2":
            b = m
        else:
            del m
    print(f"1B load s: {times}, repack {t_repack:.2f} s, file {os.path.getsize(dst)} B", flush=True)
    prompt = [int(t) for t in W.ONE_B.prompt()]
    ca, cb = T.KvCache(a, 96), T.KvCache(b, 96)
    assert np.array_equal(a.forward_seq(prompt, ca), b.forward_seq(prompt, cb))
    ta, _ = a.decode_greedy(1, 16, ca)
    tb, _ = b.decode_greedy(1, 16, cb)
    assert list(ta) == list(tb)
