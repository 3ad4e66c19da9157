"""Batched greedy decode (tmg_generate_batch): several prompts share every
decode step (weights streamed once per step for all sequences by the MFMA
GEMM).  For each sequence the ids must be the ones generate
(src/model.rs:614-663) gives for that prompt alone: checked against the
oracle's generate and the library's single-sequence generate, with ragged
prompt lengths, EOS stops and the error paths."""
import json
import os
import shutil

import numpy as np
import pytest

from conftest import model_root

pytestmark = pytest.mark.gpu


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
def untied(T, O, W):
    import dataclasses
    wl = dataclasses.replace(W.TINY, name="tiny-llama-untied-s11", tied_lm_head=False, weight_seed=11,
                             rope_theta=500.0, rms_norm_eps=1e-5)
    p = W.ensure_model(wl, model_root())
    return T.Model.load(p), O.OracleModel.load(p), wl


def test_batch_matches_per_sequence_generate(T, O, untied):
    g, o, wl = untied
    lens = [3, 16, 1, 40, 9]
    prompts = [[int(t) for t in T.synth_tokens(60 + i, n, wl.vocab_size)] for i, n in enumerate(lens)]
    print("batch tiny", lens, flush=True)
    got, ms = T.generate_batch(g, prompts, 24)
    assert ms > 0
    for b, p in enumerate(prompts):
        ref = O.generate(o, p, 24).tokens
        assert got[b] == ref, f"sequence {b}"
        assert got[b] == T.generate(g, p, T.GenParams(max_tokens=24)).tokens
    # a batch of one is generate
    one, _ = T.generate_batch(g, prompts[1:2], 24)
    assert one[0] == got[1]
    # max_tokens 1: the prefill's argmax only
    first, _ = T.generate_batch(g, prompts, 1)
    assert [f[0] for f in first] == [r[0] for r in got] and all(len(f) == 1 for f in first)


def test_batch_of_more_than_eight_takes_the_gemm_path(T, O, untied):
    # up to 8 sequences run the multi-row GEMVs, more run the MFMA GEMMs
    g, o, wl = untied
    lens = [1, 2, 3, 5, 8, 13, 21, 34, 7, 4, 9, 30]
    prompts = [[int(t) for t in T.synth_tokens(100 + i, n, wl.vocab_size)] for i, n in enumerate(lens)]
    print("batch tiny x12", flush=True)
    got, _ = T.generate_batch(g, prompts, 16)
    for b, p in enumerate(prompts):
        assert got[b] == O.generate(o, p, 16).tokens, f"sequence {b}"
    # the same sequences in batches of 8 and 4 (GEMV path) agree
    lo, _ = T.generate_batch(g, prompts[:8], 16)
    hi, _ = T.generate_batch(g, prompts[8:], 16)
    assert lo + hi == got


def test_batch_of_more_than_eight_with_norm_hand_off(T, O, W):
    """More than 8 sequences on a model whose hidden size is a multiple of
    256: the MFMA GEMM step hands the RMSNorm from the o_proj / down
    epilogues to the next GEMM (the residual times the norm weight, then
    1/rms on the consumer's dot products), a different rounding from
    forward_token's.  Every sequence's ids must still be the oracle's
    generate, and the library's single-sequence generate for a few."""
    import dataclasses
    wl = dataclasses.replace(W.TINY, name="tiny-llama-h256-q4-k2-d64-i512-s23", hidden_size=256,
                             num_attention_heads=4, num_key_value_heads=2, head_dim=64, intermediate_size=512,
                             tied_lm_head=False, weight_seed=23, rms_norm_eps=1e-5)
    p = W.ensure_model(wl, model_root())
    g, o = T.Model.load(p), O.OracleModel.load(p)
    lens = [1, 4, 9, 16, 25, 36, 2, 3, 40, 7, 11]
    prompts = [[int(t) for t in T.synth_tokens(140 + i, n, wl.vocab_size)] for i, n in enumerate(lens)]
    print("batch hidden 256 x11", flush=True)
    got, _ = T.generate_batch(g, prompts, 20)
    for b, pr in enumerate(prompts):
        assert got[b] == O.generate(o, pr, 20).tokens, f"sequence {b}"
    for b in (0, 5, 10):
        assert got[b] == T.generate(g, prompts[b], T.GenParams(max_tokens=20)).tokens, f"sequence {b} alone"


def test_batch_of_more_than_sixty_four(T, O, W):
    """70 sequences: the step's GEMMs have two token tiles, so they run the
    128-row split-K tiles, with each sequence's own position and cache in
    the QKV epilogue and the RMSNorm handed between the GEMMs (hidden 256).
    Every sequence's ids are the oracle's generate."""
    import dataclasses
    wl = dataclasses.replace(W.TINY, name="tiny-llama-h256-q4-k2-d64-i512-s23", hidden_size=256,
                             num_attention_heads=4, num_key_value_heads=2, head_dim=64, intermediate_size=512,
                             tied_lm_head=False, weight_seed=23, rms_norm_eps=1e-5)
    p = W.ensure_model(wl, model_root())
    g, o = T.Model.load(p), O.OracleModel.load(p)
    lens = [1 + (7 * i) % 40 for i in range(70)]
    prompts = [[int(t) for t in T.synth_tokens(300 + i, n, wl.vocab_size)] for i, n in enumerate(lens)]
    print("batch hidden 256 x70", flush=True)
    got, _ = T.generate_batch(g, prompts, 12)
    for b, pr in enumerate(prompts):
        assert got[b] == O.generate(o, pr, 12).tokens, f"sequence {b}"
    g.close()


def test_batch_tied_and_k_not_multiple_of_64(T, O, W, tiny_path):
    import dataclasses
    wl = dataclasses.replace(W.TINY, name="tiny-llama-h96-kv3-i160-s13", hidden_size=96, num_attention_heads=6,
                             num_key_value_heads=3, intermediate_size=160, weight_seed=13)
    for path, vocab in ((tiny_path, W.TINY.vocab_size), (W.ensure_model(wl, model_root()), wl.vocab_size)):
        g, o = T.Model.load(path), O.OracleModel.load(path)
        prompts = [[int(t) for t in T.synth_tokens(70 + i, n, vocab)] for i, n in enumerate([5, 12, 2])]
        print("batch", path, flush=True)
        got, _ = T.generate_batch(g, prompts, 16)
        for b, p in enumerate(prompts):
            assert got[b] == O.generate(o, p, 16).tokens, f"{path} sequence {b}"


def test_batch_stops_each_sequence_at_eos(T, O, W, tiny_path, tmp_path):
    # an EOS id that sequence 0 emits mid-way: that sequence stops after it
    # (src/model.rs:649-651), the others run on
    g = T.Model.load(tiny_path)
    prompts = [[int(t) for t in T.synth_tokens(80 + i, 8, W.TINY.vocab_size)] for i in range(3)]
    free, _ = T.generate_batch(g, prompts, 20)
    eos = free[0][5]
    d = tmp_path / "m"
    os.makedirs(d)
    shutil.copy(tiny_path, d / "model.safetensors")
    cfg = json.load(open(os.path.join(os.path.dirname(tiny_path), "config.json")))
    cfg["eos_token_id"] = [eos]
    json.dump(cfg, open(d / "config.json", "w"))
    ge = T.Model.load(str(d / "model.safetensors"))
    got, _ = T.generate_batch(ge, prompts, 20)
    for b in range(3):
        want = T.generate(ge, prompts[b], T.GenParams(max_tokens=20)).tokens
        assert got[b] == want
        cut = free[b].index(eos) + 1 if eos in free[b] else 20
        assert got[b] == free[b][:cut]
    assert len(got[0]) == free[0].index(eos) + 1


def test_batch_errors(T, untied):
    g, _, wl = untied
    with pytest.raises(T.TmgError, match="TMG_E_EMPTY"):
        T.generate_batch(g, [[1, 2], []], 4)
    with pytest.raises(T.TmgError, match="out of range"):
        T.generate_batch(g, [[wl.vocab_size]], 4)
    with pytest.raises(T.TmgError, match="n_seq"):
        T.generate_batch(g, [], 4)


def test_batch_one_b(T, O, W):
    p = W.ensure_model(W.ONE_B, model_root())
    g, o = T.Model.load(p), O.OracleModel.load(p)
    lens = [64, 17, 33, 64, 5, 48, 64, 30]
    prompts = [[int(t) for t in T.synth_tokens(90 + i, n, W.ONE_B.vocab_size)] for i, n in enumerate(lens)]
    print("batch 1B", lens, flush=True)
    got, ms = T.generate_batch(g, prompts, 24)
    print(f"batch 1B: 8 x 23 decode steps in {ms:.2f} ms", flush=True)
    for b, pr in enumerate(prompts):
        assert got[b] == O.generate(o, pr, 24).tokens, f"sequence {b}"
