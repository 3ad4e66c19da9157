"""GPU parity of the int8 weight-only mode (TMG_I8=1 at load, reference
src/model.rs:57-76): the load-time quantizer and the int8 decode GEMV against
the oracle bit for bit -- the codes, the scales and the integer dots are
exact, and the f32 steps around them are the same IEEE operations in the same
order -- and whole models at the decode path's logit tolerance with greedy
ids identical."""
import os

import numpy as np
import pytest

from conftest import model_root
from test_gpu_parity import close_logits

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


def load_i8(T, path):
    old = os.environ.get("TMG_I8")
    os.environ["TMG_I8"] = "1"
    try:
        return T.Model.load(path)
    finally:
        if old is None:
            del os.environ["TMG_I8"]
        else:
            os.environ["TMG_I8"] = old


def bf16_bits(v):
    return (np.asarray(v, np.float32).view(np.uint32) >> 16).astype(np.uint16)


# --- kernel level -------------------------------------------------------------

@pytest.mark.parametrize("rows,inp", [(64, 64), (3072, 2048), (2048, 6144), (160, 96), (8, 16384)])
def test_quantize_i8_vs_oracle(T, O, rows, inp):
    from tinyminigo_amd.hip import DeviceBuffer, synchronize
    print(f"quantize {rows}x{inp}", flush=True)
    w = T.synth_normal_bf16(7, f"q{rows}x{inp}", rows * inp, 0.02).reshape(rows, inp)
    if rows >= 8:
        w[3] = 0  # zero row: scale 1.0
        w[5, :3] = bf16_bits([0.06640625, -0.033203125, 0.0])  # an exact half, decided in f32
        w[5, 3:] = 0
    w = np.ascontiguousarray(w.reshape(-1))
    wq, ws = O.quantize_i8_bf16(w, rows, inp)
    wd, qd, sd = DeviceBuffer.from_array(w), DeviceBuffer(rows * inp), DeviceBuffer(rows * 4)
    qd.fill_byte(0x55)
    sd.fill_byte(0xFF)
    T.quantize_i8(wd.addr, rows, inp, qd.addr, sd.addr)
    synchronize()
    got_q = qd.to_array(np.int8, rows * inp)
    got_s = sd.to_array(np.float32, rows)
    assert np.array_equal(got_s.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(got_q, wq)
    assert np.array_equal(wd.to_array(np.uint16, rows * inp), w)  # read only
    if rows >= 8:
        assert got_s[3] == 1.0 and got_q[5 * inp + 1] == -64


@pytest.mark.parametrize("out,inp", [(2048, 2048), (3072, 2048), (12288, 2048), (2048, 6144), (24, 64),
                                     (100, 136), (8, 10240), (1, 8), (2560, 4096), (2560, 9728), (4096, 16384)])
def test_gemv_i8_vs_oracle(T, O, out, inp):
    from tinyminigo_amd.hip import DeviceBuffer, synchronize
    print(f"gemv_i8 {out}x{inp}", flush=True)
    w = T.synth_normal_bf16(2, f"w{out}x{inp}", out * inp, 0.02)
    x = T.synth_normal_f32(2, f"x{inp}", inp, 1.0)
    q, s = O.quantize_i8_bf16(w, out, inp)
    want = O.matmul_w_i8(x, q, s, out, inp)
    qd, sd, xd = DeviceBuffer.from_array(q), DeviceBuffer.from_array(s), DeviceBuffer.from_array(x)
    yd = DeviceBuffer(out * 4)
    yd.fill_byte(0xFF)  # NaN pattern: every row must be written
    T.gemv_i8(qd.addr, sd.addr, xd.addr, yd.addr, out, inp)
    synchronize()
    got = yd.to_array(np.float32, out)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # and a zero activation (scale 0) gives exact zeros
    zd = DeviceBuffer.from_array(np.zeros(inp, np.float32))
    T.gemv_i8(qd.addr, sd.addr, zd.addr, yd.addr, out, inp)
    synchronize()
    assert not yd.to_array(np.float32, out).any()


def test_gemv_i8_rejects_bad_shapes(T):
    from tinyminigo_amd.hip import DeviceBuffer
    b = DeviceBuffer(1 << 16)
    with pytest.raises(T.TmgError, match="multiple of 8"):
        T.gemv_i8(b.addr, b.addr, b.addr, b.addr, 4, 12)
    with pytest.raises(T.TmgError, match="16384"):
        T.gemv_i8(b.addr, b.addr, b.addr, b.addr, 4, 16392)
    with pytest.raises(T.TmgError, match="aligned"):
        T.gemv_i8(b.addr + 4, b.addr, b.addr, b.addr, 4, 64)


# --- model level --------------------------------------------------------------

@pytest.fixture(scope="module")
def untied_i8(T, O, W):
    import dataclasses
    wl = dataclasses.replace(W.TINY, name="tiny-llama-untied-s11", tied_lm_head=False, weight_seed=11,
                             rope_theta=500.0, rms_norm_eps=1e-5)
    p = W.ensure_model(wl, model_root())
    return load_i8(T, p), O.OracleModel.load(p, i8=True), T.Model.load(p), wl


def test_i8_teacher_forced_logits_vs_oracle(T, O, untied_i8):
    g, o, g_bf16, wl = untied_i8
    ids = [int(t) for t in T.synth_tokens(21, 80, wl.vocab_size)]
    gc, oc = T.KvCache(g, 128), o.new_cache()
    close_logits(g.forward_seq(ids[:20], gc), o.forward_seq(ids[:20], oc), "i8 prefill 20")
    for i, t in enumerate(ids[20:60]):
        close_logits(g.forward_token(t, gc), o.forward_token(t, oc), f"i8 decode {i}")
    close_logits(g.forward_seq(ids[60:80], gc), o.forward_seq(ids[60:80], oc), "i8 prefill at 60")
    # one-token prompt: the dequantizing path of a 1-row batch
    close_logits(g.forward_seq(ids[:1], T.KvCache(g, 8)), o.forward_seq(ids[:1], o.new_cache()), "i8 prefill 1")
    # the int8 path is what runs: its logits sit far closer to the int8
    # oracle than to the BF16 model's
    a = g.forward_seq(ids[:20], T.KvCache(g, 32))
    b = o.forward_seq(ids[:20], o.new_cache())
    c = g_bf16.forward_seq(ids[:20], T.KvCache(g_bf16, 32))
    assert np.abs(a - b).max() * 20 < np.abs(a - c).max()


def test_i8_tiled_prefill_vs_oracle(T, O, untied_i8):
    """A 300-token prompt takes the tiled MFMA GEMMs, whose epilogues apply the
    int8 row scales with vector loads: logits and K/V rows against the int8
    oracle, then greedy decode steps on that cache."""
    g, o, _, wl = untied_i8
    ids = [int(t) for t in T.synth_tokens(25, 306, wl.vocab_size)]
    gc, oc = T.KvCache(g, 320), o.new_cache()
    print("i8 prefill 300", flush=True)
    close_logits(g.forward_seq(ids[:300], gc), o.forward_seq(ids[:300], oc), "i8 prefill 300")
    for i, t in enumerate(ids[300:]):
        close_logits(g.forward_token(t, gc), o.forward_token(t, oc), f"i8 decode after 300, step {i}")


def test_i8_generate_greedy_vs_oracle(T, O, untied_i8):
    g, o, _, wl = untied_i8
    prompt = [int(t) for t in T.synth_tokens(23, 16, wl.vocab_size)]
    out = T.generate(g, prompt, T.GenParams(max_tokens=40))
    ref = O.generate(o, prompt, 40)
    close_logits(out.logits_first_step, ref.logits_first_step, "i8 first logits")
    assert out.tokens == ref.tokens
    c = T.KvCache(g, 64)
    g.forward_seq(prompt, c)
    toks, _ = g.decode_greedy(ref.tokens[0], 39, c)
    assert list(toks) == ref.tokens[1:]


@pytest.mark.parametrize("temp,k,p,pen,seed", [(0.8, 50, 0.9, 1.1, 42), (0.9, 0, 0.9, 1.0, 3), (1.2, 200, 1.0, 1.2, 9)])
def test_i8_sampling_teacher_forced(T, O, untied_i8, temp, k, p, pen, seed):
    # int8 weights with both sampling paths: replaying the sampled ids, each
    # step's GPU logits are within tolerance of the int8 oracle's, and the
    # oracle's sample() on the GPU's logits with the reference's StdRng draw
    # picks the GPU's id (a free-running comparison would diverge for good
    # after one draw boundary, which the int8 logit differences make likelier)
    g, o, _, wl = untied_i8
    prompt = [int(t) for t in T.synth_tokens(27, 12, wl.vocab_size)]
    n = 32
    out = T.generate(g, prompt, T.GenParams(max_tokens=n, temperature=temp, top_k=k, top_p=p,
                                            repetition_penalty=pen, seed=seed))
    ref = O.generate(o, prompt, n, forced=out.tokens, repetition_penalty=pen, keep_logits=True)
    draws = O.stdrng_uniform(seed, n)
    gc = T.KvCache(g, len(prompt) + n + 2)
    lg = g.forward_seq(prompt, gc)
    for i, tok in enumerate(out.tokens):
        lp = O.apply_repetition_penalty(lg, out.tokens[:i], pen) if i else np.asarray(lg, np.float32)
        close_logits(lp, ref.step_logits[i], f"i8 sampled step {i}")
        # the same logits and the same draw: the reference's id, exactly
        assert O.sample(lp, temp, k, p, float(draws[i])).token == tok, f"i8 sampled step {i}"
        lg = g.forward_token(tok, gc)


def test_i8_k_not_multiple_of_64(T, O, W):
    import dataclasses
    wl = dataclasses.replace(W.TINY, name="tiny-llama-h96-kv3-i160-s13", hidden_size=96, num_attention_heads=6,
                             num_key_value_heads=3, intermediate_size=160, weight_seed=13)
    p = W.ensure_model(wl, model_root())
    g, o = load_i8(T, p), O.OracleModel.load(p, i8=True)
    ids = [int(t) for t in T.synth_tokens(24, 46, wl.vocab_size)]
    for n in (40, 7):
        gc, oc = T.KvCache(g, 64), o.new_cache()
        close_logits(g.forward_seq(ids[:n], gc), o.forward_seq(ids[:n], oc), f"i8 h96 prefill {n}")
        for i, t in enumerate(ids[n:n + 6]):
            close_logits(g.forward_token(t, gc), o.forward_token(t, oc), f"i8 h96 decode {n}+{i}")


def test_i8_one_b_prefill_and_decode_noise_band(T, O, W):
    # Prefill multiplies by the dequantized weights without quantizing the
    # activations, so it is held to the BF16 tolerance.  Decode quantizes every
    # projection input, and at this size a last-bit difference in an
    # activation (the GPU's RMSNorm and attention sum in another order) flips
    # a code somewhere and the flip cascades through the layers: the oracle's
    # own logits move by the full activation-quantization effect under 1e-7
    # noise (test_oracle_i8.py::test_i8_decode_is_chaotic_at_scale).  The bar
    # for decode is therefore that the GPU stays inside that band: its
    # distance to the int8 oracle is at most a few times the distance between
    # the oracle's quantized decode and its unquantized (prefill) logits for
    # the same sequence, far below what a wrong weight, scale or row gives.
    p = W.ensure_model(W.ONE_B, model_root())
    g, o = load_i8(T, p), O.OracleModel.load(p, i8=True)
    prompt = [int(t) for t in W.ONE_B.prompt()]
    gc, oc = T.KvCache(g, 128), o.new_cache()
    lg, lo = g.forward_seq(prompt, gc), o.forward_seq(prompt, oc)
    close_logits(lg, lo, "i8 1B prefill")
    seq, tok = list(prompt), int(np.argmax(lo))
    dg, dq = [], []
    for i in range(6):
        a, b = g.forward_token(tok, gc), o.forward_token(tok, oc)
        seq.append(tok)
        c = o.forward_seq(seq, o.new_cache())
        dg.append(float(np.abs(a - b).max()))
        dq.append(float(np.abs(b - c).max()))
        tok = int(np.argmax(b))
    print("i8 1B decode: |gpu - oracle|", ["%.3f" % v for v in dg], "|oracle - unquantized|",
          ["%.3f" % v for v in dq], flush=True)
    assert np.mean(dg) <= 3.0 * np.mean(dq)
    assert max(dg) < 0.25 * float(np.abs(lo).max())
    # the device loop (graph replay + on-device argmax) follows the host
    # argmax of the same model's forward_token chain
    out = T.generate(g, prompt, T.GenParams(max_tokens=8))
    c2 = T.KvCache(g, 128)
    lg = g.forward_seq(prompt, c2)
    for i, t in enumerate(out.tokens):
        assert t == int(np.argmax(lg)), f"step {i}"
        lg = g.forward_token(t, c2)
