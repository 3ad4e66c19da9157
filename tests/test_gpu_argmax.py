"""A15 argmax on the GPU: the reference rule (src/tensor.rs:1063-1073) exactly.

The rule: scan from (index 0, -inf), take an index when its value is strictly
greater.  So the first of equal maxima wins, NaN is never taken, -0.0 equals
+0.0, and a vector of -inf/NaN (or an empty one) gives 0.

* Kernel level (tmg_argmax_f32): crafted vectors, the reference's own known
  answers (src/tensor.rs:1308-1312) and random vectors of ragged sizes against
  the oracle's argmax.
* Decode path (lm_head GEMV epilogue keys + finalize_kernel): tiny untied
  models whose lm_head rows are crafted so that every logit is one exact
  product (a single non-zero weight per row), so GPU and oracle logits are
  bitwise equal and ties are real ties; greedy ids must equal the oracle's.
"""
import dataclasses
import json
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

NAN, INF = float("nan"), float("inf")


@pytest.fixture(scope="module")
def T():
    import tinyminigo_amd as T
    return T


@pytest.fixture(scope="module")
def O():
    from oracle import oracle as O
    return O


def dev_argmax(T, x):
    from tinyminigo_amd.hip import DeviceBuffer, synchronize
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    xd = DeviceBuffer.from_array(x) if x.size else DeviceBuffer(4)
    out = DeviceBuffer(4)
    out.fill_byte(0xAB)
    T.argmax_f32(xd.addr, x.size, out.addr)
    synchronize()
    return int(out.to_array(np.uint32, 1)[0])


CRAFTED = [
    ([0.1, 3.0, 2.0], 1),           # reference argmax_basic
    ([2.0, 2.0], 0),                # reference: tie -> lowest index
    ([], 0),
    ([-5.0], 0),
    ([-INF, -INF, -INF], 0),
    ([NAN, NAN], 0),
    ([NAN, -INF, NAN], 0),
    ([NAN, 1.0, NAN], 1),
    ([-INF, -3.0, -INF], 1),
    ([-0.0, 0.0], 0),               # equal under `>`: the first wins
    ([0.0, -0.0], 0),
    ([-1.0, -0.0, 0.0, -0.0], 1),
    ([1.0, INF, INF], 1),
    ([NAN, INF], 1),
    ([3.4028235e38, 3.4028235e38, -3.4028235e38], 0),
    ([-3.4028235e38, -INF], 0),
    ([1e-45, 0.0, -1e-45], 0),      # smallest subnormals
    ([0.0, 1e-45], 1),
]


@pytest.mark.parametrize("x,want", CRAFTED)
def test_argmax_crafted(T, O, x, want):
    assert O.argmax(x) == want  # the oracle follows the same rule
    assert dev_argmax(T, x) == want


def test_argmax_ties_across_chunks(T, O):
    # equal maxima in different 4096-element chunks and at a chunk boundary
    rng = np.random.default_rng(5)
    x = rng.standard_normal(73448).astype(np.float32)
    for idx in (60000, 9000, 5000):
        x[idx] = 7.5
    assert dev_argmax(T, x) == O.argmax(x) == 5000
    x[4095] = x[4096] = 9.0
    assert dev_argmax(T, x) == O.argmax(x) == 4095
    x[:] = -INF
    x[73447] = -1.0
    assert dev_argmax(T, x) == 73447
    x[::3] = NAN
    assert dev_argmax(T, x) == O.argmax(x)


@pytest.mark.parametrize("n", [1, 2, 255, 256, 4095, 4096, 4097, 12345, 73448, 131079])
def test_argmax_random_vs_oracle(T, O, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    x[rng.integers(0, n, size=max(1, n // 50))] = NAN
    # a few duplicated maxima
    m = float(np.nanmax(x)) if n > 1 else 0.0
    x[rng.integers(0, n, size=3)] = m
    assert dev_argmax(T, x) == O.argmax(x)


# --- through the decode step: crafted lm_head rows ---------------------------

BF_ONE, BF_MINUS_ONE, BF_NAN = 0x3F80, 0xBF80, 0x7FC0


def rewrite_tensor(path, name, data: np.ndarray):
    with open(path, "r+b") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        hdr = json.loads(f.read(n))
        b, e = hdr[name]["data_offsets"]
        raw = np.ascontiguousarray(data).tobytes()
        assert e - b == len(raw)
        f.seek(8 + n + b)
        f.write(raw)


def crafted_model(T, tmp_path, kind):
    from tinyminigo_amd import workloads as W
    wl = dataclasses.replace(W.TINY, name=f"tiny-argmax-{kind}", tied_lm_head=False, weight_seed=21)
    path = T.synth_model(str(tmp_path / kind), **wl.spec())
    V, H = wl.vocab_size, wl.hidden_size
    lm = np.zeros((V, H), np.uint16)
    col = 5
    if kind == "ties":      # logits: 0 | +x5 (rows 100..299) | -x5 (rows 300..499) | 0
        lm[100:300, col] = BF_ONE
        lm[300:500, col] = BF_MINUS_ONE
    elif kind == "nan_rows":  # rows 0..49 NaN, then the "ties" pattern
        lm[0:50, col] = BF_NAN
        lm[100:300, col] = BF_ONE
        lm[300:500, col] = BF_MINUS_ONE
    elif kind == "all_nan":
        lm[:, col] = BF_NAN
    # "zeros": every logit is a signed zero
    rewrite_tensor(path, "lm_head.weight", lm)
    return path


@pytest.mark.parametrize("kind", ["ties", "nan_rows", "all_nan", "zeros"])
def test_decode_argmax_on_crafted_logits(T, O, tmp_path, kind):
    path = crafted_model(T, tmp_path, kind)
    g, o = T.Model.load(path), O.OracleModel.load(path)
    prompt = [int(t) for t in T.synth_tokens(1, 16, 1024)]
    n = 12
    got = T.generate(g, prompt, T.GenParams(max_tokens=n)).tokens
    want = O.generate(o, prompt, n).tokens
    assert list(got) == list(want)
    if kind in ("ties", "nan_rows"):
        assert set(got) <= {100, 300}
    else:
        assert list(got) == [0] * n
    # the device's own logits pick the same id as the rule
    c = T.KvCache(g, 64)
    lg = g.forward_seq(prompt, c)
    assert int(T.generate(g, prompt, T.GenParams(max_tokens=1)).tokens[0]) == O.argmax(lg)
    g.close()
