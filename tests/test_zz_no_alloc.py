"""tmg_argmax_f32_noalloc (no device allocation, a fixed per-GPU key array)
against tmg_argmax_f32, through the C ABI.

Two calls in a row, the second smaller: the first leaves larger keys in the
array beyond what the second writes, so a second call that read a stale key
would return an index of the first call's vector.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAX_N = 4096 * 4096


def run(fn_name, x, n=None):
    from tinyminigo_amd._lib import lib
    from tinyminigo_amd.hip import DeviceBuffer, synchronize
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    n = x.size if n is None else n
    xd = DeviceBuffer.from_array(x) if x.size else DeviceBuffer(4)
    out = DeviceBuffer(4)
    out.fill_byte(0xAB)
    rc = getattr(lib, fn_name)(C.c_void_p(xd.addr), n, C.c_void_p(out.addr), None)
    synchronize()
    return rc, int(out.to_array(np.uint32, 1)[0])


def both(x):
    rc_a, a = run("tmg_argmax_f32", x)
    rc_b, b = run("tmg_argmax_f32_noalloc", x)
    assert rc_a == 0 and rc_b == 0
    return a, b


def test_noalloc_two_calls_second_smaller():
    from oracle import oracle as O
    rng = np.random.default_rng(7)
    big = rng.standard_normal(1_000_003).astype(np.float32)
    big[900_000] = 50.0  # in a chunk the second call does not write
    small = rng.standard_normal(70_001).astype(np.float32)
    small[12_345] = 9.0
    small[40_000] = 9.0
    small[::7] = np.nan
    a1, b1 = both(big)
    assert a1 == b1 == O.argmax(big) == 900_000
    _, b2 = run("tmg_argmax_f32_noalloc", small)
    _, a2 = run("tmg_argmax_f32", small)
    assert b2 == a2 == O.argmax(small) == 12_345


def test_noalloc_edges_and_limit():
    assert both([]) == (0, 0)
    assert both([np.nan, -np.inf]) == (0, 0)
    assert both([-0.0, 0.0, 1.0, 1.0]) == (2, 2)
    x = np.full(MAX_N, -1.0, np.float32)
    x[MAX_N - 1] = 3.0
    x[5] = np.inf
    a, b = both(x)
    assert a == b == 5
    from tinyminigo_amd._lib import TMG_E_INVALID
    rc, out = run("tmg_argmax_f32_noalloc", np.zeros(8, np.float32), n=MAX_N + 1)
    assert rc == TMG_E_INVALID and out == 0xABABABAB
