"""Handle lifetime through the C ABI: a model may be freed before its caches.

tmg_model_free with live caches defers the release until the last cache is
freed (include/tmg.h); the cache keeps reading its KV rows in between.  The
Python Model.close() closes the caches made on it.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_model_freed_before_cache(tiny_path):
    import tinyminigo_amd as T
    from tinyminigo_amd._lib import check, lib

    m = C.c_void_p()
    check(lib.tmg_model_load(tiny_path.encode(), 0, C.byref(m)))
    c1, c2 = C.c_void_p(), C.c_void_p()
    check(lib.tmg_cache_new(m, 64, C.byref(c1)))
    check(lib.tmg_cache_new(m, 64, C.byref(c2)))
    ids = np.array([int(t) for t in T.synth_tokens(1, 12, 1024)], np.uint32)
    check(lib.tmg_forward_seq(m, c1, ids.ctypes.data_as(C.POINTER(C.c_uint32)), ids.size, None))
    kvd = 32  # tiny model: 2 KV heads x head_dim 16
    before = np.empty(12 * kvd, np.float32)
    check(lib.tmg_cache_read(c1, 1, before.ctypes.data_as(C.POINTER(C.c_float)), None))
    lib.tmg_model_free(m)  # deferred: two caches are live
    after = np.empty(12 * kvd, np.float32)
    check(lib.tmg_cache_read(c1, 1, after.ctypes.data_as(C.POINTER(C.c_float)), None))
    assert np.array_equal(before, after)
    lib.tmg_cache_free(c1)
    n = C.c_uint32()
    check(lib.tmg_cache_len(c2, 0, C.byref(n)))
    assert n.value == 0
    lib.tmg_cache_free(c2)  # last cache: the model is released here


def test_python_close_closes_caches(tiny_path):
    import tinyminigo_amd as T

    g = T.Model.load(tiny_path)
    c = T.KvCache(g, 32)
    g.forward_seq([1, 2, 3], c)
    g.close()
    assert c._h is None and g._h is None
    c.close()  # idempotent
