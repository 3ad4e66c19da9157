"""The measurement entry points (no counterpart in the reference):
tmg_profile_decode_step and tmg_profile_step_floor leave the cache as they
found it, so the decode that follows them gives the logits of a cache that
was never profiled (bit for bit: the same kernels on the same rows), and
their records describe the step's kernels."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def T():
    import tinyminigo_amd as T
    return T


def _prefilled(T, m, ids, cap):
    c = T.KvCache(m, cap)
    lg = m.forward_seq(ids, c)
    return c, int(np.argmax(lg))


def test_profiles_leave_the_cache_as_it_was(T, tiny_path):
    m = T.Model.load(tiny_path)
    V, L = m.config.vocab_size, m.config.num_hidden_layers
    ids = [int(t) for t in T.synth_tokens(5, 20, V)]
    a, tok = _prefilled(T, m, ids, 64)
    b, tok_b = _prefilled(T, m, ids, 64)
    assert tok == tok_b
    print("profile_decode_step", flush=True)
    recs = m.profile_decode_step(tok, a)
    names = [r[0] for r in recs]
    assert names[:5] == ["gemv_qkv_rope", "attn_decode", "gemv_o_resid", "gemv_gateup_swiglu", "gemv_down_resid"]
    assert all(r[2] > 0 for r in recs)
    assert [r[3] for r in recs if r[0] == "gemv_qkv_rope"] == [L]
    print("profile_step_floor", flush=True)
    f = m.profile_step_floor(tok, a)
    assert f["step_ms"] > 0 and f["floor_ms"] > 0 and f["empty_launch_ms"] > 0
    kinds = {k[0]: k for k in f["kinds"]}
    assert list(kinds) == names
    for name, nbytes, fbytes, fms, launches, nwg in f["kinds"]:
        assert fms > 0 and nwg >= 1 and launches >= 1
        # the phase reads the launch's bytes to the nearest 4 KiB per workgroup
        assert abs(fbytes - max(nbytes, 2048 * nwg)) <= 2048 * nwg, name
    # the profiled cache decodes exactly as the untouched one
    for layer in range(L):
        assert np.array_equal(a.keys_flat(layer), b.keys_flat(layer))
    for _ in range(6):
        la, lb = m.forward_token(tok, a), m.forward_token(tok, b)
        assert np.array_equal(la, lb)
        tok = int(np.argmax(la))
    a.close()
    b.close()
    m.close()


def test_step_floor_needs_free_rows(T, tiny_path):
    # nine replays of the step append rows past the length: a cache without
    # room for them is refused before anything runs
    m = T.Model.load(tiny_path)
    ids = [int(t) for t in T.synth_tokens(6, 20, m.config.vocab_size)]
    c, tok = _prefilled(T, m, ids, 26)
    with pytest.raises(T.TmgError, match="too short"):
        m.profile_step_floor(tok, c)
    assert c.len(0) == 20
    c.close()
    m.close()


def test_profile_stream(T):
    # 8 MiB in 32 KiB workgroups: 256 workgroups, exactly the bytes asked
    us, got = T.profile_stream(8 << 20, 32)
    assert got == 8 << 20 and 0.5 < us < 1000.0
    # rounded up to whole workgroups
    _, got = T.profile_stream((8 << 20) + 1, 32)
    assert got == (8 << 20) + 32768
    for kib in (0, 2, 6, 132):
        with pytest.raises(T.TmgError, match="wg_kib"):
            T.profile_stream(1 << 20, kib)
