"""TMB1 repack format (reference src/tmb.rs; load_model_tmb, src/model.rs:
90-179) on the CPU: the library's writer against the layout the reference
documents and writes, byte for byte against the oracle's restatement, its
header reader and error paths, and the oracle model loaded from a TMB file
against the same model loaded from safetensors (bit for bit).  The GPU side
is in test_gpu_tmb.py."""
import json
import os
import shutil
import struct

import numpy as np
import pytest

import tinyminigo_amd as T
from oracle import oracle as O
from oracle import tmb as OT
from test_host_cpu import _copy_model
from tinyminigo_amd import workloads as W
from conftest import model_root


@pytest.fixture(scope="module")
def untied_path():
    import dataclasses
    wl = dataclasses.replace(W.TINY, name="tiny-llama-untied-s11", tied_lm_head=False, weight_seed=11,
                             rope_theta=500.0, rms_norm_eps=1e-5)
    return W.ensure_model(wl, model_root())


@pytest.fixture(params=["tied", "untied"])
def model(request, tiny_path, untied_path):
    return tiny_path if request.param == "tied" else untied_path


def _u64(b, o):
    return struct.unpack_from("<Q", b, o)[0]


def test_layout_follows_the_reference_writer(model, tmp_path):
    dst = str(tmp_path / "m.tmb")
    T.repack_tmb(model, dst)
    b = open(dst, "rb").read()
    src = O.load_safetensors(model)
    cfg = O.load_config(os.path.join(os.path.dirname(model), "config.json"))
    assert b[:4] == b"TMB1"
    cfg_len, n = _u64(b, 4), struct.unpack_from("<I", b, 12)[0]
    cj = json.loads(b[16:16 + cfg_len])
    wlen_field = 16 + cfg_len
    weights_len = _u64(b, wlen_field)
    weights_off = (wlen_field + 8 + 7) // 8 * 8
    assert b[wlen_field + 8:weights_off] == b"\0" * (weights_off - wlen_field - 8)
    # index right after the weights, trailer after the index
    pos, names, prev_end = weights_off + weights_len, [], weights_off
    for _ in range(n):
        nl = struct.unpack_from("<I", b, pos)[0]
        name = b[pos + 4:pos + 4 + nl].decode()
        off, ln = struct.unpack_from("<QQ", b, pos + 4 + nl)
        pos += 4 + nl + 16
        assert off % 8 == 0 and off >= prev_end and off + ln <= weights_off + weights_len
        assert b[prev_end:off] == b"\0" * (off - prev_end)  # zero padding between tensors
        prev_end = off + ln
        names.append(name)
        t = src[name]
        raw = b[off:off + ln]
        if name.endswith("_proj.weight") or name == "lm_head.weight":
            assert raw == np.ascontiguousarray(t.data).tobytes()  # raw BF16, as stored
        else:
            want = O.bf16_to_f32(np.asarray(t.data)) if t.dtype == "BF16" else np.asarray(t.data, np.float32)
            assert raw == want.astype("<f4").tobytes()  # embedding / norms widened to f32
    assert prev_end == weights_off + weights_len
    index_off, meta_off, wl2, size = struct.unpack_from("<QQQQ", b, pos)
    assert (index_off, meta_off, wl2, size) == (weights_off + weights_len, pos, weights_len, len(b))
    # consumption order (src/tmb.rs:174-200)
    want_names = ["model.embed_tokens.weight"]
    for l in range(cfg.num_hidden_layers):
        want_names += [f"model.layers.{l}.{s}" for s, _ in OT.LAYER_TENSORS]
    want_names.append("model.norm.weight")
    if "lm_head.weight" in src:
        want_names.append("lm_head.weight")
    assert names == want_names
    # ModelConfig::to_json fields
    assert cj["hidden_size"] == cfg.hidden_size and cj["vocab_size"] == cfg.vocab_size
    assert np.float32(cj["rms_norm_eps"]) == np.float32(cfg.rms_norm_eps)
    assert np.float32(cj["rope_theta"]) == np.float32(cfg.rope_theta)
    assert list(cj) == sorted(cj)


def test_library_writer_equals_oracle_writer(model, tmp_path):
    a, b = str(tmp_path / "lib.tmb"), str(tmp_path / "oracle.tmb")
    T.repack_tmb(model, a)
    OT.write_tmb(model, b)
    assert open(a, "rb").read() == open(b, "rb").read()


def test_config_round_trip_drops_eos_like_the_reference(tiny_path, tmp_path):
    src = _copy_model(os.path.dirname(tiny_path), str(tmp_path / "m"))
    cpath = os.path.join(os.path.dirname(src), "config.json")
    cfg = json.load(open(cpath))
    cfg["eos_token_id"] = [2, 7]
    json.dump(cfg, open(cpath, "w"))
    dst = str(tmp_path / "m.tmb")
    T.repack_tmb(src, dst)
    a = T.ModelConfig.load(cpath)
    b = T.ModelConfig.from_tmb(dst)
    assert a.eos_token_ids == [2, 7]
    # written as "eos_token_ids", read back from "eos_token_id" (src/config.rs:
    # 65-75 vs :105): the ids do not survive the round trip
    assert b'"eos_token_ids":[2,7]' in open(dst, "rb").read(400)
    assert b.eos_token_ids == [] and O.config_from_json(OT.parse_tmb_header(open(dst, "rb").read())[0]).eos_token_ids == []
    for f in ("hidden_size", "num_hidden_layers", "num_attention_heads", "num_key_value_heads", "head_dim",
              "intermediate_size", "vocab_size", "bos_token_id", "rms_norm_eps", "rope_theta"):
        assert getattr(a, f) == getattr(b, f), f
    assert b.tied_lm_head


@pytest.mark.parametrize("x", [1e-5, 1e-6, 9.99999997e-07, 10000.0, 500.0, 5e6, 1e-4, 0.5, 3.0e-5, 1e20])
def test_config_floats_round_trip(x):
    s = OT.json_float(x)
    assert np.float32(float(s)) == np.float32(x)
    assert float(s) == float(np.float32(x))  # the f64 the f32 widens to, exactly


def test_oracle_model_from_tmb_is_bitwise_the_safetensors_model(model, tmp_path):
    dst = str(tmp_path / "m.tmb")
    T.repack_tmb(model, dst)
    a, b = O.OracleModel.load(model), O.OracleModel.load(dst)
    assert b.tied == a.tied
    ids = [int(t) for t in T.synth_tokens(41, 24, a.config.vocab_size)]
    ca, cb = a.new_cache(), b.new_cache()
    assert np.array_equal(a.forward_seq(ids[:16], ca), b.forward_seq(ids[:16], cb))
    for t in ids[16:]:
        assert np.array_equal(a.forward_token(t, ca), b.forward_token(t, cb))


def test_tmb_header_errors(tiny_path, tmp_path):
    good = str(tmp_path / "good.tmb")
    T.repack_tmb(tiny_path, good)
    b = open(good, "rb").read()

    def bad(name, data):
        p = str(tmp_path / name)
        open(p, "wb").write(data)
        return p

    with pytest.raises(T.TmgError, match="TMG_E_FORMAT.*too small"):
        T.ModelConfig.from_tmb(bad("short.tmb", b"TMB1" + b"\0" * 8))
    with pytest.raises(T.TmgError, match="wrong magic"):
        T.ModelConfig.from_tmb(bad("magic.tmb", b"TMB2" + b[4:]))
    with pytest.raises(T.TmgError, match="index truncated|past the end"):
        T.ModelConfig.from_tmb(bad("cut.tmb", b[:len(b) - 200]))
    # first index entry's offset pointed past the end of the file
    cfg_len = _u64(b, 4)
    weights_off = (16 + cfg_len + 8 + 7) // 8 * 8
    ipos = weights_off + _u64(b, 16 + cfg_len)
    nl = struct.unpack_from("<I", b, ipos)[0]
    mod = bytearray(b)
    struct.pack_into("<Q", mod, ipos + 4 + nl, len(b) + 8)
    with pytest.raises(T.TmgError, match="out of bounds"):
        T.ModelConfig.from_tmb(bad("range.tmb", bytes(mod)))
    # the model loader reads TMB files too and reports the same before any
    # device work
    with pytest.raises(T.TmgError, match="out of bounds"):
        T.Model.load(str(tmp_path / "range.tmb"))


def test_repack_errors(tiny_path, tmp_path):
    src = os.path.dirname(tiny_path)
    p = _copy_model(src, str(tmp_path / "a"), drop="model.layers.1.mlp.up_proj.weight")
    with pytest.raises(T.TmgError, match="TMG_E_MISSING.*missing model.layers.1.mlp.up_proj.weight"):
        T.repack_tmb(p, str(tmp_path / "a.tmb"))
    with pytest.raises(O.OracleError, match="missing model.layers.1.mlp.up_proj.weight"):
        OT.write_tmb(p, str(tmp_path / "a2.tmb"))
    p = _copy_model(src, str(tmp_path / "b"), dtype_of="model.layers.0.self_attn.q_proj.weight")
    with pytest.raises(T.TmgError, match="TMG_E_DTYPE"):
        T.repack_tmb(p, str(tmp_path / "b.tmb"))
    os.makedirs(tmp_path / "c")
    shutil.copy(tiny_path, tmp_path / "c" / "model.safetensors")
    with pytest.raises(T.TmgError, match="config.json not found"):
        T.repack_tmb(str(tmp_path / "c" / "model.safetensors"), str(tmp_path / "c.tmb"))
