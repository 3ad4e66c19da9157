"""CPU-side tests of the product library: the C ABI loads and exports every
symbol the headers declare, config.json parsing follows src/config.rs, model
files are validated before any device work (so their error paths run without
a GPU), and the synthetic generator is deterministic."""
import ctypes as C
import glob
import hashlib
import json
import os
import re
import struct

import numpy as np
import pytest

import tinyminigo_amd as T
from tinyminigo_amd import _lib
from tinyminigo_amd import workloads as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(tmg_[a-z0-9_]+)\s*\(", text))
    return names - {"tmg_on_token_fn"}


def test_library_exports_every_declared_symbol():
    names = declared_symbols()
    assert len(names) >= 20
    lib = C.CDLL(_lib.LIB_PATH)
    for n in sorted(names):
        assert hasattr(lib, n), f"{n} declared in include/*.h but not exported"
    assert names <= set(_lib.SIGNATURES), "ctypes binding misses a declared entry point"


def test_config_load_matches_reference_kat(tmp_path):
    from test_oracle_kat import TINY_RANDOM_MINICPM5
    p = tmp_path / "config.json"
    p.write_text(json.dumps(TINY_RANDOM_MINICPM5))
    c = T.ModelConfig.load(str(p))
    assert (c.hidden_size, c.num_hidden_layers, c.num_attention_heads, c.num_key_value_heads) == (16, 2, 16, 2)
    assert (c.head_dim, c.intermediate_size, c.vocab_size, c.bos_token_id) == (32, 64, 130560, 0)
    assert c.rms_norm_eps == np.float32(1e-6) and c.rope_theta == 5e6
    assert c.eos_token_ids == [1, 130073]


def test_config_defaults_and_errors(tmp_path):
    p = tmp_path / "config.json"
    p.write_text(json.dumps({"hidden_size": 64, "num_attention_heads": 4, "num_hidden_layers": 1,
                             "intermediate_size": 8, "vocab_size": 10, "rope_theta": 500.0}))
    c = T.ModelConfig.load(str(p))
    assert c.num_key_value_heads == 4 and c.head_dim == 16 and c.rope_theta == 500.0
    assert c.rms_norm_eps == np.float32(1e-5) and c.eos_token_ids == []
    p.write_text(json.dumps({"hidden_size": 64, "num_attention_heads": 4}))
    with pytest.raises(T.TmgError, match="num_hidden_layers"):
        T.ModelConfig.load(str(p))
    p.write_text("{not json")
    with pytest.raises(T.TmgError, match="TMG_E_FORMAT"):
        T.ModelConfig.load(str(p))
    with pytest.raises(T.TmgError, match="TMG_E_IO"):
        T.ModelConfig.load(str(tmp_path / "missing.json"))


def _copy_model(src_dir, dst_dir, mutate=None, drop=None, dtype_of=None, dtype_to="F32"):
    """Rewrite a synthetic model with one tensor dropped or retyped (its BF16
    values widened to f32 and labelled `dtype_to`)."""
    with open(os.path.join(src_dir, "model.safetensors"), "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        hdr = json.loads(f.read(n))
        data = f.read()
    out_hdr, blobs, off = {}, [], 0
    for name, meta in hdr.items():
        if name == "__metadata__" or name == drop:
            continue
        raw = data[meta["data_offsets"][0]:meta["data_offsets"][1]]
        dt = meta["dtype"]
        if name == dtype_of:
            raw = (np.frombuffer(raw, np.uint16).astype(np.uint32) << 16).view(np.float32).tobytes()
            dt = dtype_to
        out_hdr[name] = {"dtype": dt, "shape": meta["shape"], "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(out_hdr).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    os.makedirs(dst_dir, exist_ok=True)
    with open(os.path.join(dst_dir, "model.safetensors"), "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"".join(blobs))
    with open(os.path.join(src_dir, "config.json")) as f:
        cfg = f.read()
    with open(os.path.join(dst_dir, "config.json"), "w") as f:
        f.write(cfg)
    return os.path.join(dst_dir, "model.safetensors")


def test_model_load_error_paths(tiny_path, tmp_path):
    src = os.path.dirname(tiny_path)
    # missing tensor (src/model.rs:43-47)
    p = _copy_model(src, str(tmp_path / "a"), drop="model.layers.1.mlp.up_proj.weight")
    with pytest.raises(T.TmgError, match="missing tensor `model.layers.1.mlp.up_proj.weight`"):
        T.Model.load(p)
    # a weight matrix of a dtype the reference does not read
    # (src/safetensors_loader.rs:137-142)
    p = _copy_model(src, str(tmp_path / "b"), dtype_of="model.layers.0.self_attn.q_proj.weight", dtype_to="I32")
    with pytest.raises(T.TmgError, match="TMG_E_DTYPE.*unsupported dtype I32"):
        T.Model.load(p)
    # an F32 weight matrix is read (WMat::F32, src/model.rs:49-55): validation
    # passes, and without a GPU the load stops at the device
    p = _copy_model(src, str(tmp_path / "b2"), dtype_of="model.layers.0.self_attn.q_proj.weight")
    try:
        T.Model.load(p).close()
    except T.TmgError as e:
        assert "TMG_E_DTYPE" not in str(e), str(e)
    # config.json must sit next to the weights (src/config.rs:174-184)
    os.makedirs(tmp_path / "c", exist_ok=True)
    with open(tmp_path / "c" / "model.safetensors", "wb") as f:
        f.write(open(tiny_path, "rb").read())
    with pytest.raises(T.TmgError, match="config.json not found"):
        T.Model.load(str(tmp_path / "c" / "model.safetensors"))
    # truncated header (src/safetensors_loader.rs:84-95)
    os.makedirs(tmp_path / "d", exist_ok=True)
    with open(tmp_path / "d" / "model.safetensors", "wb") as f:
        f.write(struct.pack("<Q", 1 << 20) + b"{}")
    with open(tmp_path / "d" / "config.json", "w") as f:
        f.write(open(os.path.join(src, "config.json")).read())
    with pytest.raises(T.TmgError, match="header truncated"):
        T.Model.load(str(tmp_path / "d" / "model.safetensors"))


def test_synth_is_deterministic_and_documented(tiny_path):
    # generator documented in include/tmg_synth.h: SplitMix64 counter streams,
    # Box-Muller in double, BF16 round-to-nearest-even
    def mix(z):
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
        return z ^ (z >> 31)

    def fnv(s):
        h = 0xcbf29ce484222325
        for c in s.encode():
            h = ((h ^ c) * 0x100000001b3) & (2**64 - 1)
        return h

    G = 0x9E3779B97F4A7C15
    key = mix(((7 * G) & (2**64 - 1)) ^ fnv("tokens"))
    ids = [(mix((key + (i + 1) * G) & (2**64 - 1)) * 1000) >> 64 for i in range(10)]
    assert list(T.synth_tokens(7, 10, 1000)) == ids
    key = mix(((3 * G) & (2**64 - 1)) ^ fnv("w"))
    vals = []
    for e in range(6):
        a = ((mix((key + (2 * e + 1) * G) & (2**64 - 1)) >> 11) + 1) * 2.0**-53
        b = (mix((key + (2 * e + 2) * G) & (2**64 - 1)) >> 11) * 2.0**-53
        vals.append(np.float32(0.02 * np.sqrt(-2 * np.log(a)) * np.cos(2 * np.pi * b)))
    got = T.synth_normal_bf16(3, "w", 6, 0.02)
    want = np.array(vals, np.float32).view(np.uint32)
    want = ((want + 0x7FFF + ((want >> 16) & 1)) >> 16).astype(np.uint16)
    assert list(got) == list(want)
    x = T.synth_normal_f32(2, "x", 100000, 1.0)
    assert abs(float(x.mean())) < 0.02 and abs(float(x.std()) - 1.0) < 0.02


def test_tiny_model_file_fingerprint(tiny_path):
    # the model every C0 fixture under tests/golden was computed from
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", "tiny_llama.json")))
    h = hashlib.sha256(open(tiny_path, "rb").read()).hexdigest()
    assert h == fx["model_sha256"]


def test_tokens_out_of_range_and_empty_prompt_checked_without_gpu():
    with pytest.raises(T.TmgError):
        T.Model.load("/nonexistent/model.safetensors")
