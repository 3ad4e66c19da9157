"""TEST INFRASTRUCTURE ONLY -- the oracle's restatement of the TMB1 format.

Reference: src/tmb.rs (format, parse_tmb_header, write_tmb) and
load_model_tmb (src/model.rs:105-179).  Only tests/ may import this module;
the product's reader and writer are in tinyminigo_amd/csrc/host.

Layout (little-endian), as src/tmb.rs:1-14 and :211-262 write it:
  "TMB1" | cfg_len u64 | n_tensors u32 | config JSON | weights_len u64
  | zero pad to 8 | weights (each tensor 8-aligned, zero padded) | index:
  n x (name_len u32, name, file offset u64, byte length u64) | trailer:
  index_off u64, meta_off u64, weights_len u64, file_size u64.
"""
from __future__ import annotations

import json
import os
import struct
from decimal import Decimal
from typing import Dict, List, Tuple

import numpy as np

from oracle.oracle import (Config, OracleError, Tensor, bf16_to_f32, config_from_json, load_config,
                           load_safetensors)

MAGIC = b"TMB1"  # src/tmb.rs:23
ALIGN = 8  # TENSOR_ALIGN, src/tmb.rs:25

LAYER_TENSORS = [  # consumption order, src/tmb.rs:178-188 (name, stored as raw BF16)
    ("self_attn.q_proj.weight", True), ("self_attn.k_proj.weight", True), ("self_attn.v_proj.weight", True),
    ("self_attn.o_proj.weight", True), ("mlp.gate_proj.weight", True), ("mlp.up_proj.weight", True),
    ("mlp.down_proj.weight", True), ("input_layernorm.weight", False), ("post_attention_layernorm.weight", False),
]


def align_up(n: int) -> int:
    return (n + ALIGN - 1) & ~(ALIGN - 1)


def json_float(x: float) -> str:
    """An f32 config value as serde_json writes the f64 it widens to: the
    shortest round-trip digits (Python's repr gives them), laid out in
    decimal for 1e-5 <= |v| < 1e16 and as d.ddde-N otherwise.  The exact
    spelling of the reference's formatter is not pinned; the value is."""
    x = float(np.float32(x))
    if x == 0.0:
        return "-0.0" if np.signbit(x) else "0.0"
    t = Decimal(repr(abs(x))).normalize().as_tuple()  # value = digits x 10^exponent
    digits = "".join(str(d) for d in t.digits)
    n, k = len(digits), t.exponent
    kk = n + k  # 10^(kk-1) <= |v| < 10^kk
    if k >= 0 and kk <= 16:
        out = digits + "0" * k + ".0"
    elif 0 < kk <= 16:
        out = digits[:kk] + "." + digits[kk:]
    elif -5 < kk <= 0:
        out = "0." + "0" * (-kk) + digits
    elif n == 1:
        out = f"{digits}e{kk - 1}"
    else:
        out = f"{digits[0]}.{digits[1:]}e{kk - 1}"
    return ("-" if x < 0 else "") + out


def config_to_json(c: Config) -> str:
    """ModelConfig::to_json (src/config.rs:92-108) through serde_json::to_string:
    compact, keys sorted (serde_json's default map).  The EOS ids go under
    "eos_token_ids", which from_json does not read back."""
    fields = {
        "hidden_size": str(c.hidden_size), "num_hidden_layers": str(c.num_hidden_layers),
        "num_attention_heads": str(c.num_attention_heads), "num_key_value_heads": str(c.num_key_value_heads),
        "head_dim": str(c.head_dim), "intermediate_size": str(c.intermediate_size),
        "rms_norm_eps": json_float(c.rms_norm_eps), "rope_theta": json_float(c.rope_theta),
        "vocab_size": str(c.vocab_size), "eos_token_ids": "[" + ",".join(str(i) for i in c.eos_token_ids) + "]",
        "bos_token_id": str(c.bos_token_id),
    }
    return "{" + ",".join(f'"{k}":{fields[k]}' for k in sorted(fields)) + "}"


def _f32_bytes(t: Tensor) -> bytes:
    # push_f32 (src/tmb.rs:160-172): BF16 widened, F32/F16 as loaded
    v = bf16_to_f32(np.asarray(t.data)) if t.dtype == "BF16" else np.asarray(t.data, np.float32)
    return np.ascontiguousarray(v, dtype="<f4").tobytes()


def write_tmb(src: str, dst: str) -> None:
    """write_tmb (src/tmb.rs:137-262) with the config read as main.rs does
    for --repack (config.json next to the model, src/main.rs:29-36)."""
    cpath = os.path.join(os.path.dirname(os.path.abspath(src)), "config.json")
    if not os.path.exists(cpath):
        raise OracleError(f"config.json not found next to {src}")
    cfg = load_config(cpath)
    tensors = load_safetensors(src)
    items: List[Tuple[str, bytes]] = []

    def get(name, missing):
        t = tensors.get(name)
        if t is None:
            raise OracleError(missing)
        return t

    def bf16(name, t):
        if t.dtype != "BF16":
            raise OracleError(f"bf16_bytes on non-BF16 tensor {name}")
        return np.ascontiguousarray(t.data, dtype="<u2").tobytes()

    items.append(("model.embed_tokens.weight", _f32_bytes(get("model.embed_tokens.weight",
                                                              "missing embed_tokens.weight"))))
    for l in range(cfg.num_hidden_layers):
        for suffix, is_bf16 in LAYER_TENSORS:
            full = f"model.layers.{l}.{suffix}"
            t = get(full, f"missing {full}")
            items.append((full, bf16(full, t) if is_bf16 else _f32_bytes(t)))
    items.append(("model.norm.weight", _f32_bytes(get("model.norm.weight", "missing model.norm.weight"))))
    if "lm_head.weight" in tensors:
        items.append(("lm_head.weight", bf16("lm_head.weight", tensors["lm_head.weight"])))

    weights = bytearray()
    index = []
    for name, data in items:
        off = align_up(len(weights))
        weights.extend(b"\0" * (off - len(weights)))
        weights.extend(data)
        index.append((name, off, len(data)))
    cfg_bytes = config_to_json(cfg).encode()
    wlen_field = 16 + len(cfg_bytes)
    weights_off = align_up(wlen_field + 8)
    out = bytearray()
    out += MAGIC + struct.pack("<QI", len(cfg_bytes), len(index)) + cfg_bytes
    out += struct.pack("<Q", len(weights)) + b"\0" * (weights_off - (wlen_field + 8)) + weights
    index_off = weights_off + len(weights)
    for name, off, ln in index:
        nb = name.encode()
        out += struct.pack("<I", len(nb)) + nb + struct.pack("<QQ", weights_off + off, ln)
    meta_off = index_off + sum(4 + len(n.encode()) + 16 for n, _, _ in index)
    out += struct.pack("<QQQQ", index_off, meta_off, len(weights), meta_off + 32)
    with open(dst, "wb") as f:
        f.write(out)


def parse_tmb_header(buf: bytes):
    """parse_tmb_header (src/tmb.rs:81-120) -> (config JSON value, {name:
    (file offset, byte length)}).  A repeated name keeps the later entry."""
    if len(buf) < 16:
        raise OracleError("TMB file too small")
    if bytes(buf[:4]) != MAGIC:
        raise OracleError("not a TMB1 file (wrong magic)")
    buf = memoryview(buf).cast("B") if not isinstance(buf, (bytes, bytearray)) else buf
    cfg_len, n = struct.unpack_from("<QI", buf, 4)
    pos = 16
    try:
        cfg_json = json.loads(bytes(buf[pos:pos + cfg_len]).decode())
    except ValueError as e:
        raise OracleError(f"TMB config JSON: {e}")
    pos += cfg_len
    (weights_len,) = struct.unpack_from("<Q", buf, pos)
    pos = align_up(pos + 8) + weights_len
    index: Dict[str, Tuple[int, int]] = {}
    for _ in range(n):
        (nl,) = struct.unpack_from("<I", buf, pos)
        pos += 4
        name = bytes(buf[pos:pos + nl]).decode()
        pos += nl
        off, ln = struct.unpack_from("<QQ", buf, pos)
        pos += 16
        index[name] = (off, ln)
    return cfg_json, index


def load_model_tmb(path: str):
    """load_model_tmb (src/model.rs:105-179) -> (Config, tensors) in the form
    OracleModel takes: weight matrices as raw BF16 views, the embedding and
    norms as the f32 the file stores; no lm_head.weight means tied."""
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    cfg_json, index = parse_tmb_header(mm)
    config = config_from_json(cfg_json)
    tensors: Dict[str, Tensor] = {}
    for name, (off, ln) in index.items():
        raw = mm[off:off + ln]
        if len(raw) != ln:
            raise OracleError("TMB tensor range out of bounds")
        if name.endswith("_proj.weight") or name == "lm_head.weight":
            tensors[name] = Tensor([ln // 2], "BF16", raw.view(np.uint16))
        else:
            tensors[name] = Tensor([ln // 4], "F32", np.array(raw.view(np.float32)))
    emb = tensors.get("model.embed_tokens.weight")
    if emb is None:
        raise OracleError("TMB missing model.embed_tokens.weight")
    if emb.data.size != config.vocab_size * config.hidden_size:
        raise OracleError(f"TMB embed size {emb.data.size} != vocab*hidden "
                          f"{config.vocab_size * config.hidden_size}")
    return config, tensors
