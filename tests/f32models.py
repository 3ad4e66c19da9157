"""Test models with F32 / F16 weight matrices, written from a BF16 synthetic
model: the reference converts such matrices to f32 at load (WMat::F32,
src/model.rs:49-55; F16 via f16_to_f32, src/safetensors_loader.rs:149-173).

    variant(src_path, dst_root, kind) -> path of <dst_root>/<name>/model.safetensors

kinds:
  f32        every weight matrix (q, k, v, o, gate, up, down, lm_head) F32,
             each value the BF16 one times (1 + e), |e| < 2^-9 from a seeded
             stream, so that almost none is a BF16 value
  f32_exact  the same matrices F32 with the BF16 values widened (exact)
  f16        the perturbed values rounded to F16
  mixed      layer 0 F32; layer 1: q F32, k and v BF16, o BF16, gate F16,
             up BF16, down F32; lm_head F32
  tied_f32   no lm_head, the embedding F32 (perturbed): a tied f32 lm_head
Norms stay as the source holds them.
"""
import json
import os
import shutil
import struct

import numpy as np

MATS = ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
        "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight")


def write_safetensors(path, tensors):
    """tensors: name -> (dtype string, shape, raw bytes)."""
    hdr, blobs, off = {}, [], 0
    for name, (dt, shape, raw) in tensors.items():
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(hdr).encode()
    h += b" " * ((8 - (8 + len(h)) % 8) % 8)
    with open(path + ".part", "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"".join(blobs))
    os.replace(path + ".part", path)


def _widen(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def _perturbed(bits, rng):
    w = _widen(bits).astype(np.float64)
    e = rng.uniform(-1.0, 1.0, w.shape) * 2.0 ** -9
    return (w * (1.0 + e)).astype(np.float32)


def _dtype_of(kind, layer, mat):
    if kind in ("f32", "f32_exact"):
        return "F32"
    if kind == "f16":
        return "F16"
    if kind == "mixed":
        if layer == 0:
            return "F32"
        return {"self_attn.q_proj.weight": "F32", "mlp.gate_proj.weight": "F16",
                "mlp.down_proj.weight": "F32"}.get(mat, "BF16")
    return "BF16"


def variant(src_path, dst_root, kind, seed=7):
    from oracle import oracle as O
    d = os.path.join(dst_root, f"{os.path.basename(os.path.dirname(src_path))}-{kind}")
    out = os.path.join(d, "model.safetensors")
    if os.path.exists(out):
        return out
    os.makedirs(d, exist_ok=True)
    src = O.load_safetensors(src_path)
    rng = np.random.default_rng(seed)
    tensors = {}
    for name, t in src.items():
        raw = np.asarray(t.data)
        dt, data = t.dtype, raw
        mat = next((m for m in MATS if name.endswith(m)), None)
        if mat is not None or name == "lm_head.weight":
            layer = int(name.split(".")[2]) if mat else -1
            want = "F32" if (name == "lm_head.weight" and kind in ("mixed", "f32", "f32_exact")) else (
                "F16" if name == "lm_head.weight" and kind == "f16" else _dtype_of(kind, layer, mat))
            if t.dtype == "BF16" and want != "BF16":
                vals = _widen(raw) if kind == "f32_exact" else _perturbed(raw, rng)
                dt, data = want, (vals if want == "F32" else vals.astype(np.float16))
        if kind == "tied_f32" and name == "model.embed_tokens.weight" and t.dtype == "BF16":
            dt, data = "F32", _perturbed(raw, rng)
        if kind == "tied_f32" and name == "lm_head.weight":
            continue
        tensors[name] = (dt, t.shape, np.ascontiguousarray(data).tobytes())
    write_safetensors(out, tensors)
    shutil.copy(os.path.join(os.path.dirname(src_path), "config.json"), os.path.join(d, "config.json"))
    return out
