"""TEST INFRASTRUCTURE ONLY -- the oracle's Python side.

Loads a model the way the reference does and drives the C restatement in
tmg_oracle.c.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module; the product (tinyminigo_amd)
never does.

  - load_config follows ModelConfig::load (reference src/config.rs:112-172);
  - load_safetensors follows load_safetensors (src/safetensors_loader.rs:
    103-147): BF16 kept raw, F16/F32 converted to f32, anything else an error;
  - OracleModel.load follows load_model_safetensors (src/model.rs:181-244);
  - generate follows generate (src/model.rs:614-663), with the sampler's
    uniform draws supplied by the caller (rand::StdRng cannot run here).
"""
from __future__ import annotations

import ctypes as C
import json
import os
import struct
import subprocess
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle.so")


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _load_lib():
    if not os.path.exists(LIB_PATH):
        build()
    lib = C.CDLL(LIB_PATH)
    F, PF, PU16, PU32, S = C.c_float, C.POINTER(C.c_float), C.POINTER(C.c_uint16), C.POINTER(C.c_uint32), C.c_size_t
    PI8 = C.POINTER(C.c_int8)
    sig = {
        "om_set_num_threads": (None, [C.c_int]),
        "om_set_attn_threads": (None, [C.c_int]),
        "om_num_threads": (C.c_int, []),
        "om_uses_avx2": (C.c_int, []),
        "om_dot_bf16": (F, [PF, PU16, S]),
        "om_dot": (F, [PF, PF, S]),
        "om_matmul_w": (None, [PF, PU16, S, S, PF]),
        "om_matmul_batch_w": (None, [PF, PU16, S, S, S, PF]),
        "om_rms_norm": (None, [PF, PF, F, S, PF]),
        "om_rms_norm_batch": (None, [PF, PF, F, S, S]),
        "om_rope_rotate": (None, [PF, S, S, F]),
        "om_rope_table": (None, [S, F, S, PF, PF]),
        "om_softmax": (None, [PF, S, PF]),
        "om_silu": (None, [PF, S, PF]),
        "om_argmax": (S, [PF, S]),
        "om_attention_row": (None, [PF, PF, PF, S, S, S, F, PF]),
        "om_attention_batch": (None, [PF, PF, PF, S, S, S, S, S, PF]),
        "om_apply_repetition_penalty": (None, [PF, S, PU32, S, F]),
        "om_sample": (S, [PF, S, F, S, F, F, PU32, PF, C.POINTER(S)]),
        "om_chacha_block": (None, [PU32, C.c_uint64, C.c_uint64, C.c_int, PU32]),
        "om_pcg_xsh_rr": (C.c_uint32, [C.c_uint64]),
        "om_uniform_f32": (C.c_float, [C.c_uint32]),
        "om_stdrng_key": (None, [C.c_uint64, PU32]),
        "om_stdrng_uniform": (None, [C.c_uint64, S, PF]),
        "om_model_new": (C.c_void_p, [C.c_void_p]),
        "om_model_free": (None, [C.c_void_p]),
        "om_cache_new": (C.c_void_p, [C.c_int, S]),
        "om_cache_free": (None, [C.c_void_p]),
        "om_cache_len": (S, [C.c_void_p, C.c_int]),
        "om_cache_keys": (PF, [C.c_void_p, C.c_int]),
        "om_cache_values": (PF, [C.c_void_p, C.c_int]),
        "om_cache_reset": (None, [C.c_void_p]),
        "om_cache_push": (None, [C.c_void_p, C.c_int, PF, PF]),
        "om_forward_token": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, PF]),
        "om_forward_seq": (C.c_int, [C.c_void_p, C.c_void_p, PU32, S, PF]),
        "om_quantize_i8": (None, [PF, S, S, PI8, PF]),
        "om_quantize_row_i8": (F, [PF, S, PI8]),
        "om_dot_i8": (C.c_int32, [PI8, PI8, S]),
        "om_matmul_w_i8": (None, [PF, PI8, PF, S, S, PF]),
        "om_matmul_batch_w_i8": (None, [PF, PI8, PF, S, S, S, PF]),
        "om_matmul_w_f32": (None, [PF, PF, S, S, PF]),
        "om_matmul_batch_w_f32": (None, [PF, PF, S, S, S, PF]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load_lib()


def fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_float))


def u16p(a: np.ndarray):
    assert a.dtype == np.uint16 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_uint16))


def u32p(a: np.ndarray):
    assert a.dtype == np.uint32 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


def i8p(a: np.ndarray):
    assert a.dtype == np.int8 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_int8))


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------
# kernel-level wrappers (src/tensor.rs)
# ----------------------------------------------------------------------------

def dot_bf16(a, b) -> float:
    a, b = f32(a), np.ascontiguousarray(b, dtype=np.uint16)
    return float(lib.om_dot_bf16(fp(a), u16p(b), a.size))


def dot(a, b) -> float:
    a, b = f32(a), f32(b)
    return float(lib.om_dot(fp(a), fp(b), a.size))


def matmul_w(x, w_bf16: np.ndarray, out: int, inp: int) -> np.ndarray:
    x, w = f32(x), np.ascontiguousarray(w_bf16, dtype=np.uint16)
    y = np.empty(out, np.float32)
    lib.om_matmul_w(fp(x), u16p(w), out, inp, fp(y))
    return y


def matmul_batch_w(x, w_bf16: np.ndarray, out: int, inp: int, T: int) -> np.ndarray:
    x, w = f32(x), np.ascontiguousarray(w_bf16, dtype=np.uint16)
    y = np.empty(T * out, np.float32)
    lib.om_matmul_batch_w(fp(x), u16p(w), out, inp, T, fp(y))
    return y


def matmul_w_f32(x, w: np.ndarray, out: int, inp: int) -> np.ndarray:
    """matmul_w_into for WMat::F32 (src/tensor.rs:387-420): dot per row."""
    x, w = f32(x), f32(w)
    y = np.empty(out, np.float32)
    lib.om_matmul_w_f32(fp(x), fp(w), out, inp, fp(y))
    return y


def matmul_batch_w_f32(x, w: np.ndarray, out: int, inp: int, T: int) -> np.ndarray:
    """matmul_batch_w_into for WMat::F32 (src/tensor.rs:573-760): dot per
    element, as gemm_tile_avx2 computes it."""
    x, w = f32(x), f32(w)
    y = np.empty(T * out, np.float32)
    lib.om_matmul_batch_w_f32(fp(x), fp(w), out, inp, T, fp(y))
    return y


# int8 weight-only mode (TMG_I8=1; src/tensor.rs:125-170, 275-293, 341-386)

def quantize_i8(w, out: int, inp: int):
    """WMat::quantize_i8 of an f32 [out, in] matrix -> (int8 rows, f32 scales)."""
    w = f32(w)
    assert w.size == out * inp
    q = np.empty(out * inp, np.int8)
    s = np.empty(out, np.float32)
    lib.om_quantize_i8(fp(w), out, inp, i8p(q), fp(s))
    return q, s


def quantize_i8_bf16(w_bf16: np.ndarray, out: int, inp: int):
    """wmat_maybe_i8 of a BF16 tensor (src/model.rs:60-68): widen, then quantize."""
    return quantize_i8(bf16_to_f32(np.ascontiguousarray(w_bf16, dtype=np.uint16)), out, inp)


def quantize_row_i8(x):
    """quantize_row_i8 -> (int8 vector, scale)."""
    x = f32(x)
    q = np.empty(x.size, np.int8)
    s = float(lib.om_quantize_row_i8(fp(x), x.size, i8p(q)))
    return q, s


def dot_i8(a, b) -> int:
    a, b = np.ascontiguousarray(a, dtype=np.int8), np.ascontiguousarray(b, dtype=np.int8)
    assert a.size == b.size
    return int(lib.om_dot_i8(i8p(a), i8p(b), a.size))


def matmul_w_i8(x, q: np.ndarray, s: np.ndarray, out: int, inp: int) -> np.ndarray:
    x, q, s = f32(x), np.ascontiguousarray(q, dtype=np.int8), f32(s)
    y = np.empty(out, np.float32)
    lib.om_matmul_w_i8(fp(x), i8p(q), fp(s), out, inp, fp(y))
    return y


def matmul_batch_w_i8(x, q: np.ndarray, s: np.ndarray, out: int, inp: int, T: int) -> np.ndarray:
    x, q, s = f32(x), np.ascontiguousarray(q, dtype=np.int8), f32(s)
    y = np.empty(T * out, np.float32)
    lib.om_matmul_batch_w_i8(fp(x), i8p(q), fp(s), out, inp, T, fp(y))
    return y


def rms_norm(x, w, eps: float) -> np.ndarray:
    x, w = f32(x), f32(w)
    y = np.empty_like(x)
    lib.om_rms_norm(fp(x), fp(w), eps, x.size, fp(y))
    return y


def rms_norm_batch(x, w, eps: float, n: int) -> np.ndarray:
    x, w = f32(x).copy(), f32(w)
    lib.om_rms_norm_batch(fp(x), fp(w), eps, n, x.size // n)
    return x


def rope_rotate(v, pos: int, theta: float) -> np.ndarray:
    v = f32(v).copy()
    lib.om_rope_rotate(fp(v), v.size, pos, theta)
    return v


def rope_table(head_dim: int, theta: float, npos: int):
    c = np.empty(npos * (head_dim // 2), np.float32)
    s = np.empty_like(c)
    lib.om_rope_table(head_dim, theta, npos, fp(c), fp(s))
    return c.reshape(npos, head_dim // 2), s.reshape(npos, head_dim // 2)


def softmax(x) -> np.ndarray:
    x = f32(x)
    y = np.empty_like(x)
    lib.om_softmax(fp(x), x.size, fp(y))
    return y


def silu(x) -> np.ndarray:
    x = f32(x)
    y = np.empty_like(x)
    lib.om_silu(fp(x), x.size, fp(y))
    return y


def argmax(x) -> int:
    x = f32(x)
    return int(lib.om_argmax(fp(x), x.size))


def attention_row(q, keys, values, mask_len: int, scale: float) -> np.ndarray:
    q, k, v = f32(q), f32(keys), f32(values)
    out = np.empty(q.size, np.float32)
    lib.om_attention_row(fp(q), fp(k), fp(v), k.size // q.size, q.size, mask_len, scale, fp(out))
    return out


def attention_batch(q, keys, values, n_heads: int, n_kv: int, head_dim: int, start_pos: int) -> np.ndarray:
    q, k, v = f32(q), f32(keys), f32(values)
    T = q.size // (n_heads * head_dim)
    out = np.empty(q.size, np.float32)
    lib.om_attention_batch(fp(q), fp(k), fp(v), T, n_heads, n_kv, head_dim, start_pos, fp(out))
    return out


def apply_repetition_penalty(logits, generated: Sequence[int], penalty: float) -> np.ndarray:
    l = f32(logits).copy()
    g = np.ascontiguousarray(np.asarray(generated, dtype=np.uint32))
    lib.om_apply_repetition_penalty(fp(l), l.size, u32p(g) if g.size else None, g.size, penalty)
    return l


@dataclass
class SampleTrace:
    token: int
    cand_ids: np.ndarray  # candidate ids in walk order
    cand_probs: np.ndarray  # final probabilities (after the nucleus cut)


def chacha_block(key, counter: int, stream: int, rounds: int) -> np.ndarray:
    k = np.ascontiguousarray(key, np.uint32)
    out = np.empty(16, np.uint32)
    lib.om_chacha_block(u32p(k), counter, stream, rounds, u32p(out))
    return out


def pcg_xsh_rr(state: int) -> int:
    return int(lib.om_pcg_xsh_rr(state))


def uniform_f32(word: int) -> float:
    """StandardUniform f32 of one next_u32 word (exact in f32)."""
    return float(lib.om_uniform_f32(word))


def stdrng_key(seed: int) -> np.ndarray:
    out = np.empty(8, np.uint32)
    lib.om_stdrng_key(seed, u32p(out))
    return out


def stdrng_uniform(seed: int, n: int) -> np.ndarray:
    """The first n `StandardUniform` f32 draws of `StdRng::seed_from_u64(seed)`
    (src/model.rs:629, src/tensor.rs:1204), restated."""
    out = np.empty(max(n, 1), np.float32)
    lib.om_stdrng_uniform(seed, n, fp(out))
    return out[:n]


def sample(logits, temperature: float, top_k: int, top_p: float, r: float) -> SampleTrace:
    """sample (src/tensor.rs:1157-1213) with the uniform draw r given."""
    l = f32(logits)
    ids = np.empty(l.size, np.uint32)
    probs = np.empty(l.size, np.float32)
    n = C.c_size_t()
    tok = lib.om_sample(fp(l), l.size, temperature, top_k, top_p, r, u32p(ids), fp(probs), C.byref(n))
    return SampleTrace(int(tok), ids[:n.value].copy(), probs[:n.value].copy())


def set_num_threads(n: int) -> None:
    lib.om_set_num_threads(n)


def set_attn_threads(n: int) -> None:
    lib.om_set_attn_threads(n)


# ----------------------------------------------------------------------------
# config.json and safetensors (src/config.rs, src/safetensors_loader.rs)
# ----------------------------------------------------------------------------

class OracleError(RuntimeError):
    pass


@dataclass
class Config:
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    intermediate_size: int
    rms_norm_eps: float
    rope_theta: float
    vocab_size: int
    eos_token_ids: List[int] = field(default_factory=list)
    bos_token_id: int = 0


def _as_u64(v) -> Optional[int]:
    # serde_json's as_u64: integer literals >= 0 only (bools are not numbers)
    if isinstance(v, bool) or not isinstance(v, int) or v < 0:
        return None
    return v


def _as_f64(v) -> Optional[float]:
    if isinstance(v, bool) or not isinstance(v, (int, float)):
        return None
    return float(v)


def _f32(x: float) -> float:
    return float(np.float32(x))


def load_config(path: str) -> Config:
    """ModelConfig::load (src/config.rs:112-172)."""
    try:
        with open(path, "rb") as f:
            cfg = json.loads(f.read().decode())
    except OSError as e:
        raise OracleError(f"reading config {path}: {e}")
    return config_from_json(cfg)


def config_from_json(cfg) -> Config:
    """The field rules of ModelConfig::load, which ModelConfig::from_json
    (src/config.rs:37-91) repeats for a TMB file's embedded config."""
    if not isinstance(cfg, dict):
        cfg = {}

    def need(key):
        v = _as_u64(cfg.get(key))
        if v is None:
            raise OracleError(f"config missing integer field `{key}`")
        return v

    hidden = need("hidden_size")
    nq = need("num_attention_heads")
    nkv = _as_u64(cfg.get("num_key_value_heads"))
    nkv = nq if nkv is None else nkv
    hd = _as_u64(cfg.get("head_dim"))
    hd = hidden // nq if hd is None else hd
    theta = _as_f64(cfg.get("rope_theta"))
    if theta is None and isinstance(cfg.get("rope_parameters"), dict):
        theta = _as_f64(cfg["rope_parameters"].get("rope_theta"))
    theta = _f32(10000.0 if theta is None else theta)
    eos = cfg.get("eos_token_id")
    if isinstance(eos, (int, float)) and not isinstance(eos, bool):
        u = _as_u64(eos)
        if u is None:
            raise OracleError("bad eos_token_id")
        eos_ids = [u]
    elif isinstance(eos, list):
        eos_ids = [u for u in (_as_u64(x) for x in eos) if u is not None]
    else:
        eos_ids = []
    eps = _as_f64(cfg.get("rms_norm_eps"))
    bos = _as_u64(cfg.get("bos_token_id"))
    return Config(hidden_size=hidden, num_hidden_layers=need("num_hidden_layers"), num_attention_heads=nq,
                  num_key_value_heads=nkv, head_dim=hd, intermediate_size=need("intermediate_size"),
                  rms_norm_eps=_f32(1e-5 if eps is None else eps), rope_theta=theta,
                  vocab_size=need("vocab_size"), eos_token_ids=eos_ids, bos_token_id=0 if bos is None else bos)


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    """f16_to_f32 (src/safetensors_loader.rs:149-173), including its subnormal
    exponent (starts at 126)."""
    h = h.astype(np.uint32)
    sign = (h & 0x8000) << 16
    exp = (h >> 10) & 0x1F
    frac = h & 0x3FF
    out = np.empty(h.shape, np.uint32)
    norm = (exp != 0) & (exp != 0x1F)
    out[norm] = sign[norm] | ((exp[norm] + 127 - 15) << 23) | (frac[norm] << 13)
    inf = exp == 0x1F
    out[inf] = sign[inf] | 0x7F800000 | (frac[inf] << 13)
    zero = (exp == 0) & (frac == 0)
    out[zero] = sign[zero]
    for i in np.flatnonzero((exp == 0) & (frac != 0)):
        e, f = 126, int(frac.flat[i])
        while f & 0x400 == 0:
            f <<= 1
            e -= 1
        out.flat[i] = int(sign.flat[i]) | (e << 23) | ((f & 0x3FF) << 13)
    return out.view(np.float32)


@dataclass
class Tensor:
    shape: List[int]
    dtype: str
    data: np.ndarray  # uint16 raw bits for BF16, float32 otherwise


def load_safetensors(path: str) -> Dict[str, Tensor]:
    """load_safetensors (src/safetensors_loader.rs:103-147), zero-copy via a
    read-only numpy memmap for BF16."""
    size = os.path.getsize(path)
    if size < 8:
        raise OracleError(f"safetensors file too small: {path}")
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        if size < 8 + n:
            raise OracleError("safetensors header truncated")
        try:
            hdr = json.loads(f.read(n).decode())
        except ValueError as e:
            raise OracleError(f"invalid safetensors header JSON: {e}")
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    out: Dict[str, Tensor] = {}
    for name, meta in hdr.items():
        if name == "__metadata__":
            continue
        b, e = meta["data_offsets"]
        raw = mm[8 + n + b: 8 + n + e]
        dt = meta["dtype"]
        if dt == "BF16":
            data = raw.view(np.uint16)
        elif dt == "F32":
            data = np.array(raw.view(np.float32))
        elif dt == "F16":
            data = f16_to_f32(raw.view(np.uint16))
        else:
            raise OracleError(f"unsupported dtype {dt} for tensor {name} in {path}")
        out[name] = Tensor(list(meta["shape"]), dt, data)
    return out


# ----------------------------------------------------------------------------
# the model (src/model.rs)
# ----------------------------------------------------------------------------

class _Weights(C.Structure):
    _fields_ = [
        ("hidden", C.c_int), ("layers", C.c_int), ("n_heads", C.c_int), ("n_kv", C.c_int), ("head_dim", C.c_int),
        ("inter", C.c_int), ("vocab", C.c_int), ("eps", C.c_float), ("theta", C.c_float),
        ("wq", C.POINTER(C.c_void_p)), ("wk", C.POINTER(C.c_void_p)), ("wv", C.POINTER(C.c_void_p)),
        ("wo", C.POINTER(C.c_void_p)), ("wg", C.POINTER(C.c_void_p)), ("wu", C.POINTER(C.c_void_p)),
        ("wd", C.POINTER(C.c_void_p)), ("in_norm", C.POINTER(C.c_void_p)), ("post_norm", C.POINTER(C.c_void_p)),
        ("final_norm", C.c_void_p), ("embed", C.c_void_p), ("lm_bf16", C.c_void_p),
        ("q8", C.POINTER(C.c_void_p) * 7), ("s8", C.POINTER(C.c_void_p) * 7),
        ("wf", C.POINTER(C.c_void_p) * 7), ("lm_f32", C.c_void_p),
    ]


def _f32vec(t: Tensor) -> np.ndarray:
    if t.dtype == "BF16":
        return bf16_to_f32(np.asarray(t.data))
    return np.ascontiguousarray(t.data, dtype=np.float32)


class OracleCache:
    """KvCache (src/model.rs:250-332)."""

    def __init__(self, layers: int, kv_dim: int):
        self.layers, self.kv_dim = layers, kv_dim
        self._h = lib.om_cache_new(layers, kv_dim)

    def __del__(self):
        if getattr(self, "_h", None):
            lib.om_cache_free(self._h)
            self._h = None

    def len(self, layer: int) -> int:
        return int(lib.om_cache_len(self._h, layer))

    def total_len(self) -> int:
        return self.len(0)

    def reset(self) -> None:
        lib.om_cache_reset(self._h)

    def push(self, layer: int, k, v) -> None:
        k, v = f32(k), f32(v)
        if k.size != self.kv_dim:
            raise OracleError("kv row width mismatch")
        lib.om_cache_push(self._h, layer, fp(k), fp(v))

    def push_rows(self, layer: int, keys_flat, values_flat) -> None:
        """push() of every row of flat [n, kv_dim] key/value arrays."""
        k, v = f32(keys_flat), f32(values_flat)
        if k.size != v.size or k.size % self.kv_dim:
            raise OracleError("kv row width mismatch")
        stride = self.kv_dim * 4
        kb, vb = k.ctypes.data, v.ctypes.data
        for i in range(k.size // self.kv_dim):
            lib.om_cache_push(self._h, layer, C.cast(kb + i * stride, C.POINTER(C.c_float)),
                              C.cast(vb + i * stride, C.POINTER(C.c_float)))

    def keys_flat(self, layer: int) -> np.ndarray:
        n = self.len(layer) * self.kv_dim
        return np.ctypeslib.as_array(lib.om_cache_keys(self._h, layer), (n,)).copy() if n else np.empty(0, np.float32)

    def values_flat(self, layer: int) -> np.ndarray:
        n = self.len(layer) * self.kv_dim
        return np.ctypeslib.as_array(lib.om_cache_values(self._h, layer), (n,)).copy() if n else np.empty(0, np.float32)


class OracleModel:
    """Model (src/model.rs:338-591) over the C restatement."""

    def __init__(self, config: Config, tensors: Dict[str, Tensor], i8: bool = False):
        """i8: the TMG_I8=1 load (src/model.rs:57-76): q, k, v, o, gate, up and
        down quantized per row to int8; lm_head, norms and embedding unchanged."""
        self.config = c = config
        self.i8 = i8
        H, I, V = c.hidden_size, c.intermediate_size, c.vocab_size
        qd, kvd = c.num_attention_heads * c.head_dim, c.num_key_value_heads * c.head_dim

        def need(name, numel):
            t = tensors.get(name)
            if t is None:
                raise OracleError(f"missing tensor `{name}` in safetensors file")
            if int(np.prod(t.shape)) != numel:
                raise OracleError(f"tensor `{name}` has the wrong size")
            return t

        self._keep = []  # arrays the C side points into
        embed = _f32vec(need("model.embed_tokens.weight", V * H))
        if embed.size != V * H:
            raise OracleError(f"embed size {embed.size} != vocab*hidden {V * H}")
        self._keep.append(embed)
        L = c.num_hidden_layers
        arrs = {k: (C.c_void_p * L)() for k in ("wq", "wk", "wv", "wo", "wg", "wu", "wd", "in_norm", "post_norm")}
        wkeys = ("wq", "wk", "wv", "wo", "wg", "wu", "wd")
        q8 = {k: (C.c_void_p * L)() for k in wkeys}
        s8 = {k: (C.c_void_p * L)() for k in wkeys}
        # WMat::F32 (src/model.rs:49-55): an F32 or F16 matrix is converted to
        # f32 at load; its layer entry goes here instead of the BF16 table
        wf = {k: (C.c_void_p * L)() for k in wkeys}
        any_f32 = False
        shapes = {"wq": (qd, H), "wk": (kvd, H), "wv": (kvd, H), "wo": (H, qd), "wg": (I, H), "wu": (I, H),
                  "wd": (H, I)}
        for l in range(L):
            p = f"model.layers.{l}."
            spec = [("wq", "self_attn.q_proj.weight", qd * H), ("wk", "self_attn.k_proj.weight", kvd * H),
                    ("wv", "self_attn.v_proj.weight", kvd * H), ("wo", "self_attn.o_proj.weight", H * qd),
                    ("wg", "mlp.gate_proj.weight", I * H), ("wu", "mlp.up_proj.weight", I * H),
                    ("wd", "mlp.down_proj.weight", H * I)]
            for key, name, numel in spec:
                t = need(p + name, numel)
                if t.dtype == "BF16":
                    a = np.ascontiguousarray(t.data)
                    self._keep.append(a)
                    arrs[key][l] = a.ctypes.data
                    qa_src = bf16_to_f32(a) if i8 else None
                else:
                    a = np.ascontiguousarray(t.data, dtype=np.float32)
                    self._keep.append(a)
                    wf[key][l] = a.ctypes.data
                    any_f32 = True
                    qa_src = a if i8 else None
                if i8:
                    # wmat_maybe_i8 (src/model.rs:60-76): quantize the widened
                    # BF16 values or the f32 values
                    qa, sa = quantize_i8(qa_src, *shapes[key])
                    self._keep += [qa, sa]
                    q8[key][l] = qa.ctypes.data
                    s8[key][l] = sa.ctypes.data
            for key, name in (("in_norm", "input_layernorm.weight"), ("post_norm", "post_attention_layernorm.weight")):
                a = _f32vec(need(p + name, H))
                self._keep.append(a)
                arrs[key][l] = a.ctypes.data
        fnorm = _f32vec(need("model.norm.weight", H))
        self._keep.append(fnorm)
        lm = tensors.get("lm_head.weight")
        lm_arr = lm_f = None
        if lm is not None:
            t = need("lm_head.weight", V * H)
            if t.dtype == "BF16":
                lm_arr = np.ascontiguousarray(t.data)
                self._keep.append(lm_arr)
            else:
                lm_f = np.ascontiguousarray(t.data, dtype=np.float32)
                self._keep.append(lm_f)
        self.tied = lm is None
        w = _Weights(H, L, c.num_attention_heads, c.num_key_value_heads, c.head_dim, I, V, c.rms_norm_eps,
                     c.rope_theta, arrs["wq"], arrs["wk"], arrs["wv"], arrs["wo"], arrs["wg"], arrs["wu"],
                     arrs["wd"], arrs["in_norm"], arrs["post_norm"], fnorm.ctypes.data, embed.ctypes.data,
                     None if lm_arr is None else lm_arr.ctypes.data)
        if lm_f is not None:
            w.lm_f32 = lm_f.ctypes.data
        if any_f32 and not i8:
            for f, key in enumerate(wkeys):
                w.wf[f] = C.cast(wf[key], C.POINTER(C.c_void_p))
            self._keep.append(wf)
        if i8:
            for f, key in enumerate(wkeys):
                w.q8[f] = C.cast(q8[key], C.POINTER(C.c_void_p))
                w.s8[f] = C.cast(s8[key], C.POINTER(C.c_void_p))
            self._keep += [q8, s8]
        self._h = lib.om_model_new(C.byref(w))

    def __del__(self):
        if getattr(self, "_h", None):
            lib.om_model_free(self._h)
            self._h = None

    @classmethod
    def load(cls, model_path: str, i8: bool = False) -> "OracleModel":
        """Model::load -> load_model (src/model.rs:90-96): a TMB1 file goes to
        load_model_tmb (oracle/tmb.py; no int8 path there), anything else to
        load_model_safetensors (src/model.rs:181-244)."""
        with open(model_path, "rb") as f:
            head = f.read(4)
        if head == b"TMB1":
            from oracle import tmb
            config, tensors = tmb.load_model_tmb(model_path)
            return cls(config, tensors)
        cpath = os.path.join(os.path.dirname(os.path.abspath(model_path)), "config.json")
        if not os.path.exists(cpath):
            raise OracleError(f"config.json not found next to {model_path}")
        return cls(load_config(cpath), load_safetensors(model_path), i8=i8)

    def new_cache(self) -> OracleCache:
        c = self.config
        return OracleCache(c.num_hidden_layers, c.num_key_value_heads * c.head_dim)

    def forward_token(self, token: int, cache: OracleCache) -> np.ndarray:
        out = np.empty(self.config.vocab_size, np.float32)
        rc = lib.om_forward_token(self._h, cache._h, int(token), fp(out))
        if rc:
            raise OracleError(f"forward_token failed ({rc})")
        return out

    def forward_seq(self, tokens: Sequence[int], cache: OracleCache) -> np.ndarray:
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        out = np.empty(self.config.vocab_size, np.float32)
        rc = lib.om_forward_seq(self._h, cache._h, u32p(t) if t.size else None, t.size, fp(out))
        if rc == -2:
            raise OracleError("empty prompt")
        if rc:
            raise OracleError(f"forward_seq failed ({rc})")
        return out

    prefill = forward_seq


@dataclass
class OracleGen:
    tokens: List[int]
    logits_first_step: np.ndarray
    step_logits: List[np.ndarray]  # logits each token was chosen from (after the penalty)


def generate(model: OracleModel, prompt: Sequence[int], max_tokens: int, temperature: float = 0.0,
             top_k: int = 0, top_p: float = 1.0, repetition_penalty: float = 1.0,
             draws: Optional[Callable[[int], float]] = None, forced: Optional[Sequence[int]] = None,
             keep_logits: bool = False, seed: int = 0) -> OracleGen:
    """generate (src/model.rs:614-663).  When sampling, step i's uniform is
    `draws(i)` if given, else draw i of StdRng::seed_from_u64(seed)
    (stdrng_uniform); `forced` replays given ids (teacher forcing) while
    still recording the logits each one was chosen from."""
    if len(prompt) == 0:
        raise OracleError("empty prompt")
    cache = model.new_cache()
    logits = model.prefill(prompt, cache)
    first = logits.copy()
    generated: List[int] = []
    step_logits: List[np.ndarray] = []
    eos = set(model.config.eos_token_ids)
    for i in range(max_tokens):
        if repetition_penalty != 1.0 and generated:
            logits = apply_repetition_penalty(logits, generated, repetition_penalty)
        if keep_logits:
            step_logits.append(logits.copy())
        if forced is not None:
            nxt = int(forced[i])
        elif temperature <= 0.0:
            nxt = argmax(logits)
        else:
            if draws is None:
                stream = stdrng_uniform(seed, max_tokens)
                draws = lambda j: float(stream[j])  # noqa: E731
            nxt = sample(logits, temperature, top_k, top_p, draws(i)).token
        generated.append(nxt)
        if nxt in eos:
            break
        logits = model.forward_token(nxt, cache)
    return OracleGen(generated, first, step_logits)
