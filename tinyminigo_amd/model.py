"""Python mirror of the reference crate's model API over libtmg's C ABI.

Names and argument meanings follow the reference (src/model.rs, src/config.rs):
``Model.load``, ``Model.forward_token``, ``Model.prefill``,
``Model.forward_seq``, ``KvCache`` and ``generate`` with ``GenParams`` /
``GenOutput``.  Errors raise ``TmgError`` carrying the library's context text
(the reference returns anyhow errors with the same kind of context).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence

import numpy as np

import weakref

from ._lib import (
    ON_TOKEN, TmgError, check, finalizing, lib, register, tmg_config, tmg_floor_record, tmg_gen_params,
    tmg_kernel_record, tmg_synth_spec,
)

__all__ = [
    "ModelConfig", "Model", "KvCache", "GenParams", "GenOutput", "generate", "gemv_bf16", "gemv_i8", "quantize_i8", "repack_tmb",
    "argmax_f32", "profile_stream",
    "generate_batch",
    "synth_model", "synth_tokens", "synth_normal_bf16", "synth_normal_f32", "TmgError",
]


def _u32(a: Sequence[int]) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint32))


def _fptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(C.POINTER(C.c_float))


@dataclass
class ModelConfig:
    """ModelConfig (src/config.rs:6-20)."""

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
    tied_lm_head: bool = False

    @classmethod
    def _from_c(cls, c: tmg_config) -> "ModelConfig":
        return cls(
            hidden_size=c.hidden_size, num_hidden_layers=c.num_hidden_layers,
            num_attention_heads=c.num_attention_heads, num_key_value_heads=c.num_key_value_heads,
            head_dim=c.head_dim, intermediate_size=c.intermediate_size, rms_norm_eps=c.rms_norm_eps,
            rope_theta=c.rope_theta, vocab_size=c.vocab_size,
            eos_token_ids=[c.eos_token_ids[i] for i in range(c.n_eos)], bos_token_id=c.bos_token_id,
            tied_lm_head=bool(c.tied_lm_head),
        )

    @classmethod
    def load(cls, path: str) -> "ModelConfig":
        """ModelConfig::load (src/config.rs:112-172)."""
        c = tmg_config()
        check(lib.tmg_config_load(path.encode(), C.byref(c)))
        return cls._from_c(c)

    @classmethod
    def from_tmb(cls, path: str) -> "ModelConfig":
        """The config embedded in a TMB1 file (src/tmb.rs:81-120)."""
        c = tmg_config()
        check(lib.tmg_tmb_config(path.encode(), C.byref(c)))
        return cls._from_c(c)


class Model:
    """Model (src/model.rs:338-591): weights resident in HBM on one GPU."""

    def __init__(self, handle: C.c_void_p):
        self._h = handle
        self._caches = weakref.WeakSet()
        register(self, 3)
        c = tmg_config()
        check(lib.tmg_model_config(self._h, C.byref(c)))
        self.config = ModelConfig._from_c(c)

    @classmethod
    def load(cls, path: str, device: int = 0) -> "Model":
        """Model::load (src/model.rs:384-389)."""
        h = C.c_void_p()
        check(lib.tmg_model_load(str(path).encode(), device, C.byref(h)))
        return cls(h)

    def close(self) -> None:
        """Free the model and every cache made on it (tmg_model_free)."""
        for cache in list(self._caches):
            cache.close()
        if self._h:
            lib.tmg_model_free(self._h)
            self._h = None

    def __del__(self):
        if finalizing():
            return
        try:
            self.close()
        except Exception:
            pass

    def new_cache(self, max_pos: int) -> "KvCache":
        return KvCache(self, max_pos)

    def forward_token(self, token: int, cache: "KvCache", want_logits: bool = True) -> Optional[np.ndarray]:
        """Model::forward_token (src/model.rs:392-491)."""
        out = np.empty(self.config.vocab_size, np.float32) if want_logits else None
        check(lib.tmg_forward_token(self._h, cache._h, int(token), _fptr(out)))
        return out

    def forward_seq(self, tokens: Sequence[int], cache: "KvCache", want_logits: bool = True) -> Optional[np.ndarray]:
        """Model::forward_seq (src/model.rs:503-590)."""
        t = _u32(tokens)
        out = np.empty(self.config.vocab_size, np.float32) if want_logits else None
        check(lib.tmg_forward_seq(self._h, cache._h, t.ctypes.data_as(C.POINTER(C.c_uint32)), t.size, _fptr(out)))
        return out

    def prefill(self, tokens: Sequence[int], cache: "KvCache") -> np.ndarray:
        """Model::prefill (src/model.rs:494-499)."""
        t = _u32(tokens)
        out = np.empty(self.config.vocab_size, np.float32)
        check(lib.tmg_prefill(self._h, cache._h, t.ctypes.data_as(C.POINTER(C.c_uint32)), t.size, _fptr(out)))
        return out

    # -- measurement helpers (no reference counterpart) ----------------------

    def decode_greedy(self, token: int, n_steps: int, cache: "KvCache"):
        """n_steps device-resident greedy steps; returns (tokens, elapsed ms)."""
        toks = np.empty(max(n_steps, 1), np.uint32)
        ms = C.c_float()
        check(lib.tmg_decode_greedy(self._h, cache._h, int(token), int(n_steps),
                                    toks.ctypes.data_as(C.POINTER(C.c_uint32)), C.byref(ms)))
        return toks[:n_steps], ms.value

    def profile_decode_step(self, token: int, cache: "KvCache"):
        """Per-kernel timing of one decode step at the cache's position (each
        kernel kind replayed back to back from a graph; the cache is left as it
        was): list of (name, algorithmic bytes per launch, ms per launch,
        launches per step)."""
        recs = (tmg_kernel_record * 64)()
        n = C.c_size_t()
        check(lib.tmg_profile_decode_step(self._h, cache._h, int(token), recs, 64, C.byref(n)))
        return [(recs[i].name.decode(), recs[i].bytes, recs[i].ms, recs[i].launches) for i in range(n.value)]

    def profile_step_floor(self, token: int, cache: "KvCache"):
        """The greedy step at the cache's position next to its floor (every
        launch replaced by a streaming phase of the same grid and bytes; the
        cache is left as it was): dict with step_ms, floor_ms, empty_launch_ms
        and kinds, a list of (name, algorithmic bytes, phase bytes, phase ms,
        launches per step, workgroups)."""
        recs = (tmg_floor_record * 64)()
        n = C.c_size_t()
        step, floor, empty = C.c_float(), C.c_float(), C.c_float()
        check(lib.tmg_profile_step_floor(self._h, cache._h, int(token), recs, 64, C.byref(n), C.byref(step),
                                         C.byref(floor), C.byref(empty)))
        kinds = [(recs[i].name.decode(), recs[i].bytes, recs[i].floor_bytes, recs[i].floor_ms, recs[i].launches,
                  recs[i].workgroups) for i in range(n.value)]
        return {"step_ms": step.value, "floor_ms": floor.value, "empty_launch_ms": empty.value, "kinds": kinds}


class KvCache:
    """KvCache (src/model.rs:250-332) as a preallocated HBM slab of max_pos rows."""

    def __init__(self, model: Model, max_pos: int):
        self.model = model
        self.max_pos = max_pos
        self._h = None
        h = C.c_void_p()
        check(lib.tmg_cache_new(model._h, int(max_pos), C.byref(h)))
        self._h = h
        model._caches.add(self)
        register(self, 1)

    def close(self) -> None:
        if self._h:
            lib.tmg_cache_free(self._h)
            self._h = None

    def __del__(self):
        if finalizing():
            return
        try:
            self.close()
        except Exception:
            pass

    def len(self, layer: int) -> int:
        v = C.c_uint32()
        check(lib.tmg_cache_len(self._h, layer, C.byref(v)))
        return v.value

    def total_len(self) -> int:
        return self.len(0)

    def reset(self) -> None:
        check(lib.tmg_cache_reset(self._h))

    def _read(self, layer: int):
        cfg = self.model.config
        kvd = cfg.num_key_value_heads * cfg.head_dim
        n = self.len(layer)
        k = np.empty(n * kvd, np.float32)
        v = np.empty(n * kvd, np.float32)
        check(lib.tmg_cache_read(self._h, layer, _fptr(k), _fptr(v)))
        return k, v

    def keys_flat(self, layer: int) -> np.ndarray:
        return self._read(layer)[0]

    def values_flat(self, layer: int) -> np.ndarray:
        return self._read(layer)[1]


@dataclass
class GenParams:
    """GenParams (src/model.rs:597-604)."""

    max_tokens: int = 64
    temperature: float = 0.0
    top_k: int = 0
    top_p: float = 1.0
    repetition_penalty: float = 1.0
    seed: int = 42


@dataclass
class GenOutput:
    """GenOutput (src/model.rs:606-611)."""

    tokens: List[int]
    logits_first_step: np.ndarray
    prefill_secs: float


def generate(model: Model, prompt_tokens: Sequence[int], params: GenParams,
             on_token: Optional[Callable[[int], None]] = None) -> GenOutput:
    """generate (src/model.rs:614-663)."""
    t = _u32(prompt_tokens)
    p = tmg_gen_params(params.max_tokens, params.temperature, params.top_k, params.top_p,
                       params.repetition_penalty, params.seed)
    out = np.empty(max(params.max_tokens, 1), np.uint32)
    first = np.empty(model.config.vocab_size, np.float32)
    n_out = C.c_size_t()
    secs = C.c_float()
    err: List[BaseException] = []

    def _cb(tok, _user):
        if on_token is not None and not err:
            try:
                on_token(int(tok))
            except BaseException as e:  # surfaced after the call returns
                err.append(e)

    cb = ON_TOKEN(_cb)
    check(lib.tmg_generate(model._h, t.ctypes.data_as(C.POINTER(C.c_uint32)), t.size, C.byref(p), cb, None,
                           out.ctypes.data_as(C.POINTER(C.c_uint32)), out.size, C.byref(n_out), _fptr(first),
                           C.byref(secs)))
    if err:
        raise err[0]
    return GenOutput(tokens=[int(x) for x in out[:n_out.value]], logits_first_step=first,
                     prefill_secs=secs.value)


def profile_stream(nbytes: int, wg_kib: int, device: int = 0):
    """tmg_profile_stream: (us per launch, bytes read) of a kernel that only
    streams nbytes of HBM-cold data in workgroups of wg_kib KiB."""
    us = C.c_float()
    got = C.c_size_t()
    check(lib.tmg_profile_stream(int(nbytes), int(wg_kib), int(device), C.byref(us), C.byref(got)))
    return us.value, got.value


def stdrng_uniform(seed: int, n: int) -> np.ndarray:
    """The uniform draws `generate` samples with: StdRng::seed_from_u64(seed)
    (src/model.rs:629), one StandardUniform f32 per step (src/tensor.rs:1204)."""
    out = np.empty(max(n, 1), np.float32)
    check(lib.tmg_stdrng_uniform(seed, n, _fptr(out)))
    return out[:n]


def gemv_bf16(w_dev: int, x_dev: int, y_dev: int, out: int, in_: int, stream: int = 0) -> None:
    """tensor::matmul_w (src/tensor.rs:315-338) on device pointers."""
    check(lib.tmg_gemv_bf16(C.c_void_p(w_dev), C.c_void_p(x_dev), C.c_void_p(y_dev), out, in_,
                            C.c_void_p(stream)))


def gemv_f32(w_dev: int, x_dev: int, y_dev: int, out: int, in_: int, stream: int = 0) -> None:
    """tensor::matmul_w over a WMat::F32 matrix (src/tensor.rs:387-420) on
    device pointers."""
    check(lib.tmg_gemv_f32(C.c_void_p(w_dev), C.c_void_p(x_dev), C.c_void_p(y_dev), out, in_,
                           C.c_void_p(stream)))


def argmax_f32(x_dev: int, n: int, out_dev: int, stream: int = 0) -> None:
    """tensor::argmax (src/tensor.rs:1063-1073) of n device floats into a
    device uint32."""
    check(lib.tmg_argmax_f32(C.c_void_p(x_dev), int(n), C.c_void_p(out_dev), C.c_void_p(stream)))


def generate_batch(model: Model, prompts: Sequence[Sequence[int]], max_tokens: int):
    """Greedy generation for several prompts at once (tmg_generate_batch): for
    each prompt the ids generate (src/model.rs:614-663) gives alone at
    temperature 0.  Returns (list of id lists, device ms of the decode steps)."""
    n = len(prompts)
    arrs = [_u32(p) for p in prompts]
    ptrs = (C.POINTER(C.c_uint32) * n)(*[a.ctypes.data_as(C.POINTER(C.c_uint32)) for a in arrs])
    lens = (C.c_size_t * n)(*[a.size for a in arrs])
    out = np.zeros(max(1, n * max_tokens), np.uint32)
    n_out = (C.c_size_t * n)()
    ms = C.c_float(0.0)
    check(lib.tmg_generate_batch(model._h, ptrs, lens, n, max_tokens, out.ctypes.data_as(C.POINTER(C.c_uint32)),
                                 n_out, C.byref(ms)))
    return [[int(x) for x in out[b * max_tokens:b * max_tokens + n_out[b]]] for b in range(n)], ms.value


def repack_tmb(safetensors_path: str, tmb_path: str) -> None:
    """write_tmb (src/tmb.rs:137-262): the reference's `--repack`."""
    check(lib.tmg_tmb_repack(safetensors_path.encode(), tmb_path.encode()))


def gemv_i8(q_dev: int, scale_dev: int, x_dev: int, y_dev: int, out: int, in_: int, stream: int = 0) -> None:
    """matmul_w_into over WMat::I8 (src/tensor.rs:341-364) on device pointers."""
    check(lib.tmg_gemv_i8(C.c_void_p(q_dev), C.c_void_p(scale_dev), C.c_void_p(x_dev), C.c_void_p(y_dev), out,
                          in_, C.c_void_p(stream)))


def quantize_i8(w_dev: int, rows: int, in_: int, q_dev: int, scale_dev: int, stream: int = 0) -> None:
    """WMat::quantize_i8 (src/tensor.rs:275-293) of BF16 rows on device pointers."""
    check(lib.tmg_quantize_i8(C.c_void_p(w_dev), rows, in_, C.c_void_p(q_dev), C.c_void_p(scale_dev),
                              C.c_void_p(stream)))


# -- synthetic inputs ---------------------------------------------------------

def synth_model(directory: str, *, hidden_size: int, num_hidden_layers: int, num_attention_heads: int,
                num_key_value_heads: int, head_dim: int, intermediate_size: int, vocab_size: int,
                rms_norm_eps: float, rope_theta: float, tied_lm_head: bool, seed: int,
                stddev: float = 0.02) -> str:
    """Write <directory>/model.safetensors + config.json; returns the model path."""
    spec = tmg_synth_spec(hidden_size, num_hidden_layers, num_attention_heads, num_key_value_heads, head_dim,
                          intermediate_size, vocab_size, rms_norm_eps, rope_theta, int(tied_lm_head), seed, stddev)
    check(lib.tmg_synth_model(str(directory).encode(), C.byref(spec)))
    return str(directory) + "/model.safetensors"


def synth_tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    out = np.empty(max(n, 1), np.uint32)
    check(lib.tmg_synth_tokens(seed, n, vocab, out.ctypes.data_as(C.POINTER(C.c_uint32))))
    return out[:n]


def synth_normal_bf16(seed: int, name: str, n: int, stddev: float) -> np.ndarray:
    out = np.empty(max(n, 1), np.uint16)
    check(lib.tmg_synth_normal_bf16(seed, name.encode(), n, stddev, out.ctypes.data_as(C.POINTER(C.c_uint16))))
    return out[:n]


def synth_normal_f32(seed: int, name: str, n: int, stddev: float) -> np.ndarray:
    out = np.empty(max(n, 1), np.float32)
    check(lib.tmg_synth_normal_f32(seed, name.encode(), n, stddev, out.ctypes.data_as(C.POINTER(C.c_float))))
    return out[:n]
