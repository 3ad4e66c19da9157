"""ctypes binding of libtmg.so (include/tmg.h, include/tmg_synth.h).

The library is loaded from this package directory; there is no fallback:
when libtmg.so is missing, importing this module raises ImportError.
"""
from __future__ import annotations

import atexit
import ctypes as C
import os
import sys
import weakref

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtmg.so")

TMG_OK = 0
TMG_E_INVALID = -1
TMG_E_IO = -2
TMG_E_FORMAT = -3
TMG_E_MISSING = -4
TMG_E_DTYPE = -5
TMG_E_EMPTY = -6
TMG_E_CAPACITY = -7
TMG_E_DEVICE = -8
TMG_E_NOMEM = -9

ERROR_NAMES = {
    TMG_E_INVALID: "TMG_E_INVALID",
    TMG_E_IO: "TMG_E_IO",
    TMG_E_FORMAT: "TMG_E_FORMAT",
    TMG_E_MISSING: "TMG_E_MISSING",
    TMG_E_DTYPE: "TMG_E_DTYPE",
    TMG_E_EMPTY: "TMG_E_EMPTY",
    TMG_E_CAPACITY: "TMG_E_CAPACITY",
    TMG_E_DEVICE: "TMG_E_DEVICE",
    TMG_E_NOMEM: "TMG_E_NOMEM",
}


class tmg_config(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_uint32),
        ("num_hidden_layers", C.c_uint32),
        ("num_attention_heads", C.c_uint32),
        ("num_key_value_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("intermediate_size", C.c_uint32),
        ("vocab_size", C.c_uint32),
        ("bos_token_id", C.c_uint32),
        ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_float),
        ("n_eos", C.c_uint32),
        ("eos_token_ids", C.c_uint32 * 16),
        ("tied_lm_head", C.c_int32),
    ]


class tmg_gen_params(C.Structure):
    _fields_ = [
        ("max_tokens", C.c_uint32),
        ("temperature", C.c_float),
        ("top_k", C.c_uint32),
        ("top_p", C.c_float),
        ("repetition_penalty", C.c_float),
        ("seed", C.c_uint64),
    ]


class tmg_kernel_record(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("bytes", C.c_double), ("ms", C.c_float), ("launches", C.c_uint32)]


class tmg_floor_record(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("bytes", C.c_double), ("floor_bytes", C.c_double), ("floor_ms", C.c_float),
                ("launches", C.c_uint32), ("workgroups", C.c_uint32)]


class tmg_synth_spec(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_uint32),
        ("num_hidden_layers", C.c_uint32),
        ("num_attention_heads", C.c_uint32),
        ("num_key_value_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("intermediate_size", C.c_uint32),
        ("vocab_size", C.c_uint32),
        ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_float),
        ("tied_lm_head", C.c_int32),
        ("seed", C.c_uint64),
        ("stddev", C.c_float),
    ]


ON_TOKEN = C.CFUNCTYPE(None, C.c_uint32, C.c_void_p)

P = C.c_void_p
PF = C.POINTER(C.c_float)
PU32 = C.POINTER(C.c_uint32)
PU16 = C.POINTER(C.c_uint16)

# name -> (restype, argtypes); every symbol include/*.h declares
SIGNATURES = {
    "tmg_last_error": (C.c_char_p, []),
    "tmg_config_load": (C.c_int, [C.c_char_p, C.POINTER(tmg_config)]),
    "tmg_model_load": (C.c_int, [C.c_char_p, C.c_int, C.POINTER(P)]),
    "tmg_model_free": (None, [P]),
    "tmg_model_config": (C.c_int, [P, C.POINTER(tmg_config)]),
    "tmg_cache_new": (C.c_int, [P, C.c_uint32, C.POINTER(P)]),
    "tmg_cache_free": (None, [P]),
    "tmg_cache_len": (C.c_int, [P, C.c_uint32, PU32]),
    "tmg_cache_reset": (C.c_int, [P]),
    "tmg_cache_read": (C.c_int, [P, C.c_uint32, PF, PF]),
    "tmg_forward_token": (C.c_int, [P, P, C.c_uint32, PF]),
    "tmg_forward_seq": (C.c_int, [P, P, PU32, C.c_size_t, PF]),
    "tmg_prefill": (C.c_int, [P, P, PU32, C.c_size_t, PF]),
    "tmg_generate": (
        C.c_int,
        [P, PU32, C.c_size_t, C.POINTER(tmg_gen_params), ON_TOKEN, P, PU32, C.c_size_t,
         C.POINTER(C.c_size_t), PF, PF],
    ),
    "tmg_generate_batch": (C.c_int, [P, C.POINTER(PU32), C.POINTER(C.c_size_t), C.c_size_t, C.c_uint32, PU32,
                                     C.POINTER(C.c_size_t), PF]),
    "tmg_tmb_repack": (C.c_int, [C.c_char_p, C.c_char_p]),
    "tmg_tmb_config": (C.c_int, [C.c_char_p, C.POINTER(tmg_config)]),
    "tmg_gemv_bf16": (C.c_int, [P, P, P, C.c_uint32, C.c_uint32, P]),
    "tmg_gemv_f32": (C.c_int, [P, P, P, C.c_uint32, C.c_uint32, P]),
    "tmg_argmax_f32": (C.c_int, [P, C.c_uint32, P, P]),
    "tmg_argmax_f32_noalloc": (C.c_int, [P, C.c_uint32, P, P]),
    "tmg_stdrng_uniform": (C.c_int, [C.c_uint64, C.c_size_t, PF]),
    "tmg_gemv_i8": (C.c_int, [P, P, P, P, C.c_uint32, C.c_uint32, P]),
    "tmg_quantize_i8": (C.c_int, [P, C.c_uint32, C.c_uint32, P, P, P]),
    "tmg_decode_greedy": (C.c_int, [P, P, C.c_uint32, C.c_uint32, PU32, PF]),
    "tmg_profile_decode_step": (
        C.c_int, [P, P, C.c_uint32, C.POINTER(tmg_kernel_record), C.c_size_t, C.POINTER(C.c_size_t)]),
    "tmg_profile_step_floor": (
        C.c_int, [P, P, C.c_uint32, C.POINTER(tmg_floor_record), C.c_size_t, C.POINTER(C.c_size_t), PF, PF, PF]),
    "tmg_profile_stream": (C.c_int, [C.c_size_t, C.c_uint32, C.c_int, PF, C.POINTER(C.c_size_t)]),
    "tmg_synth_model": (C.c_int, [C.c_char_p, C.POINTER(tmg_synth_spec)]),
    "tmg_synth_tokens": (C.c_int, [C.c_uint64, C.c_size_t, C.c_uint32, PU32]),
    "tmg_synth_normal_bf16": (C.c_int, [C.c_uint64, C.c_char_p, C.c_size_t, C.c_float, PU16]),
    "tmg_synth_normal_f32": (C.c_int, [C.c_uint64, C.c_char_p, C.c_size_t, C.c_float, PF]),
}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built: run __graft_entry__.build() (make -C tinyminigo_amd/csrc)")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


class TmgError(RuntimeError):
    """A non-zero status from libtmg, with the library's context string."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {msg}")
        self.code = code


def check(rc: int) -> None:
    if rc != TMG_OK:
        raise TmgError(rc, lib.tmg_last_error().decode(errors="replace"))


# ---- native handle lifetime --------------------------------------------------
#
# Every Python object that owns a native handle (a model, a KV cache, a device
# buffer, a stream, a graph, timing events) registers here.  At interpreter
# exit they are released explicitly, in dependency order (graphs and events,
# then caches, buffers, models, streams), while the HIP runtime is still whole;
# after that no finalizer makes a HIP or libtmg call.

_RANKS = 5
_live = [weakref.WeakSet() for _ in range(_RANKS)]
_released = False


def register(obj, rank: int) -> None:
    """Track `obj` (which has a close() method) for release at exit."""
    _live[rank].add(obj)


def finalizing() -> bool:
    """True once native handles must no longer be touched from finalizers."""
    return _released or sys.is_finalizing()


def release_all() -> None:
    """Close every live native handle (idempotent); called at exit."""
    global _released
    if _released:
        return
    for rank in range(_RANKS):
        for obj in list(_live[rank]):
            try:
                obj.close()
            except Exception:
                pass
    _released = True


atexit.register(release_all)
