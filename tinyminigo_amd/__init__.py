"""tinyminigo_amd -- the TinyMiniGo decode path on AMD MI355X (gfx950).

The product is libtmg.so (include/tmg.h): BF16 weights resident in HBM,
hand-written HIP kernels for the decode step (fused GEMV, split-K GQA
attention, on-device argmax/sampling) captured as a hipGraph, and an MFMA
prefill.  This package binds it with ctypes behind the reference's model API.
"""
from ._lib import TmgError, lib
from .model import (
    GenOutput, GenParams, KvCache, Model, ModelConfig, argmax_f32, gemv_bf16, gemv_f32, gemv_i8, generate,
    generate_batch, profile_stream, quantize_i8, repack_tmb, stdrng_uniform, synth_model, synth_normal_bf16,
    synth_normal_f32, synth_tokens,
)

__all__ = [
    "TmgError", "lib", "argmax_f32", "GenOutput", "GenParams", "KvCache", "Model", "ModelConfig", "gemv_bf16", "gemv_f32", "gemv_i8",
    "generate", "generate_batch", "profile_stream", "quantize_i8", "repack_tmb", "stdrng_uniform", "synth_model", "synth_normal_bf16", "synth_normal_f32", "synth_tokens",
]
