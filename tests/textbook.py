"""A float64 textbook Llama decoder in numpy, independent of the reference.

Used only to pin the oracle: RMSNorm, rotate_half RoPE, causal GQA scaled
dot-product attention and a SwiGLU MLP, written from the standard model
definition (HF LlamaForCausalLM) rather than from the reference's code.
Every weight is the same BF16 value the oracle reads, widened to float64.
"""
from __future__ import annotations

import numpy as np


def bf16(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def quantize_rows(w: np.ndarray, zero_scale: float, reciprocal: bool) -> np.ndarray:
    """Symmetric per-row int8 quantization, dequantized (float64 result).
    The mode is defined in f32 arithmetic, which decides exact halves such as
    max/2, so scale and quotient are rounded to f32 as numpy's float32 ops do:
    scale = f32(max|row| / 127); code = the nearest integer to row / scale
    (or, with `reciprocal`, to row * f32(1 / scale)), halves away from zero,
    limited to +-127.  A zero row gets scale `zero_scale` and zero codes."""
    w32 = np.asarray(w, np.float64).astype(np.float32)
    m = np.abs(w32).max(axis=-1, keepdims=True)
    zero = m == 0
    s = np.where(zero, np.float32(1.0), m / np.float32(127.0)).astype(np.float32)
    if reciprocal:
        r = w32 * (np.float32(1.0) / s)
    else:
        r = w32 / s
    q = np.clip(np.sign(r) * np.floor(np.abs(r).astype(np.float64) + 0.5), -127, 127)
    s64 = np.where(zero, zero_scale, s.astype(np.float64))
    return q * s64


class TextbookLlama:
    """i8: the seven projection matrices are replaced by their per-row int8
    quantization (the TMG_I8 weight-only mode); lm_head, norms and embedding
    are kept."""

    def __init__(self, cfg, tensors, i8: bool = False):
        self.c = cfg
        H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocab_size
        self.nq, self.nkv, self.hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim

        def w(name, shape):
            t = tensors[name]
            a = bf16(t.data) if t.dtype == "BF16" else np.asarray(t.data, np.float64)
            return a.reshape(shape)

        qd, kvd = self.nq * self.hd, self.nkv * self.hd
        self.embed = w("model.embed_tokens.weight", (V, H))
        self.layers = []
        for l in range(cfg.num_hidden_layers):
            p = f"model.layers.{l}."
            self.layers.append(dict(
                q=w(p + "self_attn.q_proj.weight", (qd, H)), k=w(p + "self_attn.k_proj.weight", (kvd, H)),
                v=w(p + "self_attn.v_proj.weight", (kvd, H)), o=w(p + "self_attn.o_proj.weight", (H, qd)),
                g=w(p + "mlp.gate_proj.weight", (I, H)), u=w(p + "mlp.up_proj.weight", (I, H)),
                d=w(p + "mlp.down_proj.weight", (H, I)), n1=w(p + "input_layernorm.weight", (H,)),
                n2=w(p + "post_attention_layernorm.weight", (H,))))
        if i8:
            for L in self.layers:
                for key in ("q", "k", "v", "o", "g", "u", "d"):
                    L[key] = quantize_rows(L[key], 1.0, reciprocal=False)
        self.norm = w("model.norm.weight", (H,))
        self.lm = w("lm_head.weight", (V, H)) if "lm_head.weight" in tensors else self.embed
        inv = 1.0 / (float(cfg.rope_theta) ** (np.arange(0, self.hd, 2, dtype=np.float64) / self.hd))
        self.inv_freq = inv

    def rmsnorm(self, x, w):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + float(self.c.rms_norm_eps)) * w

    def rope(self, x, pos):
        # x [T, heads, hd]; rotate_half pairs (i, i + hd/2)
        ang = np.outer(pos, self.inv_freq)  # [T, hd/2]
        cos = np.concatenate([np.cos(ang)] * 2, axis=-1)[:, None, :]
        sin = np.concatenate([np.sin(ang)] * 2, axis=-1)[:, None, :]
        half = self.hd // 2
        rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
        return x * cos + rot * sin

    def logits_all(self, tokens, act_quant: bool = False):
        """Logits of every position for a full causal forward over `tokens`.
        act_quant: each token's input to the seven projections is quantized
        to int8 with one symmetric scale per token first (a zero row stays
        zero), as the int8 decode step does."""
        T = len(tokens)

        def lin(h, w):
            if act_quant:
                h = quantize_rows(h, 0.0, reciprocal=True)
            return h @ w.T
        pos = np.arange(T, dtype=np.float64)
        x = self.embed[np.asarray(tokens)]
        group = self.nq // self.nkv
        mask = np.triu(np.full((T, T), -np.inf), k=1)
        for L in self.layers:
            h = self.rmsnorm(x, L["n1"])
            q = lin(h, L["q"]).reshape(T, self.nq, self.hd)
            k = lin(h, L["k"]).reshape(T, self.nkv, self.hd)
            v = lin(h, L["v"]).reshape(T, self.nkv, self.hd)
            q, k = self.rope(q, pos), self.rope(k, pos)
            out = np.empty((T, self.nq, self.hd))
            for hh in range(self.nq):
                kv = hh // group
                s = q[:, hh, :] @ k[:, kv, :].T / np.sqrt(self.hd) + mask
                s = np.exp(s - s.max(axis=-1, keepdims=True))
                s /= s.sum(axis=-1, keepdims=True)
                out[:, hh, :] = s @ v[:, kv, :]
            x = x + lin(out.reshape(T, -1), L["o"])
            h = self.rmsnorm(x, L["n2"])
            g, u = lin(h, L["g"]), lin(h, L["u"])
            x = x + lin(g / (1.0 + np.exp(-g)) * u, L["d"])
        return self.rmsnorm(x, self.norm) @ self.lm.T
