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


class TextbookLlama:
    def __init__(self, cfg, tensors):
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

    def logits_all(self, tokens):
        """Logits of every position for a full causal forward over `tokens`."""
        T = len(tokens)
        pos = np.arange(T, dtype=np.float64)
        x = self.embed[np.asarray(tokens)]
        group = self.nq // self.nkv
        mask = np.triu(np.full((T, T), -np.inf), k=1)
        for L in self.layers:
            h = self.rmsnorm(x, L["n1"])
            q = (h @ L["q"].T).reshape(T, self.nq, self.hd)
            k = (h @ L["k"].T).reshape(T, self.nkv, self.hd)
            v = (h @ L["v"].T).reshape(T, self.nkv, self.hd)
            q, k = self.rope(q, pos), self.rope(k, pos)
            out = np.empty((T, self.nq, self.hd))
            for hh in range(self.nq):
                kv = hh // group
                s = q[:, hh, :] @ k[:, kv, :].T / np.sqrt(self.hd) + mask
                s = np.exp(s - s.max(axis=-1, keepdims=True))
                s /= s.sum(axis=-1, keepdims=True)
                out[:, hh, :] = s @ v[:, kv, :]
            x = x + out.reshape(T, -1) @ L["o"].T
            h = self.rmsnorm(x, L["n2"])
            g, u = h @ L["g"].T, h @ L["u"].T
            x = x + (g / (1.0 + np.exp(-g)) * u) @ L["d"].T
        return self.rmsnorm(x, self.norm) @ self.lm.T
