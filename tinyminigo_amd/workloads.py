"""The benchmark workloads: synthetic model shapes, seeds and decode lengths.

Shapes follow the reference's MiniCPM5/Llama layout (src/config.rs:6-20).
Weights are N(0, 0.02) BF16 with all-one norm weights, drawn by
tmg_synth_model; prompts are uniform token ids from tmg_synth_tokens.
"""
from __future__ import annotations

import os
from dataclasses import dataclass

from .model import synth_model, synth_tokens


@dataclass(frozen=True)
class Workload:
    name: str
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    intermediate_size: int
    vocab_size: int
    rms_norm_eps: float
    rope_theta: float
    tied_lm_head: bool
    weight_seed: int
    prompt_seed: int
    prompt_len: int
    gen_tokens: int

    def spec(self) -> dict:
        return dict(hidden_size=self.hidden_size, num_hidden_layers=self.num_hidden_layers,
                    num_attention_heads=self.num_attention_heads, num_key_value_heads=self.num_key_value_heads,
                    head_dim=self.head_dim, intermediate_size=self.intermediate_size, vocab_size=self.vocab_size,
                    rms_norm_eps=self.rms_norm_eps, rope_theta=self.rope_theta, tied_lm_head=self.tied_lm_head,
                    seed=self.weight_seed)

    def prompt(self):
        return synth_tokens(self.prompt_seed, self.prompt_len, self.vocab_size)

    # algorithmic bytes streamed per decode token (BF16 weights, f32 norms,
    # one embedding row, f32 KV read at n_ctx and the KV row written); with
    # i8 the layer matrices are int8 codes plus one f32 scale per row and the
    # lm_head stays BF16
    def weight_bytes(self, i8: bool = False) -> int:
        H, I, V = self.hidden_size, self.intermediate_size, self.vocab_size
        qd = self.num_attention_heads * self.head_dim
        kvd = self.num_key_value_heads * self.head_dim
        params = qd * H + 2 * kvd * H + H * qd + 3 * H * I
        rows = qd + 2 * kvd + H + 2 * I + H
        per_layer = params + 4 * rows if i8 else params * 2
        return self.num_hidden_layers * per_layer + V * H * 2

    def kv_bytes(self, n_ctx: int) -> int:
        kvd = self.num_key_value_heads * self.head_dim
        return 2 * self.num_hidden_layers * n_ctx * kvd * 4 + 2 * self.num_hidden_layers * kvd * 4

    def misc_bytes(self) -> int:
        H = self.hidden_size
        return (2 * self.num_hidden_layers + 1) * H * 4 + H * 2

    def decode_bytes(self, n_ctx: int, i8: bool = False) -> int:
        return self.weight_bytes(i8) + self.kv_bytes(n_ctx) + self.misc_bytes()

    def prefill_flops(self, T: int, start: int = 0) -> float:
        H, I, V = self.hidden_size, self.intermediate_size, self.vocab_size
        qd = self.num_attention_heads * self.head_dim
        kvd = self.num_key_value_heads * self.head_dim
        params = qd * H + 2 * kvd * H + H * qd + 3 * H * I
        attn = 4.0 * self.num_hidden_layers * qd * sum(start + t + 1 for t in range(T))
        return 2.0 * T * params * self.num_hidden_layers + 2.0 * V * H + attn


# C0: tiny random Llama, tied lm_head, 16-token prompt + 40 greedy steps
TINY = Workload("tiny-llama-h64-l2", 64, 2, 4, 2, 16, 128, 1024, 1e-6, 10000.0, True, 0, 1, 16, 40)
# C2: 1B-class MiniCPM5-shaped model, 64-token prompt + 256 greedy steps
ONE_B = Workload("minicpm5-1b-synthetic", 2048, 24, 16, 8, 128, 6144, 73448, 1e-5, 10000.0, False, 3, 4, 64, 256)
# C3: the 1B model after an 8192-token prefill, 128 greedy steps
LONG_CTX = Workload("minicpm5-1b-synthetic-8k", 2048, 24, 16, 8, 128, 6144, 73448, 1e-5, 10000.0, False, 3, 5, 8192,
                    128)
# C4: 4B-class, 128-token prompt + 256 sampled tokens
FOUR_B = Workload("minicpm5-4b-synthetic", 2560, 36, 32, 8, 128, 10240, 73448, 1e-5, 10000.0, False, 6, 7, 128, 256)

# C1 GEMV sweep shapes (out x in)
GEMV_SHAPES = [(2048, 2048), (6144, 2048), (2048, 6144), (73448, 2048)]


def ensure_model(w: Workload, root: str) -> str:
    """Synthesize the workload's model under root/<name> once; returns its path."""
    d = os.path.join(root, w.name)
    path = os.path.join(d, "model.safetensors")
    stamp = os.path.join(d, "synth.ok")
    if not (os.path.exists(path) and os.path.exists(stamp)):
        os.makedirs(d, exist_ok=True)
        synth_model(d, **w.spec())
        with open(stamp, "w") as f:
            f.write("ok\n")
    return path
