"""Text front-end around the decode path: tokenizer, chat template, streamed
generation.

Mirrors the reference's host-side text handling:
- `Tokenizer` and `resolve_tokenizer_path` (src/tokenizer.rs:1-45) wrap the
  HuggingFace `tokenizers` library, as the reference wraps its Rust crate
  (the Python package binds the same Rust implementation);
- `render_chat_template` (src/template.rs:1-29) renders a HF chat template
  for one user turn with Jinja2, where the reference uses minijinja with its
  Python-compatibility method callback (Jinja2 runs Python's own string
  methods);
- `generate_text` is the generation step of src/main.rs:73-133: render,
  encode without special tokens, `generate` with streaming detokenization of
  each new token, the first-step logits dump and the timing summary line
  (the argument parsing around it, src/cli.rs, is not mirrored).

Everything here is host text processing; the ids go through `generate`
(libtmg) unchanged.
"""
from __future__ import annotations

import json
import os
import time
from dataclasses import dataclass
from typing import Callable, List, Optional, Sequence, TextIO

import numpy as np


class TextError(RuntimeError):
    pass


class Tokenizer:
    """src/tokenizer.rs:4-34."""

    def __init__(self, inner) -> None:
        self._inner = inner

    @classmethod
    def from_file(cls, path: str) -> "Tokenizer":
        import tokenizers
        try:
            return cls(tokenizers.Tokenizer.from_file(str(path)))
        except Exception as e:  # the library raises its own exception type
            raise TextError(f"loading tokenizer from {path}: {e}") from e

    def encode(self, text: str, add_special_tokens: bool) -> List[int]:
        try:
            return list(self._inner.encode(text, add_special_tokens=add_special_tokens).ids)
        except Exception as e:
            raise TextError(f"tokenization failed: {e}") from e

    def decode(self, ids: Sequence[int], skip_special_tokens: bool) -> str:
        try:
            return self._inner.decode([int(i) for i in ids], skip_special_tokens=skip_special_tokens)
        except Exception as e:
            raise TextError(f"detokenization failed: {e}") from e

    def vocab_size(self) -> int:
        return self._inner.get_vocab_size(with_added_tokens=True)


def resolve_tokenizer_path(explicit: Optional[str], model_path: str) -> str:
    """src/tokenizer.rs:36-45: the explicit path, else tokenizer.json next to
    the model file."""
    if explicit is not None:
        return explicit
    parent = os.path.dirname(str(model_path))
    if str(model_path) in ("", "/"):
        raise TextError(f"model path {model_path} has no parent dir")
    return os.path.join(parent, "tokenizer.json")


def render_chat_template(template_path: str, user_prompt: str, bos_token: str) -> str:
    """src/template.rs:6-29: one user message, add_generation_prompt true,
    eos_token and pad_token "</s>"."""
    import jinja2
    try:
        with open(template_path, encoding="utf-8") as f:
            src = f.read()
    except OSError as e:
        raise TextError(f"reading chat template {template_path}: {e}") from e
    env = jinja2.Environment()  # no autoescape, no block trimming: the minijinja defaults
    try:
        tmpl = env.from_string(src)
    except jinja2.TemplateSyntaxError as e:
        raise TextError(f"parsing chat template {template_path}: {e}") from e
    ctx = {
        "messages": [{"role": "user", "content": user_prompt}],
        "add_generation_prompt": True,
        "bos_token": bos_token,
        "eos_token": "</s>",
        "pad_token": "</s>",
    }
    try:
        return tmpl.render(**ctx)
    except jinja2.TemplateError as e:
        raise TextError(f"rendering chat template {template_path}: {e}") from e


def first_logits_dump(logits: np.ndarray) -> dict:
    """The --dump-first-logits record (src/main.rs:100-114): the five largest
    logits (ties by lower id) and the first eight values."""
    lg = np.asarray(logits, np.float32)
    top = sorted(range(lg.size), key=lambda i: (-float(lg[i]), i))[:5]
    return {"top5_ids": top, "top5_vals": [float(lg[i]) for i in top], "first8": [float(v) for v in lg[:8]]}


def summary_line(n_gen: int, elapsed: float, n_prompt: int, prefill_secs: float) -> str:
    """The timing line src/main.rs:117-132 prints after generation."""
    decode_tokens = max(n_gen - 1, 0)
    return (f"[{n_gen} tokens generated in {elapsed:.2f}s | prefill: {n_prompt} tok in {prefill_secs:.2f}s "
            f"({n_prompt / max(prefill_secs, 1e-9):.1f} tok/s) | decode: ~{decode_tokens} tok in "
            f"{elapsed - prefill_secs:.2f}s ({decode_tokens / max(elapsed - prefill_secs, 1e-9):.2f} tok/s)]")


@dataclass
class TextOutput:
    prompt_rendered: str
    prompt_ids: List[int]
    tokens: List[int]
    text: str
    logits_first_step: np.ndarray
    prefill_secs: float
    elapsed: float
    summary: str


def generate_text(model, tokenizer: Tokenizer, template_path: str, prompt: str, params,
                  out: Optional[TextIO] = None, bos_token: str = "<s>",
                  dump_first_logits: Optional[str] = None,
                  on_text: Optional[Callable[[str], None]] = None) -> TextOutput:
    """src/main.rs:73-133: render the chat template, encode it without
    special tokens, generate, and stream each new token's text (decoded
    alone, special tokens skipped) to `out` as it arrives."""
    from .model import generate
    rendered = render_chat_template(template_path, prompt, bos_token)
    ids = tokenizer.encode(rendered, False)
    pieces: List[str] = []

    def _on_token(t: int) -> None:
        try:
            s = tokenizer.decode([t], True)
        except TextError:
            return  # the reference prints nothing for an id it cannot decode
        pieces.append(s)
        if out is not None:
            out.write(s)
            out.flush()
        if on_text is not None:
            on_text(s)

    t0 = time.perf_counter()
    res = generate(model, ids, params, _on_token)
    if dump_first_logits is not None:
        with open(dump_first_logits, "w") as f:
            json.dump(first_logits_dump(res.logits_first_step), f, indent=2)
    elapsed = time.perf_counter() - t0
    line = summary_line(len(res.tokens), elapsed, len(ids), res.prefill_secs)
    return TextOutput(rendered, ids, res.tokens, "".join(pieces), res.logits_first_step, res.prefill_secs,
                      elapsed, line)
