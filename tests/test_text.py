"""Text front-end (tinyminigo_amd.text) against the reference's own
known-answer tests (src/template.rs:31-43, src/tokenizer.rs:47-55) and
Python string semantics (the reference's minijinja runs HF templates through
its Python-compatibility callback)."""
import json
import os

import numpy as np
import pytest

from textfixtures import make_word_tokenizer

X = pytest.importorskip("tinyminigo_amd.text")

REF_TEMPLATE = ("{{ bos_token }}{% for m in messages %}<|im_start|>{{ m.role }}\n{{ m.content }}<|im_end|>\n"
                "{% endfor %}{% if add_generation_prompt %}<|im_start|>assistant\n{% endif %}")


def test_renders_reference_template(tmp_path):
    # src/template.rs:35-42: the reference's own expected string
    p = tmp_path / "t.jinja"
    p.write_text(REF_TEMPLATE)
    assert X.render_chat_template(str(p), "Hi", "<s>") == "<s><|im_start|>user\nHi<|im_end|>\n<|im_start|>assistant\n"


def test_template_context_and_string_methods(tmp_path):
    # eos/pad tokens are "</s>"; HF templates call Python string methods
    p = tmp_path / "t.jinja"
    p.write_text("{{ eos_token }}|{{ pad_token }}|{% for m in messages %}{% if m.content.startswith(' ') %}"
                 "[{{ m.content.strip().upper() }}]{% endif %}{{ m.content.replace('a', 'o') }}{% endfor %}")
    assert X.render_chat_template(str(p), "  banana ", "<s>") == "</s>|</s>|[BANANA]  bonono "


def test_template_errors(tmp_path):
    with pytest.raises(X.TextError, match="reading chat template"):
        X.render_chat_template(str(tmp_path / "missing.jinja"), "x", "<s>")
    p = tmp_path / "bad.jinja"
    p.write_text("{% for m in messages %}")
    with pytest.raises(X.TextError, match="parsing chat template"):
        X.render_chat_template(str(p), "x", "<s>")


def test_resolve_tokenizer_path():
    # src/tokenizer.rs:51-54, and the default next to the model
    assert X.resolve_tokenizer_path("/x/t.json", "/y/m.safetensors") == "/x/t.json"
    assert X.resolve_tokenizer_path(None, "/y/m.safetensors") == "/y/tokenizer.json"
    assert X.resolve_tokenizer_path(None, "m.safetensors") == "tokenizer.json"
    with pytest.raises(X.TextError, match="no parent dir"):
        X.resolve_tokenizer_path(None, "/")


def test_tokenizer_round_trip(tmp_path):
    tok = X.Tokenizer.from_file(make_word_tokenizer(str(tmp_path), 64))
    assert tok.vocab_size() == 65
    ids = tok.encode("<s>w5 w17 w63", False)
    assert ids == [0, 5, 17, 63]
    assert tok.decode(ids, True) == "w5 w17 w63"
    assert tok.decode(ids, False) == "<s> w5 w17 w63"
    assert tok.decode([1], True) == ""
    with pytest.raises(X.TextError, match="loading tokenizer from"):
        X.Tokenizer.from_file(str(tmp_path / "nope.json"))


def test_first_logits_dump_and_summary():
    lg = np.array([0.5, 3.0, -1.0, 3.0, 2.0, 0.25, 7.0, 1.0, 9.0], np.float32)
    d = X.first_logits_dump(lg)
    # a stable sort by value descending: ties keep the lower id first
    assert d["top5_ids"] == [8, 6, 1, 3, 4]
    assert d["top5_vals"] == [9.0, 7.0, 3.0, 3.0, 2.0]
    assert d["first8"] == [0.5, 3.0, -1.0, 3.0, 2.0, 0.25, 7.0, 1.0]
    json.dumps(d)
    # the reference's format (src/main.rs:117-132) evaluated by hand
    assert X.summary_line(5, 2.0, 3, 0.5) == ("[5 tokens generated in 2.00s | prefill: 3 tok in 0.50s (6.0 tok/s) "
                                              "| decode: ~4 tok in 1.50s (2.67 tok/s)]")
    assert X.summary_line(0, 1.0, 2, 0.25).startswith("[0 tokens generated")
