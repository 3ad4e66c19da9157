"""The text front-end driving the device decode path: the streamed text is
the per-token decode of exactly the ids `generate` returns for the encoded
prompt, and those are the oracle's greedy ids."""
import io
import os

import pytest

from conftest import model_root
from textfixtures import make_word_tokenizer

pytestmark = pytest.mark.gpu


def test_generate_text_tiny(tmp_path):
    import tinyminigo_amd as T
    from oracle import oracle as O
    from tinyminigo_amd import text as X
    from tinyminigo_amd import workloads as W
    path = W.ensure_model(W.TINY, model_root())
    tok = X.Tokenizer.from_file(make_word_tokenizer(str(tmp_path), W.TINY.vocab_size))
    tpl = tmp_path / "t.jinja"
    tpl.write_text("{{ bos_token }}{% for m in messages %}{{ m.content }}{% endfor %}")
    m = T.Model.load(path)
    out = io.StringIO()
    dump = str(tmp_path / "first.json")
    r = X.generate_text(m, tok, str(tpl), "w5 w17 w300 w9", T.GenParams(max_tokens=12), out=out,
                        dump_first_logits=dump)
    assert r.prompt_rendered == "<s>w5 w17 w300 w9"
    assert r.prompt_ids == [0, 5, 17, 300, 9]
    ref = O.generate(O.OracleModel.load(path), r.prompt_ids, 12)
    assert r.tokens == ref.tokens
    assert out.getvalue() == r.text == "".join(tok.decode([t], True) for t in r.tokens)
    assert os.path.exists(dump) and r.summary.startswith(f"[{len(r.tokens)} tokens generated")
