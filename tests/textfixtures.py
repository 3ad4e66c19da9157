"""A synthetic word-level tokenizer for the text front-end tests: id 0 is
"<s>", id 1 "</s>" (both special), id i >= 2 the word "w<i>"."""
import os


def make_word_tokenizer(directory: str, vocab_size: int) -> str:
    from tokenizers import Tokenizer, decoders, models, pre_tokenizers
    vocab = {"<s>": 0, "</s>": 1}
    for i in range(2, vocab_size):
        vocab[f"w{i}"] = i
    vocab["<unk>"] = vocab_size  # outside the model's ids
    tk = Tokenizer(models.WordLevel(vocab, unk_token="<unk>"))
    tk.pre_tokenizer = pre_tokenizers.Whitespace()
    tk.add_special_tokens(["<s>", "</s>"])
    tk.decoder = decoders.WordPiece(prefix="##")  # words joined by spaces
    path = os.path.join(directory, "tokenizer.json")
    tk.save(path)
    return path
