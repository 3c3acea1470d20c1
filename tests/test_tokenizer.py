"""The byte-level BPE tokenizer (neonengine_amd/tokenizer.py) against the
Hugging Face `tokenizers` library on a vocabulary trained here: a byte-level
BPE model trained with the o200k pre-tokenization pattern on a synthetic
multi-script corpus.  Both must give the same ids on held-out text; decode
must invert encode.  The real o200k_harmony vocabulary is not available
offline, so the 201088-entry table itself is not checked (its special ids
are documented as published).
"""
import os

import numpy as np
import pytest

from neonengine_amd import tokenizer as ntk

tokenizers = pytest.importorskip("tokenizers")
pytest.importorskip("regex")

WORDS = ["the", "model", "Token", "loop", "expert", "gate", "ROUTER", "don't", "I'LL", "we've",
         "attention", "sink", "MXFP4", "σκύλος", "Ελλάδα", "данные", "Модель", "数据", "模型",
         "東京", "مرحبا", "שלום", "café", "naïve", "über", "😀", "🚀x", "x²", "a/b", "foo_bar",
         "3.14159", "2026", "1234567", "0x1F", "--flag", "e-mail", "(paren)", "[idx]", "#tag"]
SEPS = [" ", "  ", "\n", "\n\n", "\t", " \n ", "\r\n", ", ", ". ", "! ", "? ", ": ", "   "]


def synth_text(rng, n):
    parts = []
    for _ in range(n):
        parts.append(WORDS[rng.integers(len(WORDS))])
        parts.append(SEPS[rng.integers(len(SEPS))])
    return "".join(parts)


@pytest.fixture(scope="module")
def trained(tmp_path_factory):
    from tokenizers import Tokenizer, Regex, decoders, models, pre_tokenizers, trainers
    rng = np.random.default_rng(0)
    corpus = [synth_text(rng, 60) for _ in range(400)]
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(ntk.O200K_PATTERN), behavior="isolated"),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=1200, show_progress=False,
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                  special_tokens=["<|start|>", "<|end|>", "<|message|>"])
    tok.train_from_iterator(corpus, trainer)
    path = str(tmp_path_factory.mktemp("tok") / "tokenizer.json")
    tok.save(path)
    return tok, path


def test_matches_hf_bpe_on_held_out_text(trained):
    hf, path = trained
    ours = ntk.Tokenizer.from_hf_json(path)
    rng = np.random.default_rng(1)
    for i in range(300):
        text = synth_text(rng, int(rng.integers(1, 40)))
        want = hf.encode(text).ids
        got = ours.encode(text)
        assert got == want, (i, repr(text), got[:20], want[:20])
        assert ours.decode(got) == text


def test_specials_and_round_trip(trained):
    hf, path = trained
    ours = ntk.Tokenizer.from_hf_json(path)
    text = "<|start|>user<|message|>Hello, wörld! 12345<|end|>"
    got = ours.encode(text)
    assert got == hf.encode(text).ids
    assert got[0] == ours.specials["<|start|>"] and got[-1] == ours.specials["<|end|>"]
    assert ours.decode(got) == text
    # not allowed: the special's text is ordinary text
    plain = ours.encode(text, allowed_special=())
    assert ours.specials["<|start|>"] not in plain
    assert ours.decode(plain) == text


def test_tiktoken_file_round_trip(trained, tmp_path):
    _, path = trained
    ours = ntk.Tokenizer.from_hf_json(path)
    tt = str(tmp_path / "vocab.tiktoken")
    ours.save_tiktoken(tt)
    again = ntk.Tokenizer.from_tiktoken_file(tt, specials=ours.specials)
    rng = np.random.default_rng(2)
    for _ in range(50):
        text = synth_text(rng, 20)
        assert again.encode(text) == ours.encode(text)


def test_merges_by_rank_of_the_concatenation():
    """tiktoken's rule on a hand-built vocabulary: 'ab' (rank 256) merges
    before 'bc' (257), then 'abc' (258) joins the result; the same bytes in
    another order merge differently."""
    ranks = {bytes([b]): b for b in range(256)}
    ranks[b"ab"] = 256
    ranks[b"bc"] = 257
    ranks[b"abc"] = 258
    ranks[b"cd"] = 259
    tok = ntk.Tokenizer(ranks, {}, pattern=r"\S+|\s+")
    assert tok.encode("abcd") == [258, ord("d")]
    assert tok.encode("bcd") == [257, ord("d")]
    assert tok.encode("cab") == [ord("c"), 256]
    assert tok.decode(tok.encode("abcd abc")) == "abcd abc"


def test_vocabulary_needs_every_byte():
    with pytest.raises(ValueError):
        ntk.Tokenizer({b"a": 0}, {})
