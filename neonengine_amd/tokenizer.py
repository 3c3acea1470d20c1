"""Byte-level BPE tokenizer for the gpt-oss vocabulary (o200k_harmony).

Host-side text <-> token ids for the token loop (the library itself works on
ids).  The algorithm is tiktoken's, as gpt-oss's tokenizer is defined:
  1. special tokens are matched first and map to their ids;
  2. the rest is split by the o200k pre-tokenization pattern (the published
     `o200k_base` regular expression: letter runs with an optional leading
     non-letter and English contractions, digit runs of at most three,
     punctuation runs, newline runs, whitespace);
  3. each piece's UTF-8 bytes are merged by byte-pair ranks: repeatedly join
     the adjacent pair whose concatenation has the lowest rank in the
     vocabulary, until no adjacent pair is a vocabulary token.
Decoding concatenates the tokens' bytes.

Vocabularies are read from local files only (nothing is fetched):
  - tiktoken format: one `<base64 token bytes> <rank>` per line (e.g.
    `o200k_base.tiktoken`), with the special tokens given separately
    (`HARMONY_SPECIALS` are gpt-oss's);
  - Hugging Face `tokenizer.json` with a byte-level BPE model: `model.vocab`
    in the GPT-2 byte-to-unicode alphabet (ids are the ranks) and
    `added_tokens` as the specials.

No counterpart in the reference, which has no text path.  The parity test
(tests/test_tokenizer.py) trains a byte-level BPE vocabulary locally with
the `tokenizers` library and the same pattern, and checks that both give the
same ids.
"""
from __future__ import annotations

import base64
import json
from typing import Iterable

# The o200k_base pre-tokenization pattern (tiktoken, openai_public.py), which
# o200k_harmony keeps.
O200K_PATTERN = "|".join([
    r"[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]*[\p{Ll}\p{Lm}\p{Lo}\p{M}]+(?i:'s|'t|'re|'ve|'m|'ll|'d)?",
    r"[^\r\n\p{L}\p{N}]?[\p{Lu}\p{Lt}\p{Lm}\p{Lo}\p{M}]+[\p{Ll}\p{Lm}\p{Lo}\p{M}]*(?i:'s|'t|'re|'ve|'m|'ll|'d)?",
    r"\p{N}{1,3}",
    r" ?[^\s\p{L}\p{N}]+[\r\n/]*",
    r"\s*[\r\n]+",
    r"\s+(?!\S)",
    r"\s+",
])

# gpt-oss's special tokens (o200k_harmony) as the openai-harmony package
# publishes them: ids 199998.. of the 201088-entry vocabulary, the unnamed
# ids up to 201087 reserved.  No vocabulary file is available offline, so
# these ids are not checked here; from_hf_json takes the specials from the
# file instead.
HARMONY_SPECIALS = {
    "<|startoftext|>": 199998,
    "<|endoftext|>": 199999,
    "<|return|>": 200002,
    "<|constrain|>": 200003,
    "<|channel|>": 200005,
    "<|start|>": 200006,
    "<|end|>": 200007,
    "<|message|>": 200008,
    "<|call|>": 200012,
}


def _byte_unicode_map() -> dict[str, int]:
    """GPT-2's byte-level alphabet: printable bytes stand for themselves, the
    other 68 map to code points 256.. in byte order (inverse direction)."""
    keep = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAC + 1)) + \
        list(range(0xAE, 0xFF + 1))
    chars, n = {}, 0
    for b in range(256):
        if b in keep:
            chars[chr(b)] = b
        else:
            chars[chr(256 + n)] = b
            n += 1
    return chars


class Tokenizer:
    def __init__(self, ranks: dict[bytes, int], specials: dict[str, int] | None = None,
                 pattern: str = O200K_PATTERN):
        import regex
        self.ranks = dict(ranks)
        self.specials = dict(specials or {})
        self.decoder = {r: t for t, r in self.ranks.items()}
        for s, i in self.specials.items():
            self.decoder[i] = s.encode("utf-8")
        self._pat = regex.compile(pattern)
        self._special_pat = (regex.compile("|".join(regex.escape(s) for s in
                                                    sorted(self.specials, key=len, reverse=True)))
                             if self.specials else None)
        missing = [b for b in range(256) if bytes([b]) not in self.ranks]
        if missing:
            raise ValueError(f"vocabulary lacks {len(missing)} single bytes (first {missing[:4]}): "
                             "every byte must be a token for byte-level BPE")

    # ---- loading -----------------------------------------------------------
    @classmethod
    def from_tiktoken_file(cls, path: str, specials: dict[str, int] | None = None,
                           pattern: str = O200K_PATTERN) -> "Tokenizer":
        ranks = {}
        with open(path, "rb") as f:
            for line in f:
                line = line.strip()
                if not line:
                    continue
                tok, rank = line.split()
                ranks[base64.b64decode(tok)] = int(rank)
        return cls(ranks, HARMONY_SPECIALS if specials is None else specials, pattern)

    @classmethod
    def from_hf_json(cls, path: str, pattern: str = O200K_PATTERN) -> "Tokenizer":
        with open(path, encoding="utf-8") as f:
            d = json.load(f)
        model = d["model"]
        if model.get("type") != "BPE":
            raise ValueError(f"{path}: model type {model.get('type')!r}, expected BPE")
        inv = _byte_unicode_map()
        specials = {t["content"]: int(t["id"]) for t in d.get("added_tokens", [])
                    if t.get("special", False)}
        # added tokens may also sit in model.vocab; they are never merge results
        ranks = {bytes(inv[c] for c in tok): int(i) for tok, i in model["vocab"].items()
                 if tok not in specials}
        return cls(ranks, specials, pattern)

    def save_tiktoken(self, path: str) -> None:
        with open(path, "wb") as f:
            for tok, rank in sorted(self.ranks.items(), key=lambda kv: kv[1]):
                f.write(base64.b64encode(tok) + b" " + str(rank).encode() + b"\n")

    # ---- encoding ----------------------------------------------------------
    def _bpe(self, piece: bytes) -> list[int]:
        r = self.ranks.get(piece)
        if r is not None:
            return [r]
        parts = [piece[i:i + 1] for i in range(len(piece))]
        while len(parts) > 1:
            best, best_i = None, -1
            for i in range(len(parts) - 1):
                rr = self.ranks.get(parts[i] + parts[i + 1])
                if rr is not None and (best is None or rr < best):
                    best, best_i = rr, i
            if best is None:
                break
            parts[best_i:best_i + 2] = [parts[best_i] + parts[best_i + 1]]
        return [self.ranks[p] for p in parts]

    def _encode_ordinary(self, text: str, out: list[int]) -> None:
        for m in self._pat.finditer(text):
            out.extend(self._bpe(m.group().encode("utf-8")))

    def encode(self, text: str, allowed_special: str | Iterable[str] = "all") -> list[int]:
        """Token ids of `text`.  Special tokens in `allowed_special` ("all" or
        a set of names) map to their ids; elsewhere their text is encoded as
        ordinary text."""
        allowed = set(self.specials) if allowed_special == "all" else set(allowed_special)
        out: list[int] = []
        pos = 0
        if self._special_pat is not None and allowed:
            for m in self._special_pat.finditer(text):
                if m.group() not in allowed:
                    continue
                self._encode_ordinary(text[pos:m.start()], out)
                out.append(self.specials[m.group()])
                pos = m.end()
        self._encode_ordinary(text[pos:], out)
        return out

    def decode_bytes(self, ids: Iterable[int]) -> bytes:
        return b"".join(self.decoder[int(i)] for i in ids)

    def decode(self, ids: Iterable[int], errors: str = "replace") -> str:
        return self.decode_bytes(ids).decode("utf-8", errors=errors)

    @property
    def n_vocab(self) -> int:
        return max(max(self.ranks.values(), default=-1),
                   max(self.specials.values(), default=-1)) + 1
