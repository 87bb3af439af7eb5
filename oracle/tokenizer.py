r"""CPU oracle of the byte-level BPE tokenizer (test infrastructure only: imported by
tests/, never by the product).

A restatement, in Python, of /root/reference/src/tokenizer.cpp:
  * byte alphabet          tokenizer.cpp:68-85, 108-120 (printable Latin-1 bytes keep
                           their code point, the other 68 take 256, 257, ...)
  * from_json              tokenizer.cpp:174-248 (ids of model.vocab and added_tokens
                           cover 0 .. N-1; merges ranked by position)
  * decode                 tokenizer.cpp:250-275
  * encode                 tokenizer.cpp:277-357 (added tokens cut the raw text at the
                           earliest match, the longest at a tie; each other segment is
                           NFC-normalized, split by the pre-token pattern :143-146 and
                           BPE-merged; the best-ranked pair is joined at every
                           non-overlapping occurrence, left to right, until none is left)
NFC comes from `unicodedata` (the reference uses ICU) and the pattern runs on the
`regex` module (the reference uses PCRE2 with UTF/UCP).  Under PCRE2_UCP, \s is
\p{Z} plus \h plus \v, which is Unicode White_Space plus U+180E (MONGOLIAN VOWEL
SEPARATOR, kept in PCRE2's \h); `regex`'s \s is White_Space alone, so the pattern below
spells \s as [\s\u180E] and \S as its complement.  The split is pinned against PCRE2
itself (the system libpcre2-8, the library the reference links) and the whole encoder
against HF `tokenizers` on the committed fixture in tests/test_tokenizer.py.
"""
from __future__ import annotations

import json
import unicodedata

import regex

PATTERN = regex.compile(
    r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?[\p{L}\p{M}]+|\p{N}"
    r"| ?[^\s\u180E\p{L}\p{M}\p{N}]+[\r\n]*|[\s\u180E]*[\r\n]+|[\s\u180E]+(?![^\s\u180E])|[\s\u180E]+")


def pretokens(text: str) -> list[str]:
    """The pre-token split of already-normalized text (tokenizer.cpp:135-172)."""
    return PATTERN.findall(text)


def byte_alphabet() -> list[str]:
    """byte -> its alphabet character (tokenizer.cpp:108-120)."""
    printable = set(range(33, 127)) | set(range(161, 173)) | set(range(174, 256))
    out, extra = [], 256
    for b in range(256):
        if b in printable:
            out.append(chr(b))
        else:
            out.append(chr(extra))
            extra += 1
    return out


class OracleTokenizer:
    def __init__(self, document: bytes | str):
        doc = json.loads(document)
        model = doc["model"]
        vocab, added = model["vocab"], doc["added_tokens"]
        size = 1 + max([int(i) for i in vocab.values()] + [int(a["id"]) for a in added])
        self.pieces = [None] * size
        self.ids = {}
        for piece, i in vocab.items():
            if self.pieces[i] is not None:
                raise ValueError("duplicated vocabulary id")
            self.pieces[i] = piece
            self.ids[piece] = i
        self.added = []
        for a in added:
            self.pieces[a["id"]] = a["content"]
            self.ids[a["content"]] = a["id"]
            self.added.append((a["content"], a["id"]))
        if any(p is None for p in self.pieces):
            raise ValueError("an id has no piece")
        self.ranks = {}
        for rank, m in enumerate(model["merges"]):
            left, right = m.split(" ") if isinstance(m, str) else m
            self.ranks.setdefault((left, right), rank)
        self.added.sort(key=lambda a: -len(a[0]))  # stable: the longest first
        self.alphabet = byte_alphabet()
        self.inverse = {c: b for b, c in enumerate(self.alphabet)}

    def _bpe(self, pretoken: str) -> list[int]:
        symbols = [self.alphabet[b] for b in pretoken.encode("utf-8")]
        while len(symbols) > 1:
            best = None
            for i in range(len(symbols) - 1):
                r = self.ranks.get((symbols[i], symbols[i + 1]))
                if r is not None and (best is None or r < best[0]):
                    best = (r, symbols[i], symbols[i + 1])
            if best is None:
                break
            _, left, right = best
            joined, i = [], 0
            while i < len(symbols):
                if i + 1 < len(symbols) and symbols[i] == left and symbols[i + 1] == right:
                    joined.append(left + right)
                    i += 2
                else:
                    joined.append(symbols[i])
                    i += 1
            symbols = joined
        return [self.ids[s] for s in symbols]

    def _segment(self, text: str) -> list[int]:
        out = []
        for piece in pretokens(unicodedata.normalize("NFC", text)):
            out.extend(self._bpe(piece))
        return out

    def encode(self, text: str) -> list[int]:
        out, cursor = [], 0
        while cursor < len(text):
            best = None
            for content, i in self.added:
                at = text.find(content, cursor)
                if at >= 0 and (best is None or at < best[0]):
                    best = (at, content, i)
            if best is None:
                out.extend(self._segment(text[cursor:]))
                break
            at, content, i = best
            out.extend(self._segment(text[cursor:at]))
            out.append(i)
            cursor = at + len(content)
        return out

    def decode_bytes(self, ids) -> bytes:
        return bytes(self.inverse[c] for i in ids for c in self.pieces[i])


def render_chat_prompt(prompt: str) -> str:
    """cli/main.cpp:1037-1039."""
    return ("<|im_start|>user\n" + prompt +
            "<|im_end|>\n<|im_start|>assistant\n<think>\n\n</think>\n\n")
