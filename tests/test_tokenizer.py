"""Byte-level BPE tokenizer and chat prompt (reference src/tokenizer.cpp,
cli/main.cpp:1037-1039): the library (C-ABI, gfxinfer_tokenizer_*) against the Python
oracle (oracle/tokenizer.py), and the oracle pinned against HF `tokenizers` 0.22, an
independent implementation of the tokenizer.json format, on the committed fixture
tests/golden/tokenizer_small.json (written by tests/golden/make_tokenizer_fixture.py),
and its pre-token split against PCRE2 itself (the system libpcre2-8 the reference links,
with the reference's pattern and flags).  CPU only."""
import json
import os
import random
import unicodedata

import pytest

from gfxinfer_amd import GfxinferError, CORRUPT_ARTIFACT, INVALID_ARGUMENT
from gfxinfer_amd.runtime import Tokenizer, render_chat_prompt
from oracle.tokenizer import OracleTokenizer, byte_alphabet
from oracle.tokenizer import render_chat_prompt as oracle_render

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "tokenizer_small.json")

CASES = [
    "", " ", "  ", "\n", "\r\n", " \n \n  x", "a", "Hello world!", "Hello  world", "trailing space ",
    "tabs\tand\ttabs", "It's we'll they've I'M she'D you'RE 'tis 'hello", "don't, won't; can't...",
    "12345 and 3.14159 and -7", "x²+y²=z² ½ ① ٣", "naïve café Straße déjà vu", "ÉCOLE Ωμέγα Привет мир",
    "你好，世界！東京 こんにちは 안녕하세요", "emoji 🙂🚀 mix", "é vs é", "Å ring",
    "line1\nline2\r\nline3\n\n\nend", "   leading spaces", "punct!!! ??? ;;; (a) [b] {c}",
    " nbsp here", "mixed em spaces", "<|im_start|>user\nhi<|im_end|>",
    "<think>\n\n</think>\n\n", "<|im_end|><|im_end|>", "x<|endoftext|>y", "<|im_start|>",
    "code: if (a == b) { return x[i] * 2; }", "path/to/file.txt #tag @user $5 %20 ^_^ ~~",
    "'s'S'ſ", "\t\n\t \n", "ending with newline\n",
]


@pytest.fixture(scope="module")
def document():
    with open(FIXTURE, "rb") as f:
        return f.read()


@pytest.fixture(scope="module")
def library(document):
    tok = Tokenizer(document)
    yield tok
    tok.close()


@pytest.fixture(scope="module")
def oracle(document):
    return OracleTokenizer(document)


# U+180E is \s for PCRE2 with UCP (\h keeps it) but not for White_Space-based engines
# such as HF's: these cases follow the reference's engine.
MVS_CASES = ["a!\u180e", "x \u180e y", "\u180e\u180e\n", "word\u180e!!", "\u180e", "a\u180e\u180eb",
             "!!\u180e\r\n", " \u180e  z"]


def random_texts(count=300, seed=7):
    rng = random.Random(seed)
    pool = list("abcXYZ éèüßñ ΩЖ你好🙂 0123456789 .,!?'\"-_()[]{}<>/\\|@#$%^&*+=~` \t\n\r") + \
        ["'s", "'LL", " \n", "\r\n", "<|im_end|>", "<think>", "é", " "]
    return ["".join(rng.choice(pool) for _ in range(rng.randint(0, 40))) for _ in range(count)]


def test_oracle_matches_hf_tokenizers(document, oracle):
    """Pins the oracle: HF tokenizers reads the same document (NFC, the Split pattern,
    ByteLevel, BPE) and must give the same ids and decoded bytes."""
    hf_tokenizers = pytest.importorskip("tokenizers")
    hf = hf_tokenizers.Tokenizer.from_str(document.decode("utf-8"))
    for text in CASES + random_texts():
        want = hf.encode(text, add_special_tokens=False).ids
        assert oracle.encode(text) == want, repr(text)
        assert oracle.decode_bytes(want).decode("utf-8") == hf.decode(want, skip_special_tokens=False)


def _pcre2_split(lib, code, text: str) -> list[str]:
    """split_pretokens (tokenizer.cpp:135-172): anchored matches from each offset."""
    import ctypes
    raw = text.encode("utf-8")
    match = lib.pcre2_match_data_create_from_pattern_8(code, None)
    out, offset = [], 0
    try:
        while offset < len(raw):
            rc = lib.pcre2_match_8(code, raw, len(raw), offset, 0x80000000, match, None)  # PCRE2_ANCHORED
            assert rc >= 1, (text, offset)
            vec = ctypes.cast(lib.pcre2_get_ovector_pointer_8(match), ctypes.POINTER(ctypes.c_size_t))
            assert vec[0] == offset and vec[1] > offset
            out.append(raw[vec[0]:vec[1]].decode("utf-8"))
            offset = vec[1]
    finally:
        lib.pcre2_match_data_free_8(match)
    return out


def test_oracle_pretokens_match_pcre2():
    """The oracle's pre-token split equals PCRE2's with the reference's pattern and
    flags (PCRE2_UTF | PCRE2_UCP, tokenizer.cpp:137-146), U+180E included."""
    import ctypes
    import ctypes.util
    from oracle.tokenizer import pretokens
    name = ctypes.util.find_library("pcre2-8") or "libpcre2-8.so.0"
    try:
        lib = ctypes.CDLL(name)
    except OSError:
        pytest.skip("libpcre2-8 is not installed")
    P, SZ = ctypes.c_void_p, ctypes.c_size_t
    lib.pcre2_compile_8.restype = P
    lib.pcre2_compile_8.argtypes = [ctypes.c_char_p, SZ, ctypes.c_uint32, ctypes.POINTER(ctypes.c_int),
                                    ctypes.POINTER(SZ), P]
    lib.pcre2_match_data_create_from_pattern_8.restype = P
    lib.pcre2_match_data_create_from_pattern_8.argtypes = [P, P]
    lib.pcre2_match_8.restype = ctypes.c_int
    lib.pcre2_match_8.argtypes = [P, ctypes.c_char_p, SZ, SZ, ctypes.c_uint32, P, P]
    lib.pcre2_get_ovector_pointer_8.restype = P
    lib.pcre2_get_ovector_pointer_8.argtypes = [P]
    lib.pcre2_match_data_free_8.argtypes = [P]
    lib.pcre2_code_free_8.argtypes = [P]
    pattern = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?[\p{L}\p{M}]+|\p{N}"
               r"| ?[^\s\p{L}\p{M}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+")
    err, off = ctypes.c_int(0), SZ(0)
    code = lib.pcre2_compile_8(pattern.encode(), SZ(-1).value, 0x00080000 | 0x00020000,  # UTF | UCP
                               ctypes.byref(err), ctypes.byref(off), None)
    assert code, err.value
    try:
        for text in CASES + MVS_CASES + random_texts(seed=17):
            nfc = unicodedata.normalize("NFC", text)
            assert pretokens(nfc) == _pcre2_split(lib, code, nfc), repr(text)
    finally:
        lib.pcre2_code_free_8(code)


def test_library_matches_oracle(library, oracle):
    for text in CASES + MVS_CASES + random_texts(seed=11):
        ids = library.encode(text)
        assert ids == oracle.encode(text), repr(text)
        assert library.decode_bytes(ids) == oracle.decode_bytes(ids)


def test_round_trip_is_nfc(library):
    """decode(encode(text)) == NFC(text) outside added tokens (the byte alphabet loses
    nothing)."""
    for text in CASES + random_texts(seed=13):
        if "<" in text:
            continue
        assert library.decode(library.encode(text)) == unicodedata.normalize("NFC", text), repr(text)


def test_byte_alphabet_and_every_byte_encodes(library, oracle):
    alphabet = byte_alphabet()
    assert len(set(alphabet)) == 256 and alphabet[ord("A")] == "A" and alphabet[0x20] == "Ġ"
    raw = bytes(range(1, 256))
    # invalid UTF-8 cannot be passed as text; every single byte of valid UTF-8 is covered
    # by decoding each alphabet piece back to its byte
    ids = [oracle.ids[alphabet[b]] for b in raw]
    assert library.decode_bytes(ids) == raw


def test_merges_as_strings_or_pairs(document, library):
    doc = json.loads(document)
    doc["model"]["merges"] = [" ".join(m) if isinstance(m, list) else m for m in doc["model"]["merges"]]
    strings = Tokenizer(json.dumps(doc, ensure_ascii=False).encode("utf-8"))
    for text in CASES:
        assert strings.encode(text) == library.encode(text)
    strings.close()


def test_vocabulary_size_and_added_tokens(library, oracle):
    assert library.vocabulary_size == len(oracle.pieces)
    for content, i in oracle.added:
        assert library.encode(content) == [i]
        assert library.decode([i]) == content
    # the longest added token wins where two start at the same position
    assert library.encode("<|im_end|>x") == [oracle.ids["<|im_end|>"]] + oracle.encode("x")


def test_chat_prompt(library, oracle):
    prompt = "What is 12*7? Answer briefly, please."
    rendered = render_chat_prompt(prompt)
    assert rendered == oracle_render(prompt)
    assert rendered.startswith("<|im_start|>user\n") and rendered.endswith("<think>\n\n</think>\n\n")
    ids = library.encode(rendered)
    assert ids == oracle.encode(rendered)
    assert ids[0] == oracle.ids["<|im_start|>"] and oracle.ids["<think>"] in ids
    assert render_chat_prompt("") == oracle_render("")


def test_rejects_malformed_documents(document):
    doc = json.loads(document)

    def status(payload):
        with pytest.raises(GfxinferError) as err:
            Tokenizer(payload)
        return err.value.code

    assert status(b"") == INVALID_ARGUMENT
    assert status(b"{") == CORRUPT_ARTIFACT
    assert status(b"[1, 2]") == CORRUPT_ARTIFACT
    assert status(document + b" x") == CORRUPT_ARTIFACT
    gap = json.loads(document)
    piece = next(iter(gap["model"]["vocab"]))
    gap["model"]["vocab"][piece] = len(gap["model"]["vocab"]) + 50  # leaves ids without a piece
    assert status(json.dumps(gap).encode()) == CORRUPT_ARTIFACT
    dup = json.loads(document)
    keys = list(dup["model"]["vocab"])
    dup["model"]["vocab"][keys[1]] = dup["model"]["vocab"][keys[0]]
    assert status(json.dumps(dup).encode()) == CORRUPT_ARTIFACT
    bad_merge = json.loads(document)
    bad_merge["model"]["merges"][0] = "nospace"
    assert status(json.dumps(bad_merge).encode()) == CORRUPT_ARTIFACT
    no_vocab = dict(doc)
    no_vocab["model"] = {k: v for k, v in doc["model"].items() if k != "vocab"}
    assert status(json.dumps(no_vocab).encode()) == CORRUPT_ARTIFACT


def test_rejects_ids_outside_the_vocabulary(library):
    with pytest.raises(GfxinferError) as err:
        library.decode([library.vocabulary_size])
    assert err.value.code == INVALID_ARGUMENT
    assert library.decode([]) == ""
    assert library.encode("") == []
