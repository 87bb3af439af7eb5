"""Writes tests/golden/tokenizer_small.json: a small byte-level BPE tokenizer in the Qwen
tokenizer.json layout (NFC normalizer, the Qwen pre-token pattern of
/root/reference/src/tokenizer.cpp:143-146 as an isolated Split, ByteLevel without its own
regex, BPE model, the chat special tokens as added tokens), trained by HF `tokenizers`
(0.22) on a seeded synthetic multilingual corpus.  The real Qwen file has ~248k pieces;
this one keeps the format and every code path at a size a CPU test loads in
milliseconds.  Run from the repository root: python3 tests/golden/make_tokenizer_fixture.py
"""
import json
import os
import random

from tokenizers import Regex, Tokenizer, decoders, models, normalizers, pre_tokenizers, trainers

HERE = os.path.dirname(os.path.abspath(__file__))
PATTERN = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?[\p{L}\p{M}]+|\p{N}"
           r"| ?[^\s\p{L}\p{M}\p{N}]+[\r\n]*|\s*[\r\n]+|\s+(?!\S)|\s+")
SPECIAL = ["<|endoftext|>", "<|im_start|>", "<|im_end|>", "<think>", "</think>", "<tool_call>", "</tool_call>"]


def corpus(seed=2026, lines=3000):
    rng = random.Random(seed)
    words = ("the quick brown fox jumps over lazy dog speculative decoding verify draft token accepted "
             "rejected window state head layer matrix weight scale group value key query we they it "
             "i you don't it's we'll they've she'd I'm can't won't shouldn't").split()
    extra = ["héllo", "naïve", "café", "Straße", "größer", "déjà", "ÉCOLE", "Ωμέγα", "αβγ", "Привет", "мир",
             "你好", "世界", "東京", "こんにちは", "안녕하세요", "🙂", "🚀", "x²", "½", "①", "٣", "é"]
    punct = [".", ",", "!", "?", ";", ":", "...", "--", "(", ")", "[", "]", "{", "}", "\"", "'", "#", "$", "%",
             "&", "*", "+", "=", "<", ">", "/", "\\", "|", "@", "^", "_", "`", "~"]
    out = []
    for _ in range(lines):
        parts = []
        for _ in range(rng.randint(3, 14)):
            r = rng.random()
            if r < 0.55:
                w = rng.choice(words)
                parts.append(w.capitalize() if rng.random() < 0.15 else w)
            elif r < 0.7:
                parts.append(rng.choice(extra))
            elif r < 0.85:
                parts.append(str(rng.randint(0, 10 ** rng.randint(1, 6))))
            else:
                parts.append(rng.choice(punct))
        sep = rng.choice([" ", " ", " ", "  ", "\t", "\n", " \n", "\r\n"])
        out.append(sep.join(parts))
    return out


def build(vocab_size=900):
    tok = Tokenizer(models.BPE())
    tok.normalizer = normalizers.NFC()
    tok.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(PATTERN), behavior="isolated"),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=vocab_size, special_tokens=SPECIAL, show_progress=False,
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    tok.train_from_iterator(corpus(), trainer=trainer)
    return tok


if __name__ == "__main__":
    doc = json.loads(build().to_str())
    with open(os.path.join(HERE, "tokenizer_small.json"), "w", encoding="utf-8") as f:
        json.dump(doc, f, ensure_ascii=False, indent=None, separators=(",", ":"))
        f.write("\n")
    print("pieces", len(doc["model"]["vocab"]), "merges", len(doc["model"]["merges"]))
