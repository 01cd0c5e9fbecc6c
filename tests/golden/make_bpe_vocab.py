"""Writes bpe_vocab.json: a small byte-level BPE vocabulary for the tokenizer tests — TEST DATA.

    python3 tests/golden/make_bpe_vocab.py

The vocabulary is trained with the Hugging Face `tokenizers` library (a BPE trainer over Qwen2's
pre-tokenizer pattern and GPT-2's byte alphabet, which puts "!" at id 0 as in the Qwen2 and GPT-2
vocabularies) on the corpus below: English with contractions, numbers, code and white-space runs,
and text in several other scripts. Special tokens follow the learned ones, with GGUF token types
3 (CONTROL) and 4 (USER_DEFINED); "<|im" is a prefix of "<|im_start|>" and "<|im_end|>", to test
that the longest special token wins. The JSON holds the arrays a GGUF's tokenizer.ggml.tokens,
.merges and .token_type carry.
"""
from __future__ import annotations

import json
import pathlib

from tokenizers import Regex, Tokenizer, decoders, models, pre_tokenizers, trainers

QWEN2_PATTERN = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}| ?[^\s\p{L}\p{N}]+[\r\n]*|"
                 r"\s*[\r\n]+|\s+(?!\S)|\s+")
SPECIALS = [("<|endoftext|>", 3), ("<|im_start|>", 3), ("<|im_end|>", 3), ("<tool_call>", 4), ("<|im", 4)]

CORPUS = [
    "Hello world! It's a test of the tokenizer, isn't it? We'll see what they've done.",
    "I'm sure you'd like it. They're here. IT'S LOUD. You'LL see. We'RE done, I'D say.",
    "The quick brown fox jumps over the lazy dog. THE QUICK BROWN FOX. the the the the",
    "Numbers: 0 1 2 3 4 5 6 7 8 9, 10, 100, 2048, 3.14159, 1e-6, 65504, 151936 and 1,000,000.",
    "def forward(self, x):\n    return self.proj(x) * 2 + 1\n\nfor i in range(10):\n\tprint(i)\n",
    "int main(void) { return 0; }\r\n// comment\r\n#include <stdio.h>\r\n",
    "Spaces   between    words,\ttabs\t\tand\n\nnewlines \n  \n trailing   ",
    "Καλημέρα κόσμε, τι κάνεις; Ελληνικά γράμματα: αβγδε ΑΒΓΔΕ.",
    "Привет, мир! Как дела? Русский язык: абвгд АБВГД.",
    "你好，世界！今天天气很好。我们一起学习机器学习。",
    "こんにちは世界。カタカナとひらがな。日本語のテキスト。",
    "مرحبا بالعالم. هذا نص عربي للاختبار.",
    "नमस्ते दुनिया। यह हिंदी पाठ है।",
    "Café, naïve, façade, Ångström, Øre, straße, œuvre, déjà vu.",
    "Emoji: 😀 🎉 👍🏽 ❤️ 🇫🇷 — and symbols: © ® ™ € £ ¥ § ¶ • … ← → ≤ ≥ ≠ ∞.",
    "Mixed: abc123def 4ever x86_64 GPT-2 Qwen2.5-0.5B MI355X gfx950 HBM3E.",
    "URLs: https://example.com/path?query=1&x=y#frag and emails a.b@c.de",
    "Quotes: \"double\" 'single' `back` «guillemets» „low“ ‘curly’ “curly”.",
]


def train(vocab_size: int = 1200) -> tuple[list[str], list[str]]:
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(QWEN2_PATTERN), behavior="isolated", invert=False),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=vocab_size, initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                  special_tokens=[], show_progress=False)
    tok.train_from_iterator(CORPUS * 40, trainer)
    model = json.loads(tok.to_str())["model"]
    vocab = sorted(model["vocab"].items(), key=lambda kv: kv[1])
    assert [i for _, i in vocab] == list(range(len(vocab)))
    merges = [m if isinstance(m, str) else " ".join(m) for m in model["merges"]]
    return [t for t, _ in vocab], merges


def main() -> None:
    tokens, merges = train()
    types = [1] * len(tokens)
    for text, kind in SPECIALS:
        tokens.append(text)
        types.append(kind)
    out = {"tokens": tokens, "merges": merges, "token_type": types, "corpus": CORPUS}
    path = pathlib.Path(__file__).with_name("bpe_vocab.json")
    path.write_text(json.dumps(out, ensure_ascii=False, indent=0) + "\n", encoding="utf-8")
    print(f"{path}: {len(tokens)} tokens, {len(merges)} merges")


if __name__ == "__main__":
    main()
