"""Writes tokenizer_cases.json: the reference tokenizer's outputs on fixed texts — TEST DATA.

    make -C oracle ref && python3 tests/golden/make_tokenizer_golden.py

Runs the reference's own muyo_llm::Tokenizer (src/Tokenizer.cpp with the llama.cpp Unicode files it
vendors), compiled from the reference tree into oracle/_ref/libref_tokenizer.so, over the texts
below with the vocabulary of bpe_vocab.json, once with tokenizer.ggml.pre = "qwen2" and once with
"gpt2". Records each text (hex), the ids with and without special-token parsing (null where the
reference throws), and every id's TokenBytes and IsSpecial.
"""
from __future__ import annotations

import ctypes
import json
import pathlib
import random
import sys
import tempfile

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
import gguf_writer  # noqa: E402

REF = HERE.parent.parent / "oracle" / "_ref" / "libref_tokenizer.so"

FIXED = [
    "", "!", "Hello world!", "Hello world", " Hello", "  Hello", "Hello ", "Hello  ", "\tHello", "\t\tHello",
    "It's", "IT'S", "it'S", "we'Re", "they'VE", "I'm", "I'M", "you'll", "YOU'LL", "he'd", "'s", "'", "''", "'x",
    "'re", "'ll't", "don't stop", "rock 'n' roll",
    "12345", "3.14159", "1,000,000", " 42", "x86_64", "abc123def", "٣٤٥", "Ⅻ", "½",
    "a\nb", "a\r\nb", "a \n b", "a\n\n\nb", "a  \n\n  b", "a\r\rb", "\n", "\r\n", " \n", "\n ", "   ", " ",
    "a b", "a　b", "a b", "a\u0085b", "a\x0bb", "a\x0cb", "a\x1cb", "a​b", "a  b",
    "end.\n", "Wow!!!\n\n", "...\r\n", " ...", "(x)", "[1, 2]", "a-b_c.d", "#include <x>", "<<>>",
    "Καλημέρα κόσμε", "Привет мир", "你好，世界！", "こんにちは世界。", "مرحبا بالعالم", "नमस्ते दुनिया",
    "Café naïve façade", "été", "😀🎉👍🏽", "❤️", "🇫🇷", "👨‍👩‍👧", "©®™€", "←→≤≥",
    "<|im_start|>", "<|im_start|>user\nHi<|im_end|>\n", "<|im", "<|imx", "<|im_end|>x", "<|im_start|",
    "<|endoftext|><|endoftext|>", "a<tool_call>b", "<tool_call", "x <|im_start|> y",
    "<|im_start|>system\nYou are Qwen, created by Alibaba Cloud. You are a helpful assistant.<|im_end|>\n"
    "<|im_start|>user\nHello<|im_end|>\n<|im_start|>assistant\n",
    "def f(x):\n    return x * 2\n", "\tif (a) {\n\t\treturn;\n\t}\n",
    "The quick brown fox jumps over the lazy dog.", "THE QUICK BROWN FOX",
]

# Byte strings that are not valid UTF-8, and one code point above U+10FFFF (the reference throws).
RAW = [b"\x80", b"a\x80b", b"\xc3", b"\xc3(", b"\xe2\x82", b"\xe2\x82(", b"\xf0\x9f\x98", b"\xc0\x80",
       b"\xc1\xbf", b"\xed\xa0\x80", b"\xf8\x88\x80\x80\x80", b"\xff\xfe", b"\xf4\x90\x80\x80", b"ok\xf7\xbf\xbf\xbf",
       b"\xef\xbf\xbd", b"caf\xe9"]

POOL = (list("abcXYZ'sStTreREvVmMlLdD") + list("0123456789") + list(" \t\n\r\x0b\x0c") +
        list("!?.,;:-_()[]{}<>|/\\\"#$%&*+=@^`~") + list("αβγДЖж中文日本ひらカナ한국ـعربي") +
        [" ", "　", " ", "\u0085", "́", "‍", "️", "😀", "👍", "🏽", "١", "½", "Ⅻ"] +
        ["<|im_start|>", "<|im_end|>", "<|im", "<tool_call>", "<|endoftext|>", "<|"])


def random_texts(n: int, seed: int) -> list[bytes]:
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        s = "".join(rng.choice(POOL) for _ in range(rng.randint(1, 40)))
        b = s.encode("utf-8")
        if rng.random() < 0.15:  # splice in a stray byte
            at = rng.randint(0, len(b))
            b = b[:at] + bytes([rng.choice([0x80, 0xbf, 0xc3, 0xe2, 0xf0, 0xff])]) + b[at:]
        out.append(b)
    return out


def load_ref():
    lib = ctypes.CDLL(str(REF))
    lib.ref_tok_open.restype = ctypes.c_void_p
    lib.ref_tok_open.argtypes = [ctypes.c_char_p]
    lib.ref_tok_close.argtypes = [ctypes.c_void_p]
    lib.ref_tok_vocab_size.restype = ctypes.c_uint64
    lib.ref_tok_vocab_size.argtypes = [ctypes.c_void_p]
    lib.ref_tok_encode.restype = ctypes.c_int64
    lib.ref_tok_encode.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_uint64, ctypes.c_int,
                                   ctypes.POINTER(ctypes.c_int32), ctypes.c_uint64]
    lib.ref_tok_token_bytes.restype = ctypes.c_int64
    lib.ref_tok_token_bytes.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_char_p, ctypes.c_uint64]
    lib.ref_tok_is_special.argtypes = [ctypes.c_void_p, ctypes.c_int32]
    lib.ref_tok_last_error.restype = ctypes.c_char_p
    return lib


def ref_encode(lib, h, data: bytes, parse_special: bool):
    cap = 4 * len(data) + 4
    ids = (ctypes.c_int32 * cap)()
    n = lib.ref_tok_encode(h, data, len(data), int(parse_special), ids, cap)
    return None if n < 0 else list(ids[:n])


def main() -> None:
    if not REF.exists():
        sys.exit(f"{REF} is missing: build it with `make -C oracle ref` where the reference tree is present")
    vocab = json.loads((HERE / "bpe_vocab.json").read_text(encoding="utf-8"))
    texts = [t.encode("utf-8") for t in FIXED] + RAW + random_texts(200, 20261202)
    lib = load_ref()
    out = {"vocab": "bpe_vocab.json", "cases": {}, "token_bytes": None, "is_special": None}
    with tempfile.TemporaryDirectory() as tmp:
        for pre in ("qwen2", "gpt2"):
            path = pathlib.Path(tmp) / f"{pre}.gguf"
            gguf_writer.tokenizer_file(path, vocab, pre)
            h = lib.ref_tok_open(str(path).encode())
            assert h, lib.ref_tok_last_error()
            cases = []
            for t in texts:
                cases.append({"hex": t.hex(), "ids": ref_encode(lib, h, t, True),
                              "ids_plain": ref_encode(lib, h, t, False)})
            out["cases"][pre] = cases
            if pre == "qwen2":
                n = lib.ref_tok_vocab_size(h)
                buf = ctypes.create_string_buffer(256)
                tb = []
                for i in range(-1, n + 1):
                    k = lib.ref_tok_token_bytes(h, i, buf, 256)
                    tb.append(buf.raw[:k].hex())
                out["token_bytes"] = tb  # ids -1 .. vocab
                out["is_special"] = [lib.ref_tok_is_special(h, i) for i in range(-1, n + 1)]
            lib.ref_tok_close(h)
    path = HERE / "tokenizer_cases.json"
    path.write_text(json.dumps(out, separators=(",", ":")) + "\n")
    print(f"{path}: {len(texts)} texts x 2 patterns")


if __name__ == "__main__":
    main()
