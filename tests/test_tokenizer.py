"""The tokenizer (muyo_tokenizer_*, csrc/tokenizer.cpp) and its oracle (oracle/tokenizer.py). No GPU:
tokenizing is host work.

Pins, in order of strength:
- the reference's own Tokenizer, built from src/Tokenizer.cpp and its vendored llama.cpp Unicode
  files into oracle/_ref/ (skipped where the reference tree was absent at build time): every
  case, plus 2000 more random texts, plus the code-point classes over all of Unicode;
- tests/golden/tokenizer_cases.json, which that build wrote (312 texts, both patterns, with and
  without special-token parsing, every id's bytes and special flag): runs everywhere;
- the Hugging Face `tokenizers` library, an independent byte-level BPE implementation, on valid
  text without special tokens;
- GPT-2's published byte table (188 printable bytes stand for themselves, space is U+0120, the
  68 others follow 256 in byte order), the "!" -> [0] anchor of the reference's --tokenize mode
  (src/Tokenize.cpp:33-44), and decode(encode(x)) == x on valid text.
The vocabulary is tests/golden/bpe_vocab.json (975 tokens trained on a small multilingual corpus).
"""
import ctypes
import os
import sys
import json
import pathlib
import random

import pytest

import gguf_writer as gw
import oracle
import tokenizer as otok

sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent / "golden"))

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
VOCAB = json.loads((GOLDEN / "bpe_vocab.json").read_text(encoding="utf-8"))
CASES = json.loads((GOLDEN / "tokenizer_cases.json").read_text())
REF_PATH = oracle.HERE / "_ref" / "libref_tokenizer.so"
needs_ref = pytest.mark.skipif(not REF_PATH.exists(), reason="oracle/_ref/libref_tokenizer.so was not built")


@pytest.fixture(scope="module", params=["qwen2", "gpt2"])
def pre(request):
    return request.param


@pytest.fixture(scope="module")
def files(tmp_path_factory):
    d = tmp_path_factory.mktemp("tok")
    out = {}
    for p in ("qwen2", "gpt2"):
        out[p] = d / f"{p}.gguf"
        gw.tokenizer_file(out[p], VOCAB, p)
    return out


@pytest.fixture(scope="module")
def product(mh, files):
    made = {}
    for p, path in files.items():
        with mh.Gguf(path) as g:
            made[p] = mh.Tokenizer(g)
    yield made
    for t in made.values():
        t.close()


@pytest.fixture(scope="module")
def restated():
    return {p: otok.Tokenizer(VOCAB["tokens"], VOCAB["merges"], VOCAB["token_type"], p) for p in ("qwen2", "gpt2")}


class RefTokenizer:
    def __init__(self, path):
        lib = ctypes.CDLL(str(REF_PATH))
        vp, u64, i32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int32
        sig = {"ref_tok_open": (vp, [ctypes.c_char_p]), "ref_tok_close": (None, [vp]),
               "ref_tok_vocab_size": (u64, [vp]), "ref_tok_last_error": (ctypes.c_char_p, []),
               "ref_tok_encode": (ctypes.c_int64, [vp, ctypes.c_char_p, u64, ctypes.c_int, ctypes.POINTER(i32), u64]),
               "ref_tok_decode": (ctypes.c_int64, [vp, ctypes.POINTER(i32), u64, ctypes.c_char_p, u64]),
               "ref_tok_token_bytes": (ctypes.c_int64, [vp, i32, ctypes.c_char_p, u64]),
               "ref_tok_token_text": (ctypes.c_int64, [vp, u64, ctypes.c_char_p, u64]),
               "ref_tok_is_special": (ctypes.c_int, [vp, i32]), "ref_unicode_flags": (ctypes.c_uint32, [ctypes.c_uint32])}
        for name, (res, args) in sig.items():
            getattr(lib, name).restype, getattr(lib, name).argtypes = res, args
        self.lib = lib
        self.h = lib.ref_tok_open(str(path).encode())
        assert self.h, lib.ref_tok_last_error()

    def encode(self, data: bytes, parse_special=True):
        cap = 4 * len(data) + 4
        ids = (ctypes.c_int32 * cap)()
        n = self.lib.ref_tok_encode(self.h, data, len(data), int(parse_special), ids, cap)
        return None if n < 0 else list(ids[:n])

    def decode(self, ids) -> bytes:
        arr = (ctypes.c_int32 * max(1, len(ids)))(*ids)
        buf = ctypes.create_string_buffer(8 * len(ids) + 8)
        n = self.lib.ref_tok_decode(self.h, arr, len(ids), buf, len(buf))
        return buf.raw[:n]

    def close(self):
        self.lib.ref_tok_close(self.h)


def product_encode(tok, data: bytes, parse_special=True):
    """Ids, or None where the entry point refuses the text (a code point above U+10FFFF)."""
    import muyo_hip

    try:
        return tok.encode(data, parse_special)
    except muyo_hip.MuyoError as e:
        assert e.status == muyo_hip.MUYO_E_RANGE
        return None


def oracle_encode(tok, data: bytes, parse_special=True):
    try:
        return tok.encode(data, parse_special)
    except ValueError:
        return None


def texts(pre):
    return [(bytes.fromhex(c["hex"]), c["ids"], c["ids_plain"]) for c in CASES["cases"][pre]]


# ------------------------------------------------------------------------------------------------
# The product against the golden vectors (everywhere) and the reference build (where present).

def test_product_matches_golden_vectors(product, pre):
    tok = product[pre]
    bad = []
    for data, ids, plain in texts(pre):
        if product_encode(tok, data, True) != ids or product_encode(tok, data, False) != plain:
            bad.append(data)
    assert not bad, (len(bad), bad[:5])


def test_product_token_bytes_and_specials_match_golden(product):
    tok = product["qwen2"]
    n = tok.vocab_size()
    assert n == len(VOCAB["tokens"])
    got = [tok.token_bytes(i).hex() for i in range(-1, n + 1)]
    assert got == CASES["token_bytes"]
    assert [int(tok.is_special(i)) for i in range(-1, n + 1)] == CASES["is_special"]
    assert tok.token_for(0) == "!" and tok.token_for(n) == "" and tok.token_for(n - 1) == "<|im"


def test_decode_concatenates_token_bytes(product):
    tok = product["qwen2"]
    ids = [5, -3, 840, 10 ** 6, 826, len(VOCAB["tokens"]) - 2, 0]
    assert tok.decode_bytes(ids) == b"".join(tok.token_bytes(i) for i in ids)
    assert tok.decode_bytes([]) == b""


@needs_ref
def test_product_matches_reference_on_random_texts(product, files, pre):
    import make_tokenizer_golden as mk

    ref = RefTokenizer(files[pre])
    try:
        bad = []
        for data in mk.random_texts(2000, 7 + len(pre)):
            for special in (True, False):
                if product_encode(product[pre], data, special) != ref.encode(data, special):
                    bad.append((data, special))
        assert not bad, (len(bad), bad[:3])
    finally:
        ref.close()


@needs_ref
def test_product_decode_matches_reference(product, files):
    ref = RefTokenizer(files["qwen2"])
    try:
        rng = random.Random(3)
        for _ in range(200):
            ids = [rng.randrange(-2, len(VOCAB["tokens"]) + 2) for _ in range(rng.randint(0, 30))]
            assert product["qwen2"].decode_bytes(ids) == ref.decode(ids)
    finally:
        ref.close()


@needs_ref
def test_code_point_classes_agree_with_reference_tables(mh):
    """The product's letter/number/white-space classes over all of Unicode against the vendored
    llama.cpp tables the reference splits with. Their only differences are code points those
    tables (Unicode 15.1) hold as unassigned and the product's (Unicode 17) as letters or numbers."""
    import regex

    ref = ctypes.CDLL(str(REF_PATH))
    ref.ref_unicode_flags.restype = ctypes.c_uint32
    ref.ref_unicode_flags.argtypes = [ctypes.c_uint32]
    table = (GOLDEN.parent.parent / "muyo-llm_amd" / "csrc" / "unicode_classes.inc").read_text()
    classes = {}
    for name, bit in (("kLetterRanges", 0x4), ("kNumberRanges", 0x2), ("kWhiteSpaceRanges", 0x100)):
        body = table.split(name)[1].split("};")[0]
        spans = [tuple(int(x, 16) for x in pair.split(",")) for pair in regex.findall(r"\{(0x[0-9A-F]+, 0x[0-9A-F]+)\}", body)]
        classes[bit] = spans
    member = {bit: bytearray(0x110000) for bit in classes}
    for bit, spans in classes.items():
        for a, b in spans:
            member[bit][a:b + 1] = b"\x01" * (b - a + 1)
    newer = 0
    for cp in range(0x110000):
        f = ref.ref_unicode_flags(cp)
        for bit in classes:
            if bool(member[bit][cp]) != bool(f & bit):
                assert f == 0x0001 and bit != 0x100, (hex(cp), hex(f), bit)
                newer += 1
    assert newer < 10000, newer


# ------------------------------------------------------------------------------------------------
# The oracle's own pins.

def test_oracle_matches_golden_vectors(restated, pre):
    bad = []
    for data, ids, plain in texts(pre):
        if oracle_encode(restated[pre], data, True) != ids or oracle_encode(restated[pre], data, False) != plain:
            bad.append(data)
    assert not bad, (len(bad), bad[:5])
    n = len(VOCAB["tokens"])
    assert [restated["qwen2"].token_bytes(i).hex() for i in range(-1, n + 1)] == CASES["token_bytes"]


def test_oracle_byte_table_is_gpt2s():
    table = otok.bytes_to_unicode()
    identity = [b for b in range(256) if table[b] == chr(b)]
    assert len(identity) == 188
    assert table[ord(" ")] == "Ġ" and table[ord("\n")] == "Ċ" and table[0] == "Ā" and table[0xAD] == "\u0143"
    assert sorted(ord(table[b]) for b in range(256) if b not in identity) == list(range(256, 256 + 68))


def test_oracle_and_product_agree_with_hf_tokenizers(product, restated):
    """An independent implementation of byte-level BPE over the same pattern, vocabulary and merges
    (no special tokens; valid UTF-8 only)."""
    tokenizers = pytest.importorskip("tokenizers")
    from tokenizers import Regex, decoders, models, pre_tokenizers

    import make_bpe_vocab as mk

    vocab = {t: i for i, t in enumerate(VOCAB["tokens"]) if VOCAB["token_type"][i] == 1}
    merges = [tuple(m.split(" ", 1)) for m in VOCAB["merges"]]
    hf = tokenizers.Tokenizer(models.BPE(vocab=vocab, merges=merges))
    hf.pre_tokenizer = pre_tokenizers.Sequence([
        pre_tokenizers.Split(Regex(mk.QWEN2_PATTERN), behavior="isolated", invert=False),
        pre_tokenizers.ByteLevel(add_prefix_space=False, use_regex=False)])
    hf.decoder = decoders.ByteLevel()
    rng = random.Random(11)
    pool = [c for c in "abcXYZ'sStTreRE0123456789 \t\n\r!?.,;:-_()<>|αβγДЖж中文日本ひら" ] + ["　", "\xa0", "😀"]
    samples = [t for t in mk.CORPUS] + ["".join(rng.choice(pool) for _ in range(rng.randint(1, 30))) for _ in range(500)]
    for s in samples:
        want = hf.encode(s).ids
        assert product["qwen2"].encode(s, False) == want, s
        assert restated["qwen2"].encode(s, False) == want, s


def test_anchor_and_round_trip(product, restated, pre):
    assert product[pre].encode("!") == [0] and restated[pre].encode("!") == [0]
    for s in VOCAB["corpus"] + ["x" * 3000, " " * 100 + "y", "\n" * 50, "<|im_start|>user\nHi<|im_end|>\n"]:
        ids = product[pre].encode(s)
        assert product[pre].decode(ids) == s
        assert restated[pre].decode(ids) == s.encode()


def test_long_input_is_not_quadratic(product):
    import time

    text = ("lorem ipsum dolor sit amet " * 4000) + "z" * 20000  # a 20000-byte piece at the end
    t0 = time.perf_counter()
    ids = product["qwen2"].encode(text)
    assert time.perf_counter() - t0 < 2.0
    assert product["qwen2"].decode(ids) == text


# ------------------------------------------------------------------------------------------------
# Refusals.

def test_refusals(mh, tmp_path):
    path = tmp_path / "none.gguf"
    gw.write(path, [("general.architecture", gw.STRING, "qwen2")], [])
    with mh.Gguf(path) as g:
        with pytest.raises(mh.MuyoError) as e:
            mh.Tokenizer(g)
    assert e.value.status == mh.MUYO_E_CONTRACT
    lib = mh.load()
    n = ctypes.c_uint64()
    assert lib.muyo_tokenizer_create(None, None) == mh.MUYO_E_NULL
    assert lib.muyo_tokenizer_encode(None, b"x", 1, 1, None, 0, ctypes.byref(n)) == mh.MUYO_E_NULL
    assert lib.muyo_tokenizer_vocab_size(None) == 0 and lib.muyo_tokenizer_is_special(None, 0) == 0


def test_encode_reports_the_needed_room(product, mh):
    tok = product["qwen2"]
    lib = mh.load()
    data = b"Hello world! Hello world!"
    n = ctypes.c_uint64()
    ids = (ctypes.c_int32 * 2)()
    assert lib.muyo_tokenizer_encode(tok.handle, data, len(data), 1, ids, 2, ctypes.byref(n)) == mh.MUYO_E_RANGE
    assert n.value == len(tok.encode(data))
    assert product_encode(tok, b"ok\xf4\x90\x80\x80") is None


def test_cli_tokenize(files, product):
    """`muyo_llm --tokenize <gguf> <text>` (src/Tokenize.cpp): the ids, the round trip and the "!"
    anchor; no device is needed."""
    import subprocess

    cli = pathlib.Path(os.environ.get("MUYO_LLM_CLI") or GOLDEN.parent.parent / "muyo-llm_amd" / "muyo_llm")
    if not cli.exists():
        pytest.skip("the muyo_llm CLI is not built")
    text = "Hello world! It's <|im_start|>user\n  ok"
    p = subprocess.run([str(cli), "--tokenize", str(files["qwen2"]), text], capture_output=True, timeout=60)
    assert p.returncode == 0, p.stderr
    lines = p.stdout.decode().splitlines()
    assert lines[0] == f"[tokenize] vocab {len(VOCAB['tokens'])}, model gpt2"
    assert [int(x) for x in p.stdout.decode().split("->", 1)[1].splitlines()[0].split()] == product["qwen2"].encode(text)
    assert "[tokenize] anchor OK" in lines[-2] and lines[-1].startswith("[tokenize] OK")
    p = subprocess.run([str(cli), "--tokenize", str(files["qwen2"]), "x\xf4"], capture_output=True, timeout=60)
    assert p.returncode == 0  # U+00F4 is valid text
    p = subprocess.run([str(cli), "--tokenize", str(files["qwen2"])], capture_output=True, timeout=60)
    assert p.returncode == 2
