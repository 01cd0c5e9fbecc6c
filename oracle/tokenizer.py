"""CPU restatement of the reference's byte-level BPE tokenizer — TEST INFRASTRUCTURE ONLY.

Only tests/ may import this; the product's tokenizer is muyo-llm_amd/csrc/tokenizer.cpp. Each
function cites the reference code it restates:
- the table build: src/Tokenizer.cpp:89-152 (tokens, merges split at the first space, the
  pre-type switch, special tokens of types 3 and 4 from an INT32 token_type array);
- GPT-2's byte map: src/Tokenizer.cpp:154-183;
- the pre-split: src/Tokenizer.cpp:209-214, which calls the vendored llama.cpp
  unicode_regex_split (src/llama/unicode.cpp:1216-1408) with the pattern of
  src/Tokenizer.cpp:121-129. Both patterns have hand-written matchers there
  (unicode.cpp:474-606 for Qwen2's, :215-330 for GPT-2's), which also take what the pattern
  leaves (a lone white-space character before a non-space, then any single code point), so the
  restatement runs each pattern with the third-party `regex` module with those two fallbacks
  appended. \\s and \\S mean the White_Space property, as the vendored tables do
  (unicode-data.cpp's unicode_set_whitespace);
- the UTF-8 decode of the pre-split: unicode.cpp:30-72 and :1130-1145 (invalid bytes become
  U+FFFD one at a time; a code point above U+10FFFF makes the re-encode throw,
  unicode.cpp:1088-1115);
- the merge loop: src/Tokenizer.cpp:225-270 (lowest rank, leftmost, one merge at a time; symbols
  missing from the vocabulary fall back to their code points);
- Encode: src/Tokenizer.cpp:272-320 (longest special token at each byte, lowest id among equals);
- Decode, TokenBytes: src/Tokenizer.cpp:185-207, 322-345.

Pinned by tests/test_tokenizer.py against the reference's own Tokenizer built from its sources
into oracle/_ref/ (where the reference tree is present), against the fixed vectors that build
wrote into tests/golden/tokenizer_cases.json, against the independent Hugging Face `tokenizers`
implementation of the same algorithm, and against GPT-2's published byte table.

Letter and number classes come from the `regex` module's Unicode database (Unicode 17); the
reference's vendored tables are Unicode 15.1, so code points assigned in 16.0 and 17.0 are
letters or numbers here and unassigned there.
"""
from __future__ import annotations

import regex

WS = r"\t\n\x0b\x0c\r \x85\xa0\u1680\u2000-\u200a\u2028\u2029\u202f\u205f\u3000"

QWEN2_PRE = ("(?:'[sS]|'[tT]|'[rR][eE]|'[vV][eE]|'[mM]|'[lL][lL]|'[dD])|[^\\r\\n\\p{L}\\p{N}]?\\p{L}+|\\p{N}|"
             " ?[^\\s\\p{L}\\p{N}]+[\\r\\n]*|\\s*[\\r\\n]+|\\s+(?!\\S)|\\s+")
GPT2_PRE = "'s|'t|'re|'ve|'m|'ll|'d| ?\\p{L}+| ?\\p{N}+| ?[^\\s\\p{L}\\p{N}]+|\\s+(?!\\S)"
QWEN2_PRE_TYPES = ("qwen2", "stablelm2", "hunyuan", "solar-open")


def _compile(pattern: str) -> "regex.Pattern":
    # The matchers' fallbacks, then \s -> White_Space (inside and outside classes).
    pattern = pattern + "|\\s+|."
    pattern = pattern.replace("[^\\s", "[^" + WS).replace("\\S", "[^" + WS + "]").replace("\\s", "[" + WS + "]")
    return regex.compile(pattern, regex.DOTALL)


_PATTERNS = {True: _compile(QWEN2_PRE), False: _compile(GPT2_PRE)}


def bytes_to_unicode() -> dict[int, str]:
    """GPT-2's byte -> code point map (src/Tokenizer.cpp:154-183)."""
    printable = set(range(ord("!"), ord("~") + 1)) | set(range(0xA1, 0xAD)) | set(range(0xAE, 0x100))
    out, nxt = {}, 256
    for b in range(256):
        if b in printable:
            out[b] = chr(b)
        else:
            out[b] = chr(nxt)
            nxt += 1
    return out


def decode_for_split(data: bytes) -> list[int]:
    """unicode_cpts_from_utf8 (src/llama/unicode.cpp:30-72, 1130-1145)."""
    cps, i, n = [], 0, len(data)
    while i < n:
        b0 = data[i]
        if b0 < 0x80:
            cps.append(b0)
            i += 1
            continue
        if not b0 & 0x40:
            need = None
        elif not b0 & 0x20:
            need, cp = 1, b0 & 0x1F
        elif not b0 & 0x10:
            need, cp = 2, b0 & 0x0F
        elif not b0 & 0x08:
            need, cp = 3, b0 & 0x07
        else:
            need = None
        if need is None or i + need >= n or any(data[i + k] & 0xC0 != 0x80 for k in range(1, need + 1)):
            cps.append(0xFFFD)
            i += 1
            continue
        for k in range(1, need + 1):
            cp = (cp << 6) | (data[i + k] & 0x3F)
        cps.append(cp)
        i += need + 1
    return cps


def cpt_to_utf8(cp: int) -> bytes:
    """unicode_cpt_to_utf8 (src/llama/unicode.cpp:1088-1115): surrogates encode as written."""
    if cp <= 0x7F:
        return bytes([cp])
    if cp <= 0x7FF:
        return bytes([0xC0 | (cp >> 6), 0x80 | (cp & 0x3F)])
    if cp <= 0xFFFF:
        return bytes([0xE0 | (cp >> 12), 0x80 | ((cp >> 6) & 0x3F), 0x80 | (cp & 0x3F)])
    if cp <= 0x10FFFF:
        return bytes([0xF0 | (cp >> 18), 0x80 | ((cp >> 12) & 0x3F), 0x80 | ((cp >> 6) & 0x3F), 0x80 | (cp & 0x3F)])
    raise ValueError("invalid codepoint")


def lenient_code_points(s: bytes) -> list[bytes]:
    """src/Tokenizer.cpp:44-87: split a UTF-8 string by its lead bytes, without validation."""
    out, i = [], 0
    while i < len(s):
        b0 = s[i]
        length = 4 if b0 >= 0xF0 else 3 if b0 >= 0xE0 else 2 if b0 >= 0xC0 else 1
        out.append(s[i:i + length])
        i += length
    return out


def lenient_value(piece: bytes) -> int:
    b0 = piece[0]
    if b0 >= 0xF0:
        cp = b0 & 0x07
    elif b0 >= 0xE0:
        cp = b0 & 0x0F
    elif b0 >= 0xC0:
        cp = b0 & 0x1F
    else:
        cp = b0
    for b in piece[1:]:
        cp = (cp << 6) | (b & 0x3F)
    return cp


class Tokenizer:
    """src/Tokenizer.h:22-88, from the arrays a GGUF's tokenizer.ggml.* metadata holds."""

    def __init__(self, tokens: list[str], merges: list[str], token_type: list[int] | None = None,
                 pre: str = "gpt2"):
        if not tokens:
            raise ValueError("Tokenizer: GGUF has no tokenizer.ggml.tokens")
        self.tokens = [t.encode("utf-8", "surrogatepass") for t in tokens]
        self.token_to_id: dict[bytes, int] = {}
        for i, t in enumerate(self.tokens):
            self.token_to_id.setdefault(t, i)
        self.rank: dict[tuple[bytes, bytes], int] = {}
        for i, m in enumerate(merges):
            m = m.encode("utf-8", "surrogatepass")
            if b" " not in m:
                continue
            a, b = m.split(b" ", 1)
            self.rank.setdefault((a, b), i)
        self.byte_map = {b: c.encode("utf-8") for b, c in bytes_to_unicode().items()}
        self.cp_to_byte = {ord(c): b for b, c in bytes_to_unicode().items()}
        self.qwen2 = pre in QWEN2_PRE_TYPES
        self.specials: list[tuple[bytes, int]] = []
        self.special = [False] * len(tokens) if token_type is not None else []
        if token_type is not None:
            for i, t in enumerate(token_type[:len(tokens)]):
                if t in (3, 4):
                    self.special[i] = True
                    if self.tokens[i]:
                        self.specials.append((self.tokens[i], i))

    def pre_tokenize(self, data: bytes) -> list[bytes]:
        cps = decode_for_split(data)
        text = "".join(chr(c) if c <= 0x10FFFF else "�" for c in cps)
        pieces, start = [], 0
        for m in _PATTERNS[self.qwen2].finditer(text):
            assert m.start() == start, "the patterns with their fallbacks match every position"
            pieces.append(b"".join(cpt_to_utf8(cps[j]) for j in range(m.start(), m.end())))
            start = m.end()
        return pieces

    def merge_piece(self, encoded: bytes) -> list[int]:
        symbols = lenient_code_points(encoded)
        while len(symbols) > 1:
            best, at = None, 0
            for i in range(len(symbols) - 1):
                r = self.rank.get((symbols[i], symbols[i + 1]))
                if r is not None and (best is None or r < best):
                    best, at = r, i
            if best is None:
                break
            symbols[at:at + 2] = [symbols[at] + symbols[at + 1]]
        ids = []
        for s in symbols:
            if s in self.token_to_id:
                ids.append(self.token_to_id[s])
                continue
            for cp in lenient_code_points(s):
                if cp in self.token_to_id:
                    ids.append(self.token_to_id[cp])
        return ids

    def encode(self, text: bytes | str, parse_special: bool = True) -> list[int]:
        data = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        ids: list[int] = []
        buf = bytearray()

        def flush():
            if buf:
                for piece in self.pre_tokenize(bytes(buf)):
                    ids.extend(self.merge_piece(b"".join(self.byte_map[b] for b in piece)))
                buf.clear()

        i = 0
        while i < len(data):
            match = None
            if parse_special:
                for s, sid in self.specials:
                    if data.startswith(s, i) and (match is None or len(s) > len(match[0])):
                        match = (s, sid)
            if match is not None:
                flush()
                ids.append(match[1])
                i += len(match[0])
            else:
                buf.append(data[i])
                i += 1
        flush()
        return ids

    def token_bytes(self, id: int) -> bytes:
        if id < 0 or id >= len(self.tokens):
            return b""
        out = bytearray()
        for piece in lenient_code_points(self.tokens[id]):
            b = self.cp_to_byte.get(lenient_value(piece))
            if b is not None:
                out.append(b)
        return bytes(out)

    def decode(self, ids) -> bytes:
        return b"".join(self.token_bytes(i) for i in ids)

    def is_special(self, id: int) -> bool:
        return 0 <= id < len(self.special) and self.special[id]
