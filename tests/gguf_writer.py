"""Writes synthetic GGUF files for the loader's tests — TEST INFRASTRUCTURE ONLY.

The layout is the one the reference's GgufReader reads (src/Gguf.cpp:155-219): magic "GGUF",
version, tensor count and metadata count; each metadata entry as a string key, a type word and a
value (strings and arrays length-prefixed with u64); each tensor entry as name, dimension count,
dimensions (fastest-varying first), ggml type and offset into the data section; the data section
starting at the header's end rounded up to the alignment, each tensor's offset aligned too.
"""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
GGML_F32, GGML_F16 = 0, 1
_PACK = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
         I64: "<q", F64: "<d"}


def _string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(kind: int, value) -> bytes:
    if kind == STRING:
        return _string(value)
    if kind == ARRAY:
        element, items = value
        head = struct.pack("<IQ", element, len(items))
        if element == STRING:
            return head + b"".join(_string(x) for x in items)
        return head + b"".join(struct.pack(_PACK[element], int(x) if element == BOOL else x) for x in items)
    return struct.pack(_PACK[kind], int(value) if kind == BOOL else value)


def write(path, metadata, tensors, version: int = 3, alignment: int = 32) -> int:
    """metadata: [(key, type, value)], arrays as (element type, items); tensors: [(name, ggml type,
    dims fastest-first, bytes)]. `alignment` must be what the file's general.alignment says (32 when
    it has none). Returns the data section's offset."""
    header = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(metadata))
    for key, kind, value in metadata:
        header += _string(key) + struct.pack("<I", kind) + _value(kind, value)
    offsets, cursor = [], 0
    for _, _, _, data in tensors:
        cursor = (cursor + alignment - 1) // alignment * alignment
        offsets.append(cursor)
        cursor += len(data)
    for (name, ggml_type, dims, _), offset in zip(tensors, offsets):
        header += _string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        header += struct.pack("<IQ", ggml_type, offset)
    start = (len(header) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(header + b"\0" * (start - len(header)))
        at = 0
        for (_, _, _, data), offset in zip(tensors, offsets):
            f.write(b"\0" * (offset - at) + data)
            at = offset + len(data)
    return start


def tokenizer_metadata(vocab: dict, pre: str = "qwen2", bos: int | None = None, eos: int | None = None) -> list:
    """tokenizer.ggml.* entries for a vocabulary dict with "tokens", "merges" and "token_type" (as in
    tests/golden/bpe_vocab.json)."""
    meta = [("tokenizer.ggml.model", STRING, "gpt2"),
            ("tokenizer.ggml.pre", STRING, pre),
            ("tokenizer.ggml.tokens", ARRAY, (STRING, vocab["tokens"])),
            ("tokenizer.ggml.token_type", ARRAY, (I32, vocab["token_type"])),
            ("tokenizer.ggml.merges", ARRAY, (STRING, vocab["merges"]))]
    if bos is not None:
        meta.append(("tokenizer.ggml.bos_token_id", U32, bos))
    if eos is not None:
        meta.append(("tokenizer.ggml.eos_token_id", U32, eos))
    return meta


def tokenizer_file(path, vocab: dict, pre: str = "qwen2") -> None:
    """A GGUF holding only a tokenizer's metadata."""
    write(path, tokenizer_metadata(vocab, pre), [])


def qwen2_file(path, model, alignment: int = 32, order: str = "reference", vocab: dict | None = None) -> None:
    """An oracle.Model's weights as a Qwen2 GGUF (the names of src/FullModel.cpp:582-600): q, k and
    v split back out of the stacked QKV tensor, output.weight when the model is untied. With
    `vocab` (len(vocab["tokens"]) == the model's vocab) the file carries that tokenizer, with
    <|endoftext|> as BOS and <|im_end|> as EOS, instead of placeholder token strings."""
    m = model
    qdim, kvdim = m.heads * m.head_dim, m.kv_heads * m.head_dim
    meta = [
        ("general.architecture", STRING, "qwen2"),
        ("qwen2.block_count", U32, m.layers),
        ("qwen2.embedding_length", U32, m.hidden),
        ("qwen2.feed_forward_length", U32, m.ffn),
        ("qwen2.attention.head_count", U32, m.heads),
        ("qwen2.attention.head_count_kv", U32, m.kv_heads),
        ("qwen2.attention.layer_norm_rms_epsilon", F32, m.eps),
        ("qwen2.rope.freq_base", F32, m.rope_base),
    ]
    if vocab is None:
        meta += [("tokenizer.ggml.tokens", ARRAY, (STRING, [f"t{i}" for i in range(m.vocab)])),
                 ("tokenizer.ggml.bos_token_id", U32, 1),
                 ("tokenizer.ggml.eos_token_id", U32, 2)]
    else:
        assert len(vocab["tokens"]) == m.vocab, (len(vocab["tokens"]), m.vocab)
        meta += tokenizer_metadata(vocab, "qwen2", bos=vocab["tokens"].index("<|endoftext|>"),
                                   eos=vocab["tokens"].index("<|im_end|>"))
    if alignment != 32:
        meta.append(("general.alignment", U32, alignment))
    t = m.t
    tensors = [("token_embd.weight", GGML_F16, [m.hidden, m.vocab], t[("TOKEN_EMBD", 0)].tobytes()),
               ("output_norm.weight", GGML_F32, [m.hidden], t[("OUTPUT_NORM", 0)].tobytes())]
    if m.untied_output:
        tensors.append(("output.weight", GGML_F16, [m.hidden, m.vocab], t[("OUTPUT", 0)].tobytes()))
    for layer in range(m.layers):
        p = f"blk.{layer}."
        qkv, bias = t[("ATTN_QKV", layer)], t[("ATTN_QKV_B", layer)]
        tensors += [
            (p + "attn_norm.weight", GGML_F32, [m.hidden], t[("ATTN_NORM", layer)].tobytes()),
            (p + "attn_q.weight", GGML_F16, [m.hidden, qdim], qkv[:qdim].tobytes()),
            (p + "attn_q.bias", GGML_F32, [qdim], bias[:qdim].tobytes()),
            (p + "attn_k.weight", GGML_F16, [m.hidden, kvdim], qkv[qdim:qdim + kvdim].tobytes()),
            (p + "attn_k.bias", GGML_F32, [kvdim], bias[qdim:qdim + kvdim].tobytes()),
            (p + "attn_v.weight", GGML_F16, [m.hidden, kvdim], qkv[qdim + kvdim:].tobytes()),
            (p + "attn_v.bias", GGML_F32, [kvdim], bias[qdim + kvdim:].tobytes()),
            (p + "attn_output.weight", GGML_F16, [qdim, m.hidden], t[("ATTN_OUTPUT", layer)].tobytes()),
            (p + "ffn_norm.weight", GGML_F32, [m.hidden], t[("FFN_NORM", layer)].tobytes()),
            (p + "ffn_gate.weight", GGML_F16, [m.hidden, m.ffn], t[("FFN_GATE", layer)].tobytes()),
            (p + "ffn_up.weight", GGML_F16, [m.hidden, m.ffn], t[("FFN_UP", layer)].tobytes()),
            (p + "ffn_down.weight", GGML_F16, [m.ffn, m.hidden], t[("FFN_DOWN", layer)].tobytes()),
        ]
    if order == "reversed":
        tensors = tensors[::-1]
    write(path, meta, tensors, alignment=alignment)
