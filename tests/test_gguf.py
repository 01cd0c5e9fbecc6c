"""The GGUF reader (muyo_gguf_*, csrc/gguf.cpp) against the reference's own GgufReader, compiled
from src/Gguf.cpp into oracle/_ref, on files tests/gguf_writer.py writes. No GPU: parsing and the
Qwen2 configuration are host work.

Pins: every tensor-table field, the data offset (alignment from general.alignment, 32 without
one or when it is not a scalar), each typed lookup with its conversion and fallback on every
value type, string arrays element by element, tensor bytes, the refusals (bad magic, truncation,
quantised data, data past the end), and the Qwen2 configuration as src/FullModel.cpp:85-108
reads it. Skipped where the reference tree was absent when the oracle was built.
"""
import ctypes
import os

import numpy as np
import pytest

import gguf_writer as gw
import oracle

REF_PATH = oracle.HERE / "_ref" / "libref_gguf.so"
needs_ref = pytest.mark.skipif(not REF_PATH.exists(), reason="oracle/_ref/libref_gguf.so was not built")


class RefGguf:
    def __init__(self, path):
        lib = ctypes.CDLL(str(REF_PATH))
        c, vp, u64, u32 = ctypes.c_char_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32
        sig = {
            "ref_gguf_open": (vp, [c]), "ref_gguf_close": (None, [vp]), "ref_gguf_version": (u32, [vp]),
            "ref_gguf_data_offset": (u64, [vp]), "ref_gguf_tensor_count": (u64, [vp]),
            "ref_gguf_tensor_name": (c, [vp, u64]), "ref_gguf_tensor_type": (u32, [vp, u64]),
            "ref_gguf_tensor_ndims": (u32, [vp, u64]), "ref_gguf_tensor_dim": (u64, [vp, u64, u32]),
            "ref_gguf_tensor_offset": (u64, [vp, u64]), "ref_gguf_has": (ctypes.c_int, [vp, c]),
            "ref_gguf_uint_or": (u64, [vp, c, u64]), "ref_gguf_float_or": (ctypes.c_double, [vp, c, ctypes.c_double]),
            "ref_gguf_string_or": (c, [vp, c, c]), "ref_gguf_string_array_size": (u64, [vp, c]),
            "ref_gguf_string_array_at": (c, [vp, c, u64]),
            "ref_gguf_read_tensor": (ctypes.c_int64, [vp, c, vp, u64]),
        }
        for name, (res, args) in sig.items():
            getattr(lib, name).restype, getattr(lib, name).argtypes = res, args
        self.lib = lib
        self.h = lib.ref_gguf_open(os.fsencode(path))

    def tensors(self):
        L, h = self.lib, self.h
        return [(L.ref_gguf_tensor_name(h, i).decode(), L.ref_gguf_tensor_type(h, i),
                 [L.ref_gguf_tensor_dim(h, i, d) for d in range(L.ref_gguf_tensor_ndims(h, i))],
                 L.ref_gguf_tensor_offset(h, i)) for i in range(L.ref_gguf_tensor_count(h))]

    def tensor_bytes(self, name):
        n = self.lib.ref_gguf_read_tensor(self.h, name.encode(), None, 0)
        if n < 0:
            return None
        buf = ctypes.create_string_buffer(max(n, 1))
        self.lib.ref_gguf_read_tensor(self.h, name.encode(), buf, n)
        return buf.raw[:n]

    def close(self):
        if self.h:
            self.lib.ref_gguf_close(self.h)
            self.h = None


SCALARS = [
    ("u8", gw.U8, 200), ("i8", gw.I8, -7), ("u16", gw.U16, 65000), ("i16", gw.I16, -30000),
    ("u32", gw.U32, 4000000000), ("i32", gw.I32, -5), ("f32", gw.F32, 3.25), ("bool_t", gw.BOOL, True),
    ("bool_f", gw.BOOL, False), ("u64", gw.U64, 2**63 + 5), ("i64", gw.I64, -(2**40)), ("f64", gw.F64, 1e-6),
    ("str", gw.STRING, "héllo"), ("empty_str", gw.STRING, ""),
]
ARRAYS = [
    ("a_u8", gw.U8, [1, 2, 255]), ("a_i8", gw.I8, [-1, 5]), ("a_u16", gw.U16, [9]), ("a_i16", gw.I16, [-2, 2]),
    ("a_u32", gw.U32, [7, 8]), ("a_i32", gw.I32, [-9]), ("a_f32", gw.F32, [0.5, -1.5]), ("a_bool", gw.BOOL, [1, 0, 1]),
    ("a_u64", gw.U64, [2**40]), ("a_i64", gw.I64, [-3]), ("a_f64", gw.F64, [2.5]), ("a_empty", gw.F32, []),
    ("a_str", gw.STRING, ["alpha", "", "γδ"]), ("a_str_empty", gw.STRING, []),
]


def diverse_file(path, alignment=64, alignment_kind=gw.U32):
    meta = [("general.architecture", gw.STRING, "qwen2")] + SCALARS
    meta += [(k, gw.ARRAY, (t, v)) for k, t, v in ARRAYS]
    if alignment_kind is not None:
        meta.append(("general.alignment", alignment_kind, alignment if alignment_kind != gw.STRING else "64"))
    rng = np.random.default_rng(1)
    tensors = [
        ("w16", gw.GGML_F16, [8, 3], rng.integers(0, 2**16, 24, dtype=np.uint16).tobytes()),
        ("w32", gw.GGML_F32, [5], rng.standard_normal(5).astype(np.float32).tobytes()),
        ("q8", 8, [32, 2], bytes(68)),  # Q8_0: two blocks of 34 bytes
        ("w3d", gw.GGML_F32, [2, 3, 4], rng.standard_normal(24).astype(np.float32).tobytes()),
    ]
    real = alignment if alignment_kind in (gw.U32,) else 32
    gw.write(path, meta, tensors, alignment=real)
    return meta, tensors


def compare(mh, path, keys):
    ref = RefGguf(path)
    assert ref.h, ref.lib.ref_gguf_last_error() if hasattr(ref.lib, "ref_gguf_last_error") else "reference failed"
    try:
        with mh.Gguf(path) as ours:
            assert ours.version == ref.lib.ref_gguf_version(ref.h)
            assert ours.data_offset == ref.lib.ref_gguf_data_offset(ref.h)
            assert ours.tensors() == ref.tensors()
            L, h = ref.lib, ref.h
            for key in keys + ["missing.key"]:
                k = key.encode()
                assert bool(mh.load().muyo_gguf_has(ours.handle, k)) == bool(L.ref_gguf_has(h, k)), key
                assert ours.uint_or(key, 12345) == L.ref_gguf_uint_or(h, k, 12345), key
                ours_f, ref_f = ours.float_or(key, 0.25), L.ref_gguf_float_or(h, k, 0.25)
                assert ours_f == ref_f or (np.isnan(ours_f) and np.isnan(ref_f)), key
                assert ours.string_or(key, "fb") == L.ref_gguf_string_or(h, k, b"fb").decode(), key
                n = ours.string_array_size(key)
                assert n == L.ref_gguf_string_array_size(h, k), key
                for i in range(n + 1):
                    got = ours.string_array_at(key, i)
                    want = L.ref_gguf_string_array_at(h, k, i)
                    assert got == (None if want is None else want.decode()), (key, i)
            for name, *_ in ours.tensors():
                want = ref.tensor_bytes(name)
                if want is None:
                    with pytest.raises(mh.MuyoError):
                        ours.tensor_bytes(name)
                else:
                    assert ours.tensor_bytes(name) == want, name
    finally:
        ref.close()


@needs_ref
@pytest.mark.parametrize("alignment,kind", [(64, gw.U32), (32, None), (32, gw.STRING), (128, gw.U32)])
def test_reader_matches_reference_reader(tmp_path, mh, alignment, kind):
    path = tmp_path / "diverse.gguf"
    meta, _ = diverse_file(path, alignment, kind)
    keys = [k for k, _, _ in meta]
    # A negative float cast to an unsigned integer is undefined behaviour in C++: keep such keys
    # (none here have one) out of the unsigned lookup.
    compare(mh, path, keys)


@needs_ref
@pytest.mark.parametrize("untied", [False, True])
def test_qwen2_file_and_configuration(tmp_path, mh, untied):
    model = oracle.Model(layers=2, hidden=128, ffn=256, heads=2, kv_heads=1, head_dim=64, vocab=300, max_seq=64,
                         untied_output=untied)
    model.fill_random(4)
    path = tmp_path / "qwen2.gguf"
    gw.qwen2_file(path, model)
    keys = ["qwen2.block_count", "qwen2.embedding_length", "qwen2.feed_forward_length", "qwen2.attention.head_count",
            "qwen2.attention.head_count_kv", "qwen2.attention.layer_norm_rms_epsilon", "qwen2.rope.freq_base",
            "tokenizer.ggml.tokens", "tokenizer.ggml.eos_token_id"]
    compare(mh, path, keys)
    with mh.Gguf(path) as g:
        c = g.qwen2_config(2048)
    # src/FullModel.cpp:85-108, restated with the reference reader's lookups.
    ref = RefGguf(path)
    L, h = ref.lib, ref.h
    want = dict(layers=L.ref_gguf_uint_or(h, b"qwen2.block_count", 0),
                hidden=L.ref_gguf_uint_or(h, b"qwen2.embedding_length", 0),
                feedForward=L.ref_gguf_uint_or(h, b"qwen2.feed_forward_length", 0),
                heads=L.ref_gguf_uint_or(h, b"qwen2.attention.head_count", 0),
                kvHeads=L.ref_gguf_uint_or(h, b"qwen2.attention.head_count_kv", 0),
                vocab=L.ref_gguf_string_array_size(h, b"tokenizer.ggml.tokens"))
    eps = np.float32(L.ref_gguf_float_or(h, b"qwen2.attention.layer_norm_rms_epsilon", 0.0))
    base = np.float32(L.ref_gguf_float_or(h, b"qwen2.rope.freq_base", 10000.0))
    ref.close()
    for field, value in want.items():
        assert getattr(c, field) == value, field
    assert c.headDim == want["hidden"] // want["heads"] and c.maxSeq == 2048
    assert np.float32(c.rmsEps) == eps and np.float32(c.ropeBase) == base
    assert c.untiedOutput == int(untied)


def test_refusals(tmp_path, mh):
    path = tmp_path / "x.gguf"
    meta, tensors = diverse_file(path)
    good = path.read_bytes()
    # Bad magic.
    path.write_bytes(b"GGUG" + good[4:])
    with pytest.raises(mh.MuyoError) as e:
        mh.Gguf(path)
    assert e.value.status == mh.MUYO_E_CONTRACT
    # Truncated anywhere in the header or tables.
    for cut in (3, 10, 30, 200, 600, len(good) // 3):
        path.write_bytes(good[:cut])
        with pytest.raises(mh.MuyoError):
            mh.Gguf(path)
    # Tensor data past the end of the file: the table parses, the bytes are refused.
    path.write_bytes(good[:-8])
    with mh.Gguf(path) as g:
        with pytest.raises(mh.MuyoError) as e:
            g.tensor_bytes("w3d")
        assert e.value.status == mh.MUYO_E_RANGE
        assert len(g.tensor_bytes("w16")) == 48
        with pytest.raises(mh.MuyoError) as e:
            g.tensor_bytes("q8")
        assert e.value.status == mh.MUYO_E_UNSUPPORTED
    # A missing file.
    with pytest.raises(mh.MuyoError):
        mh.Gguf(tmp_path / "absent.gguf")


def _exercise(g, keys):
    """Every read the reader offers on an opened file; refusals are fine, crashes are not."""
    try:
        tensors = g.tensors()
    except UnicodeDecodeError:  # a corrupted name; the table itself was read
        tensors = []
    for name, _, _, _ in tensors:
        try:
            g.tensor_bytes(name)
        except Exception as e:  # noqa: BLE001 - any MuyoError is an answer
            assert e.__class__.__name__ == "MuyoError", e
    for key in keys:
        g.uint_or(key, 7)
        g.float_or(key, 0.5)
        n = g.string_array_size(key)
        # Strings come back as the file's bytes; a corrupted one need not be UTF-8.
        for read in [lambda: g.string_or(key, "x")] + [lambda i=i: g.string_array_at(key, i) for i in range(min(n, 4))]:
            try:
                read()
            except UnicodeDecodeError:
                pass
        g.string_array_at(key, n)


def test_every_truncation_and_seeded_corruptions(tmp_path, mh):
    """Every prefix of the header and tables, and 400 seeded corruptions of 1-4 bytes among them:
    each file is refused with an error or opens and answers every read; none may read out of
    bounds (tests/test_sanitized_host.py runs this under AddressSanitizer and UBSan)."""
    import random

    path = tmp_path / "x.gguf"
    meta, _ = diverse_file(path)
    good = path.read_bytes()
    keys = [k for k, _, _ in meta] + ["missing.key"]
    with mh.Gguf(path) as g:
        data_offset = g.data_offset
    for cut in range(data_offset):
        path.write_bytes(good[:cut])
        try:
            with mh.Gguf(path) as g:
                assert cut >= data_offset - 64, f"a file cut at {cut} of {data_offset} header bytes opened"
                _exercise(g, keys)
        except mh.MuyoError:
            pass
    rng = random.Random(2026)
    for _ in range(400):
        b = bytearray(good)
        for _ in range(rng.randint(1, 4)):
            b[rng.randrange(data_offset)] = rng.randrange(256)
        path.write_bytes(bytes(b))
        try:
            with mh.Gguf(path) as g:
                _exercise(g, keys)
        except mh.MuyoError:
            pass
