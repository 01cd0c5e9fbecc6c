"""numpy-facing wrapper of liboracle.so — TEST INFRASTRUCTURE ONLY.

The CPU oracle the HIP kernels are checked against (see oracle.h for the reference file:line each
function restates). Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

vp = ctypes.c_void_p
u32 = ctypes.c_uint32
u64 = ctypes.c_uint64
i32 = ctypes.c_int32
f32 = ctypes.c_float

_SIGNATURES = {
    "oracle_half_to_float": (f32, [ctypes.c_uint16]),
    "oracle_float_to_half": (ctypes.c_uint16, [f32]),
    "oracle_halves_to_floats": (None, [vp, vp, u64]),
    "oracle_floats_to_halves": (None, [vp, vp, u64]),
    "oracle_mix64": (u64, [u64]),
    "oracle_fill_normal_f16": (None, [vp, u64, u64, ctypes.c_double, ctypes.c_double]),
    "oracle_fill_normal_f32": (None, [vp, u64, u64, ctypes.c_double, ctypes.c_double]),
    "oracle_fill_uniform_f32": (None, [vp, u64, u64]),
    "oracle_tensor_seed": (u64, [u64, u32, u32]),
    "oracle_set_threads": (ctypes.c_int, [ctypes.c_int]),
    "oracle_mat_vec_f16": (None, [vp, vp, vp, u32, u32, u64]),
    "oracle_mat_vec_f32": (None, [vp, vp, vp, u32, u32, u64]),
    "oracle_mat_vec_f16_f64acc": (None, [vp, vp, vp, u32, u32, u64]),
    "oracle_rms_norm": (None, [vp, vp, vp, u32, u32, f32]),
    "oracle_rms_norm_f16w": (None, [vp, vp, vp, u32, u32, f32]),
    "oracle_soft_max": (None, [vp, vp, u32, u32, f32]),
    "oracle_argmax": (i32, [vp, u32]),
    "oracle_argmax_rows": (None, [vp, vp, u32, u32]),
    "oracle_add": (None, [vp, vp, vp, u64]),
    "oracle_swiglu": (None, [vp, vp, vp, u64]),
    "oracle_rope_neox": (None, [vp, vp, u32, u32, u32, i32, f32]),
    "oracle_get_rows_f16": (None, [vp, i32, vp, u32]),
    "oracle_attention_f16kv": (None, [vp, vp, vp, vp, u32, u32, u32, u32, i32, f32]),
    "oracle_decode_step": (i32, [vp, i32, i32, vp, vp]),
    "oracle_decode_step_f32": (i32, [vp, i32, i32, vp]),
    "oracle_decode_layer": (None, [vp, u32, vp, i32, vp]),
    "oracle_sampler_new": (vp, [f32, i32, f32, f32, i32, u64]),
    "oracle_sampler_free": (None, [vp]),
    "oracle_sampler_sample": (i32, [vp, vp, i32, vp, u64]),
    "oracle_mt64_outputs": (None, [u64, u64, vp]),
    "oracle_mt64_uniform": (None, [u64, u64, vp]),
}

# Tensor kind numbers shared with the product's seeding (muyo_tensor_seed).
KIND = dict(
    TOKEN_EMBD=0, OUTPUT_NORM=1, ATTN_NORM=2, ATTN_QKV=3, ATTN_QKV_B=4, ATTN_OUTPUT=5, FFN_NORM=6,
    FFN_GATE=7, FFN_UP=8, FFN_DOWN=9, KCACHE=10, VCACHE=11, OUTPUT=13,
)

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> int:
    return int(load().oracle_set_threads(n))


def half_to_float(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    load().oracle_halves_to_floats(_p(bits), _p(out), bits.size)
    return out


def float_to_half(values: np.ndarray) -> np.ndarray:
    values = _f32(values)
    out = np.empty(values.shape, np.uint16)
    load().oracle_floats_to_halves(_p(values), _p(out), values.size)
    return out


def mix64(z: int) -> int:
    return int(load().oracle_mix64(z))


def normal_f16(count: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(count, np.uint16)
    load().oracle_fill_normal_f16(_p(out), count, seed, mean, std)
    return out


def normal_f32(count: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(count, np.float32)
    load().oracle_fill_normal_f32(_p(out), count, seed, mean, std)
    return out


def uniform_f32(count: int, seed: int) -> np.ndarray:
    out = np.empty(count, np.float32)
    load().oracle_fill_uniform_f32(_p(out), count, seed)
    return out


def tensor_seed(seed: int, kind: str, layer: int) -> int:
    return int(load().oracle_tensor_seed(seed, KIND[kind], layer))


def mat_vec_f16(w_bits: np.ndarray, x: np.ndarray, f64acc: bool = False) -> np.ndarray:
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    rows, cols = w_bits.shape
    x = _f32(x)
    y = np.empty(rows, np.float32)
    fn = load().oracle_mat_vec_f16_f64acc if f64acc else load().oracle_mat_vec_f16
    fn(_p(w_bits), _p(x), _p(y), rows, cols, cols)
    return y


def mat_vec_f32(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = _f32(w)
    rows, cols = w.shape
    x = _f32(x)
    y = np.empty(rows, np.float32)
    load().oracle_mat_vec_f32(_p(w), _p(x), _p(y), rows, cols, cols)
    return y


def rms_norm(x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
    x = _f32(x)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    y = np.empty_like(x)
    if w is None:
        load().oracle_rms_norm(_p(x), None, _p(y), rows, cols, eps)
    elif np.asarray(w).dtype == np.uint16:
        w = np.ascontiguousarray(w, dtype=np.uint16)
        load().oracle_rms_norm_f16w(_p(x), _p(w), _p(y), rows, cols, eps)
    else:
        w = _f32(w)
        load().oracle_rms_norm(_p(x), _p(w), _p(y), rows, cols, eps)
    return y


def soft_max(x: np.ndarray, scale: float) -> np.ndarray:
    x = _f32(x)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    y = np.empty_like(x)
    load().oracle_soft_max(_p(x), _p(y), rows, cols, scale)
    return y


def argmax(x: np.ndarray) -> int:
    x = _f32(x)
    return int(load().oracle_argmax(_p(x), x.size))


def argmax_rows(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    rows, cols = x.shape
    out = np.empty(rows, np.int32)
    load().oracle_argmax_rows(_p(x), _p(out), rows, cols)
    return out


def add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    d = np.empty_like(a)
    load().oracle_add(_p(a), _p(b), _p(d), a.size)
    return d


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g, u = _f32(g), _f32(u)
    d = np.empty_like(g)
    load().oracle_swiglu(_p(g), _p(u), _p(d), g.size)
    return d


def rope_neox(x: np.ndarray, pos: int, theta_scale: float, n_dims: int | None = None) -> np.ndarray:
    """x: [rows][head_dim] f32."""
    x = _f32(x)
    rows, head_dim = x.shape
    y = np.empty_like(x)
    load().oracle_rope_neox(_p(x), _p(y), rows, head_dim, n_dims or head_dim, pos, theta_scale)
    return y


def get_rows_f16(table_bits: np.ndarray, index: int) -> np.ndarray:
    table_bits = np.ascontiguousarray(table_bits, dtype=np.uint16)
    dim = table_bits.shape[1]
    d = np.empty(dim, np.float32)
    load().oracle_get_rows_f16(_p(table_bits), index, _p(d), dim)
    return d


def attention_f16kv(q, kcache_bits, vcache_bits, heads, kv_heads, head_dim, max_seq, pos, scale):
    q = _f32(q)
    kc = np.ascontiguousarray(kcache_bits, dtype=np.uint16)
    vc = np.ascontiguousarray(vcache_bits, dtype=np.uint16)
    out = np.empty(heads * head_dim, np.float32)
    load().oracle_attention_f16kv(_p(q), _p(kc), _p(vc), _p(out), heads, kv_heads, head_dim, max_seq, pos, scale)
    return out


class Sampler:
    """The reference's host sampler (src/Sampler.cpp:10-100) restated in sampler.cpp: penalty over
    the last-N history, temperature, top-k, top-p and one std::mt19937_64 draw per sampled token.
    `ref=True` drives the reference's own Sampler.cpp instead, compiled into _ref/ (present only
    where the reference tree was, when the oracle was built)."""

    REF_PATH = HERE / "_ref" / "libref_sampler.so"

    def __init__(self, temperature=0.0, top_k=40, top_p=0.95, repeat_penalty=1.0, repeat_last_n=64, seed=0,
                 ref=False):
        if ref:
            lib = ctypes.CDLL(str(self.REF_PATH))
            self._new, self._free, self._sample = lib.ref_sampler_new, lib.ref_sampler_free, lib.ref_sampler_sample
            self._new.restype, self._new.argtypes = vp, [f32, i32, f32, f32, i32, u64]
            self._free.restype, self._free.argtypes = None, [vp]
            self._sample.restype, self._sample.argtypes = i32, [vp, vp, i32, vp, u64]
        else:
            lib = load()
            self._new, self._free, self._sample = lib.oracle_sampler_new, lib.oracle_sampler_free, lib.oracle_sampler_sample
        self._h = self._new(temperature, top_k, top_p, repeat_penalty, repeat_last_n, seed)

    def sample(self, logits: np.ndarray, history) -> int:
        """Samples from `logits` (modified in place, as the reference does)."""
        assert logits.dtype == np.float32 and logits.flags["C_CONTIGUOUS"]
        hist = np.ascontiguousarray(history, dtype=np.int32)
        return int(self._sample(self._h, _p(logits), logits.size, _p(hist) if hist.size else None, hist.size))

    def __del__(self):
        if getattr(self, "_h", None):
            self._free(self._h)
            self._h = None


def mt64_outputs(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    load().oracle_mt64_outputs(seed, n, _p(out))
    return out


def mt64_uniform(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float64)
    load().oracle_mt64_uniform(seed, n, _p(out))
    return out


class _OracleQwen2(ctypes.Structure):
    _fields_ = [
        ("layers", u32), ("hidden", u32), ("ffn", u32), ("heads", u32), ("kv_heads", u32), ("head_dim", u32),
        ("vocab", u32), ("max_seq", u32), ("rms_eps", f32), ("rope_base", f32),
        ("token_embd", vp), ("output_norm", vp),
        ("attn_norm", vp), ("attn_qkv", vp), ("attn_qkv_b", vp), ("attn_out", vp), ("ffn_norm", vp),
        ("ffn_gate", vp), ("ffn_up", vp), ("ffn_down", vp), ("kcache", vp), ("vcache", vp), ("output", vp),
    ]


class Model:
    """A Qwen2-shaped model in host memory with the product decoder's tensor layout.

    Weights are drawn from the same portable generator and tensor seeds as
    muyo_decoder_fill_random, so both sides hold identical bits.
    """

    PER_LAYER = ("ATTN_NORM", "ATTN_QKV", "ATTN_QKV_B", "ATTN_OUTPUT", "FFN_NORM", "FFN_GATE", "FFN_UP",
                 "FFN_DOWN", "KCACHE", "VCACHE")

    def __init__(self, layers, hidden, ffn, heads, kv_heads, head_dim, vocab, max_seq, eps=1e-6, rope_base=1e6,
                 untied_output=False):
        self.layers, self.hidden, self.ffn = layers, hidden, ffn
        self.heads, self.kv_heads, self.head_dim = heads, kv_heads, head_dim
        self.vocab, self.max_seq, self.eps, self.rope_base = vocab, max_seq, eps, rope_base
        qkv_rows = (heads + 2 * kv_heads) * head_dim
        qdim = heads * head_dim
        self.shapes = {
            "TOKEN_EMBD": ((vocab, hidden), np.uint16), "OUTPUT_NORM": ((hidden,), np.float32),
            "ATTN_NORM": ((hidden,), np.float32), "ATTN_QKV": ((qkv_rows, hidden), np.uint16),
            "ATTN_QKV_B": ((qkv_rows,), np.float32), "ATTN_OUTPUT": ((hidden, qdim), np.uint16),
            "FFN_NORM": ((hidden,), np.float32), "FFN_GATE": ((ffn, hidden), np.uint16),
            "FFN_UP": ((ffn, hidden), np.uint16), "FFN_DOWN": ((hidden, ffn), np.uint16),
            "KCACHE": ((kv_heads, max_seq, head_dim), np.uint16), "VCACHE": ((kv_heads, max_seq, head_dim), np.uint16),
            "OUTPUT": ((vocab, hidden), np.uint16),
        }
        self.untied_output = untied_output
        self.t = {}
        for name in ("TOKEN_EMBD", "OUTPUT_NORM") + (("OUTPUT",) if untied_output else ()):
            shape, dt = self.shapes[name]
            self.t[(name, 0)] = np.zeros(shape, dt)
        for layer in range(layers):
            for name in self.PER_LAYER:
                shape, dt = self.shapes[name]
                self.t[(name, layer)] = np.zeros(shape, dt)
        self._struct = None

    # Same distributions as muyo_decoder_fill_random.
    DISTRIBUTION = {
        "TOKEN_EMBD": (0.0, 0.02), "OUTPUT_NORM": (1.0, 0.1), "ATTN_NORM": (1.0, 0.1), "ATTN_QKV": (0.0, 0.02),
        "ATTN_QKV_B": (0.0, 0.02), "ATTN_OUTPUT": (0.0, 0.02), "FFN_NORM": (1.0, 0.1), "FFN_GATE": (0.0, 0.02),
        "FFN_UP": (0.0, 0.02), "FFN_DOWN": (0.0, 0.02), "OUTPUT": (0.0, 0.02),
    }

    def fill_random(self, seed: int) -> None:
        for (name, layer), arr in self.t.items():
            if name in ("KCACHE", "VCACHE"):
                arr[...] = 0
                continue
            mean, std = self.DISTRIBUTION[name]
            s = tensor_seed(seed, name, layer)
            if arr.dtype == np.uint16:
                arr[...] = normal_f16(arr.size, s, mean, std).reshape(arr.shape)
            else:
                arr[...] = normal_f32(arr.size, s, mean, std).reshape(arr.shape)

    def fill_kv_random(self, positions: int, seed: int) -> None:
        for layer in range(self.layers):
            for name in ("KCACHE", "VCACHE"):
                arr = self.t[(name, layer)]
                arr[...] = normal_f16(arr.size, tensor_seed(seed, name, layer), 0.0, 1.0).reshape(arr.shape)
                arr[:, positions:, :] = 0

    def _build_struct(self):
        m = _OracleQwen2()
        m.layers, m.hidden, m.ffn, m.heads, m.kv_heads = self.layers, self.hidden, self.ffn, self.heads, self.kv_heads
        m.head_dim, m.vocab, m.max_seq, m.rms_eps, m.rope_base = (
            self.head_dim, self.vocab, self.max_seq, self.eps, self.rope_base)
        m.token_embd = _p(self.t[("TOKEN_EMBD", 0)])
        m.output_norm = _p(self.t[("OUTPUT_NORM", 0)])
        m.output = _p(self.t[("OUTPUT", 0)]) if self.untied_output else None
        keep = []
        fields = dict(attn_norm="ATTN_NORM", attn_qkv="ATTN_QKV", attn_qkv_b="ATTN_QKV_B", attn_out="ATTN_OUTPUT",
                      ffn_norm="FFN_NORM", ffn_gate="FFN_GATE", ffn_up="FFN_UP", ffn_down="FFN_DOWN",
                      kcache="KCACHE", vcache="VCACHE")
        for field, name in fields.items():
            arr = (vp * self.layers)(*[_p(self.t[(name, layer)]) for layer in range(self.layers)])
            keep.append(arr)
            setattr(m, field, ctypes.cast(arr, vp))
        self._struct = (m, keep)
        return m

    def step(self, token: int, pos: int) -> tuple[int, np.ndarray, tuple[float, float]]:
        m = self._struct[0] if self._struct else self._build_struct()
        logits = np.empty(self.vocab, np.float32)
        top2 = np.empty(2, np.float32)
        best = load().oracle_decode_step(ctypes.byref(m), token, pos, _p(logits), _p(top2))
        if best < 0:
            raise ValueError("oracle_decode_step rejected its arguments")
        return best, logits, (float(top2[0]), float(top2[1]))

    def step_f32(self, token: int, pos: int) -> tuple[int, np.ndarray]:
        """The reference's CPU path (f32 running sums in index order): the timed CPU baseline."""
        m = self._struct[0] if self._struct else self._build_struct()
        logits = np.empty(self.vocab, np.float32)
        best = load().oracle_decode_step_f32(ctypes.byref(m), token, pos, _p(logits))
        if best < 0:
            raise ValueError("oracle_decode_step_f32 rejected its arguments")
        return best, logits

    def layer(self, layer: int, x: np.ndarray, pos: int) -> np.ndarray:
        m = self._struct[0] if self._struct else self._build_struct()
        x = _f32(x)
        out = np.empty(self.hidden, np.float32)
        load().oracle_decode_layer(ctypes.byref(m), layer, _p(x), pos, _p(out))
        return out

    def greedy(self, token: int, pos: int, count: int):
        ids, margins = [], []
        for i in range(count):
            best, _, (top1, top2) = self.step(token, pos + i)
            ids.append(best)
            margins.append(top1 - top2)
            token = best
        return ids, margins
