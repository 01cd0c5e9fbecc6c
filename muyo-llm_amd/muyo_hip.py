"""ctypes binding of libmuyo_hip.so (the C ABI declared in include/muyo_hip.h).

Device pointers are plain integers (e.g. a torch tensor's ``data_ptr()``); ``stream`` is a
``hipStream_t`` as an integer (``torch.cuda.current_stream().cuda_stream``) or 0 for the default
stream. There is no fallback: if the shared library is missing, ``load()`` raises.

The ``*_push_constants`` helpers fill the contract blocks the way the reference's graph nodes do
(src/FullModel.cpp:133-485, src/MatVec.cpp:136-159, src/Swiglu.cpp:118-150,
src/KvCache.cpp:181-226), so callers and tests build the same bytes the reference would push.
"""
from __future__ import annotations

import ctypes
import math
import os
import pathlib
import struct

HERE = pathlib.Path(__file__).resolve().parent
# MUYO_HIP_LIBRARY names another build of the same library (the sanitizer build, for instance).
LIB_PATH = pathlib.Path(os.environ.get("MUYO_HIP_LIBRARY") or HERE / "libmuyo_hip.so")

u32 = ctypes.c_uint32
i32 = ctypes.c_int32
f32 = ctypes.c_float
vp = ctypes.c_void_p
u64 = ctypes.c_uint64


class LlamaAddPushConstants(ctypes.Structure):
    _fields_ = (
        [("ne", u32)]
        + [(n, u32) for n in ("ne00", "ne01", "ne02", "ne03", "nb00", "nb01", "nb02", "nb03")]
        + [(n, u32) for n in ("ne10", "ne11", "ne12", "ne13", "nb10", "nb11", "nb12", "nb13")]
        + [(n, u32) for n in ("ne20", "ne21", "ne22", "ne23", "nb20", "nb21", "nb22", "nb23")]
        + [("misalignOffsets", u32), ("param1", f32), ("param2", f32), ("param3", i32)]
    )


class LlamaMatVecPushConstants(ctypes.Structure):
    _fields_ = [
        (n, u32)
        for n in (
            "ncols", "strideA", "strideB", "strideD", "batchStrideA", "batchStrideB", "batchStrideD",
            "fusionFlags", "baseWorkGroupY", "ne02", "ne12", "broadcast2", "broadcast3",
        )
    ]


class LlamaRopePushConstants(ctypes.Structure):
    _fields_ = [
        ("ropeMode", u32), ("nrows", u32), ("nDims", u32), ("nOffs", u32),
        ("freqScale", f32), ("freqBase", f32), ("extFactor", f32), ("attnFactor", f32),
        ("corrDims", f32 * 2), ("thetaScale", f32), ("hasFf", u32), ("sections", i32 * 4),
        ("isImrope", u32), ("isBack", u32), ("setRowsStride", u32),
        ("ne00", u32), ("ne01", u32), ("ne02", u32), ("nb01", u32), ("nb02", u32), ("nb03", u32),
        ("nb11", u32), ("nb12", u32), ("nb13", u32), ("aOffset", u32), ("dOffset", u32),
    ]


class LlamaGluPushConstants(ctypes.Structure):
    _fields_ = (
        [("N", u32), ("ne00", u32), ("ne20", u32), ("mode", u32), ("alpha", f32), ("limit", f32)]
        + [(n, u32) for n in ("nb00", "nb01", "nb02", "nb03", "nb10", "nb11", "nb12", "nb13",
                               "nb20", "nb21", "nb22", "nb23", "ne21", "ne22", "misalignOffsets",
                               "ne2_012mp", "ne2_012L", "ne2_01mp", "ne2_01L", "ne2_0mp", "ne2_0L")]
    )


class LlamaGenericHeadPushConstants(ctypes.Structure):
    _fields_ = [("KX", u32), ("KY", u32), ("param1", f32), ("param2", f32), ("param3", f32), ("param4", f32)]


class LlamaSoftMaxPushConstants(ctypes.Structure):
    _fields_ = (
        [(n, u32) for n in ("KX", "KY", "ne00", "ne01", "ne02", "ne12", "ne13", "nb11", "nb12", "nb13")]
        + [("scale", f32), ("maxBias", f32), ("m0", f32), ("m1", f32)]
        + [("nHeadLog2", u32), ("nrowsX", u32), ("hasSinks", u32)]
    )


class LlamaCopyPushConstants(ctypes.Structure):
    _fields_ = (
        [("ne", u32)]
        + [(n, u32) for n in ("ne00", "ne01", "ne02", "ne03", "nb00", "nb01", "nb02", "nb03")]
        + [(n, u32) for n in ("ne10", "ne11", "ne12", "ne13", "nb10", "nb11", "nb12", "nb13")]
        + [("misalignOffsets", u32), ("param1", f32), ("param2", f32), ("param3", f32), ("param4", f32)]
        + [(n, u32) for n in ("ne0_012mp", "ne0_01mp", "ne0_0mp", "ne0_Ls",
                               "ne1_012mp", "ne1_01mp", "ne1_0mp", "ne1_Ls")]
    )


class MuyoMatVecSpec(ctypes.Structure):
    _fields_ = [("blockSize", u32), ("numRows", u32), ("numCols", u32)]


class MuyoQwen2Config(ctypes.Structure):
    _fields_ = [
        ("layers", u32), ("hidden", u32), ("feedForward", u32), ("heads", u32), ("kvHeads", u32),
        ("headDim", u32), ("vocab", u32), ("maxSeq", u32), ("rmsEps", f32), ("ropeBase", f32),
        ("untiedOutput", u32),
    ]


class MuyoSamplerParams(ctypes.Structure):
    """SamplerParams (src/Sampler.h:16-23); see muyo_sample_f32."""
    _fields_ = [
        ("temperature", f32), ("top_k", i32), ("top_p", f32), ("repeat_penalty", f32), ("repeat_last_n", i32),
        ("reserved", u32), ("seed", ctypes.c_uint64),
    ]


def sampler_params(temperature=0.0, top_k=40, top_p=0.95, repeat_penalty=1.0, repeat_last_n=64, seed=0):
    """The reference's defaults (src/Sampler.h:18-23)."""
    return MuyoSamplerParams(temperature, top_k, top_p, repeat_penalty, repeat_last_n, 0, seed)


CONTRACT_WORDS = {
    LlamaAddPushConstants: 29, LlamaMatVecPushConstants: 13, LlamaRopePushConstants: 30,
    LlamaGluPushConstants: 27, LlamaGenericHeadPushConstants: 6, LlamaSoftMaxPushConstants: 17,
    LlamaCopyPushConstants: 30,
}

# Status codes and constants of muyo_hip.h / LlamaContracts.h.
MUYO_OK, MUYO_E_NULL, MUYO_E_CONTRACT, MUYO_E_DISPATCH = 0, -1, -2, -3
MUYO_E_UNSUPPORTED, MUYO_E_RANGE, MUYO_E_NOMEM, MUYO_E_STATE = -4, -5, -6, -7
FUSION_BIAS0, FUSION_BIAS1 = 0x1, 0x2
ROPE_NEOX = 2
GLU_SPLIT = 2

KERNEL = dict(EMBED=0, QKV=1, ATTENTION=2, O_PROJ=3, GATE_UP=4, DOWN=5, LM_HEAD=6, FFN=7)

TENSOR = dict(
    TOKEN_EMBD=0, OUTPUT_NORM=1, ATTN_NORM=2, ATTN_QKV=3, ATTN_QKV_B=4, ATTN_OUTPUT=5, FFN_NORM=6,
    FFN_GATE=7, FFN_UP=8, FFN_DOWN=9, KCACHE=10, VCACHE=11, LOGITS=12, OUTPUT=13,
)

_SIGNATURES = {
    "muyo_last_error": (ctypes.c_char_p, []),
    "muyo_version": (ctypes.c_char_p, []),
    "muyo_mul_mat_vec_f16_f32_f32": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, vp]),
    "muyo_mul_mat_vec_f32_f32_f32": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, vp]),
    "muyo_rms_norm_f32": (ctypes.c_int, [vp, u32, vp, vp, vp, vp, u32, u32, u32, vp]),
    "muyo_rms_norm_f32_f16w": (ctypes.c_int, [vp, u32, vp, vp, vp, vp, u32, u32, u32, vp]),
    "muyo_add_f32": (ctypes.c_int, [vp, u32, vp, vp, vp, vp, u32, u32, u32, vp]),
    "muyo_swiglu_f32": (ctypes.c_int, [vp, vp, vp, vp, u32, u32, u32, vp]),
    "muyo_rope_neox_f32": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, u32, u32, u32, vp]),
    "muyo_soft_max_f32": (ctypes.c_int, [vp, vp, vp, vp, vp, u32, u32, u32, vp]),
    "muyo_argmax_f32": (ctypes.c_int, [vp, vp, vp, u32, u32, u32, vp]),
    "muyo_get_rows_f16_f32": (ctypes.c_int, [vp, vp, vp, vp, u32, u32, u32, vp]),
    "muyo_get_rows_f32": (ctypes.c_int, [vp, vp, vp, vp, u32, u32, u32, vp]),
    "muyo_cpy_f32_f32": (ctypes.c_int, [vp, vp, vp, u32, u32, u32, vp]),
    "muyo_attention_decode_f16kv_workspace_bytes": (ctypes.c_size_t, [u32, u32, u32, u32]),
    "muyo_attention_decode_f16kv": (ctypes.c_int, [vp, vp, vp, vp, vp, u32, u32, u32, u32, f32, vp, u64, vp]),
    "muyo_attention_decode_f16kv_static": (ctypes.c_int, [vp, vp, vp, vp, vp, u32, u32, u32, u32, f32, vp]),
    "muyo_rope_append_f16kv": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, f32, vp]),
    "muyo_decoder_create": (ctypes.c_int, [vp, ctypes.POINTER(vp)]),
    "muyo_decoder_destroy": (None, [vp]),
    "muyo_decoder_tensor": (ctypes.c_int, [vp, u32, u32, ctypes.POINTER(vp), ctypes.POINTER(ctypes.c_uint64)]),
    "muyo_decoder_upload": (ctypes.c_int, [vp, u32, u32, vp, ctypes.c_uint64]),
    "muyo_decoder_download": (ctypes.c_int, [vp, u32, u32, vp, ctypes.c_uint64]),
    "muyo_decoder_fill_random": (ctypes.c_int, [vp, ctypes.c_uint64]),
    "muyo_decoder_fill_kv_random": (ctypes.c_int, [vp, u32, ctypes.c_uint64]),
    "muyo_decoder_step": (ctypes.c_int, [vp, i32, i32, ctypes.POINTER(i32)]),
    "muyo_decoder_generate": (ctypes.c_int, [vp, i32, i32, u32, vp, vp]),
    "muyo_decoder_generate_async": (ctypes.c_int, [vp, i32, i32, u32, vp]),
    "muyo_decoder_generated_ids": (ctypes.c_int, [vp, vp, u32]),
    "muyo_decoder_launches_per_step": (u32, [vp]),
    "muyo_decoder_set_state": (ctypes.c_int, [vp, i32, i32, vp]),
    "muyo_decoder_enqueue_kernel": (ctypes.c_int, [vp, u32, u32, vp]),
    "muyo_self_test": (ctypes.c_int, [ctypes.c_char_p]),
    "muyo_decoder_config": (ctypes.c_int, [vp, vp]),
    "muyo_gguf_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(vp)]),
    "muyo_gguf_close": (None, [vp]),
    "muyo_gguf_version": (u32, [vp]),
    "muyo_gguf_data_offset": (ctypes.c_uint64, [vp]),
    "muyo_gguf_metadata_count": (ctypes.c_uint64, [vp]),
    "muyo_gguf_tensor_count": (ctypes.c_uint64, [vp]),
    "muyo_gguf_tensor_info": (ctypes.c_int, [vp, ctypes.c_uint64, ctypes.POINTER(ctypes.c_char_p),
                                             ctypes.POINTER(u32), ctypes.POINTER(u32),
                                             ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "muyo_gguf_has": (ctypes.c_int, [vp, ctypes.c_char_p]),
    "muyo_gguf_uint_or": (ctypes.c_uint64, [vp, ctypes.c_char_p, ctypes.c_uint64]),
    "muyo_gguf_float_or": (ctypes.c_double, [vp, ctypes.c_char_p, ctypes.c_double]),
    "muyo_gguf_string_or": (ctypes.c_char_p, [vp, ctypes.c_char_p, ctypes.c_char_p]),
    "muyo_gguf_string_array_size": (ctypes.c_uint64, [vp, ctypes.c_char_p]),
    "muyo_gguf_string_array_at": (ctypes.c_char_p, [vp, ctypes.c_char_p, ctypes.c_uint64]),
    "muyo_gguf_tensor_data": (ctypes.c_int, [vp, ctypes.c_char_p, ctypes.POINTER(vp), ctypes.POINTER(ctypes.c_uint64)]),
    "muyo_gguf_qwen2_config": (ctypes.c_int, [vp, u32, vp]),
    "muyo_decoder_load_gguf": (ctypes.c_int, [vp, vp]),
    "muyo_decoder_set_sampler": (ctypes.c_int, [vp, vp]),
    "muyo_decoder_set_history": (ctypes.c_int, [vp, vp, u32]),
    "muyo_sampler_state_bytes": (ctypes.c_size_t, []),
    "muyo_sampler_seed": (ctypes.c_int, [vp, ctypes.c_uint64, vp]),
    "muyo_sample_workspace_bytes": (ctypes.c_size_t, [u32, vp]),
    "muyo_sample_f32": (ctypes.c_int, [vp, u32, vp, u32, vp, vp, vp, vp, vp]),
    "muyo_decoder_prefill": (ctypes.c_int, [vp, vp, u32, i32, ctypes.POINTER(i32)]),
    "muyo_split_f32_f16x2": (ctypes.c_int, [vp, ctypes.c_uint64, vp, vp, vp]),
    "muyo_rms_norm_split_f16x2": (ctypes.c_int, [vp, vp, u32, u32, f32, vp, vp, vp]),
    "muyo_gemm_split_f16": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, u32, u32, u32, vp]),
    "muyo_gemm_swiglu_split_f16": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, u32, u32, u32, vp]),
    "muyo_rope_split_append_f16kv": (ctypes.c_int, [vp, u32, i32, u32, u32, u32, u32, vp, vp, vp, vp, vp, vp]),
    "muyo_prefill_attention_f16kv": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, u32, i32, u32, u32, u32, u32, f32, vp]),
    "muyo_prefill_attention_workspace_bytes": (ctypes.c_size_t, [u32, u32, u32]),
    "muyo_prefill_attention_f16kv_ws": (ctypes.c_int, [vp, vp, vp, vp, vp, vp, u32, i32, u32, u32, u32, u32, f32, vp,
                                                       u64, vp]),
    "muyo_tokenizer_create": (ctypes.c_int, [vp, ctypes.POINTER(vp)]),
    "muyo_tokenizer_destroy": (None, [vp]),
    "muyo_tokenizer_vocab_size": (ctypes.c_uint64, [vp]),
    "muyo_tokenizer_token_text": (ctypes.c_char_p, [vp, ctypes.c_uint64]),
    "muyo_tokenizer_is_special": (ctypes.c_int, [vp, i32]),
    "muyo_tokenizer_encode": (ctypes.c_int, [vp, ctypes.c_char_p, ctypes.c_uint64, ctypes.c_int, vp, ctypes.c_uint64,
                                             ctypes.POINTER(ctypes.c_uint64)]),
    "muyo_tokenizer_decode": (ctypes.c_int, [vp, vp, ctypes.c_uint64, vp, ctypes.c_uint64,
                                             ctypes.POINTER(ctypes.c_uint64)]),
    "muyo_tokenizer_token_bytes": (ctypes.c_int, [vp, i32, vp, ctypes.c_uint64, ctypes.POINTER(ctypes.c_uint64)]),
    "muyo_fill_normal_f16": (ctypes.c_int, [vp, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double, ctypes.c_double, vp]),
    "muyo_fill_normal_f32": (ctypes.c_int, [vp, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double, ctypes.c_double, vp]),
    "muyo_fill_uniform_f32": (ctypes.c_int, [vp, ctypes.c_uint64, ctypes.c_uint64, vp]),
    "muyo_tensor_seed": (ctypes.c_uint64, [ctypes.c_uint64, u32, u32]),
}


class MuyoError(RuntimeError):
    """A launcher returned a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"muyo_hip status {status}: {message}")
        self.status = status


class LibraryMissing(RuntimeError):
    pass


_lib = None


def load(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Load the shared library (once). Raises LibraryMissing if it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    target = pathlib.Path(path) if path is not None else LIB_PATH
    if not target.exists():
        raise LibraryMissing(f"{target} is not built; run __graft_entry__.build() (make -C muyo-llm_amd/csrc)")
    # torch carries its own HIP runtime. Loaded first, it is the one the library binds to, so the
    # process holds a single runtime; loaded after the library, torch's device calls made the
    # library's first launch fail with "no ROCm-capable device".
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(target))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if path is None:
        _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return sorted(_SIGNATURES)


def check(status: int) -> None:
    if status != MUYO_OK:
        raise MuyoError(status, load().muyo_last_error().decode())


def ref(struct_value) -> ctypes.c_void_p:
    return ctypes.cast(ctypes.pointer(struct_value), vp)


# --------------------------------------------------------------------------------------------
# Push-constant fills, as the reference's node factories do them.

def init_fastdiv(d: int) -> tuple[int, int]:
    """ggml's init_fastdiv_values (src/Swiglu.cpp:46-54): (mp, L)."""
    shift = 0
    while shift < 32 and (1 << shift) < d:
        shift += 1
    mp = ((1 << 32) * ((1 << shift) - d) // d + 1) & 0xFFFFFFFF
    return mp, shift


def mat_vec_push_constants(ncols, rows, stride_a=0, stride_b=0, batch_stride_a=0, batch_stride_b=0,
                           batch_stride_d=0, fusion_flags=0, ne02=1, ne12=1, broadcast2=1, broadcast3=1):
    """MatVecExecute (src/FullModel.cpp:133-175)."""
    pc = LlamaMatVecPushConstants()
    pc.ncols = ncols
    pc.strideA = stride_a or ncols
    pc.strideB = stride_b or ncols
    pc.strideD = rows
    pc.batchStrideA, pc.batchStrideB, pc.batchStrideD = batch_stride_a, batch_stride_b, batch_stride_d
    pc.fusionFlags = fusion_flags
    pc.baseWorkGroupY = 0
    pc.ne02, pc.ne12, pc.broadcast2, pc.broadcast3 = ne02, ne12, broadcast2, broadcast3
    return pc


def rows_push_constants(length, rows=1, eps=0.0, weight_length=None):
    """RmsNormExecute / AddExecute (src/FullModel.cpp:215-284) for `rows` contiguous rows."""
    pc = LlamaAddPushConstants()
    pc.ne = length * rows
    pc.ne00, pc.ne01, pc.ne02, pc.ne03 = length, rows, 1, 1
    pc.nb00, pc.nb01, pc.nb02, pc.nb03 = 1, length, length * rows, length * rows
    wl = length if weight_length is None else weight_length
    pc.ne10, pc.ne11, pc.ne12, pc.ne13 = wl, 1, 1, 1
    pc.nb10, pc.nb11, pc.nb12, pc.nb13 = 1, wl, wl, wl
    pc.ne20, pc.ne21, pc.ne22, pc.ne23 = length, rows, 1, 1
    pc.nb20, pc.nb21, pc.nb22, pc.nb23 = 1, length, length * rows, length * rows
    pc.param1 = eps
    return pc


def add_push_constants(count, row=None):
    """MakeAddPushConstants (src/ElementwiseAdd.cpp:59-88) for a flat tensor, or [rows][row]."""
    if row is None:
        return rows_push_constants(count, 1)
    return rows_push_constants(row, count // row)


def add_dispatch(count):
    """add.comp's canonical dispatch: (1, ceil(ne/512)) split into z past 512 y-blocks."""
    y = (count + 511) // 512
    if y > 512:
        return 1, 512, (y + 511) // 512
    return 1, y, 1


def glu_push_constants(count, row=None):
    """SwigluExecute (src/FullModel.cpp:287-327), split mode, flat or [rows][row]."""
    pc = LlamaGluPushConstants()
    ne20 = count if row is None else row
    ne21 = 1 if row is None else count // row
    pc.N, pc.ne00, pc.ne20, pc.mode = count, ne20, ne20, GLU_SPLIT
    for prefix in ("nb0", "nb1", "nb2"):
        setattr(pc, prefix + "0", 1)
        setattr(pc, prefix + "1", ne20)
        setattr(pc, prefix + "2", ne20 * ne21)
        setattr(pc, prefix + "3", ne20 * ne21)
    pc.ne21, pc.ne22 = ne21, 1
    pc.ne2_012mp, pc.ne2_012L = init_fastdiv(ne20 * ne21)
    pc.ne2_01mp, pc.ne2_01L = init_fastdiv(ne20 * ne21)
    pc.ne2_0mp, pc.ne2_0L = init_fastdiv(ne20)
    return pc


def rope_push_constants(rows, head_dim, freq_base, input_row_stride=None, output_row_stride=None,
                        destination_offset=0, tokens=1):
    """RopeExecute (src/FullModel.cpp:179-212): `rows` heads per token, `tokens` positions."""
    pc = LlamaRopePushConstants()
    pc.ropeMode = ROPE_NEOX
    pc.nrows = rows * tokens
    pc.nDims = head_dim
    pc.freqScale, pc.freqBase, pc.extFactor, pc.attnFactor = 1.0, freq_base, 0.0, 1.0
    pc.thetaScale = theta_scale(freq_base, head_dim)
    pc.ne00, pc.ne01, pc.ne02 = head_dim, rows, tokens
    irs = input_row_stride or head_dim
    ors = output_row_stride or head_dim
    pc.nb01, pc.nb02, pc.nb03 = irs, irs * rows, irs * rows * tokens
    pc.nb11, pc.nb12, pc.nb13 = ors, ors * rows, ors * rows * tokens
    pc.dOffset = destination_offset
    return pc


def theta_scale(freq_base: float, head_dim: int) -> float:
    """std::pow(freqBase, -2.0F / headDim) in f32, as src/FullModel.cpp:201 computes it."""
    import numpy as np

    return float(np.power(np.float32(freq_base), np.float32(-2.0) / np.float32(head_dim), dtype=np.float32))


def soft_max_push_constants(rows, columns, scale):
    """SoftMaxExecute (src/FullModel.cpp:331-349)."""
    pc = LlamaSoftMaxPushConstants()
    pc.KX, pc.KY, pc.ne00, pc.ne01, pc.ne02 = columns, 0, columns, rows, 1
    pc.ne12, pc.ne13 = 1, 1
    pc.scale = scale
    pc.nrowsX = rows
    return pc


def row_dispatch(rows):
    """Workgroup grid for a one-workgroup-per-row op (row = z*262144 + y*512 + x)."""
    if rows <= 512:
        return rows, 1, 1
    y = (rows + 511) // 512
    if y <= 512:
        return 512, y, 1
    return 512, 512, (rows + 262143) // 262144


def argmax_push_constants(columns, rows=1):
    """ArgmaxExecute (src/FullModel.cpp:461-484)."""
    pc = LlamaGenericHeadPushConstants()
    pc.KX, pc.KY = columns, rows
    return pc


def get_rows_push_constants(embed_dim, vocab, count=1):
    """GetRowsExecute (src/FullModel.cpp:424-458) gathering `count` indices."""
    pc = LlamaAddPushConstants()
    pc.ne = embed_dim * vocab
    pc.ne00, pc.ne01, pc.ne02, pc.ne03 = embed_dim, vocab, 1, 1
    pc.nb00, pc.nb01, pc.nb02, pc.nb03 = 1, embed_dim, embed_dim * vocab, embed_dim * vocab
    pc.ne10, pc.ne11, pc.ne12, pc.ne13 = count, 1, 1, 1
    pc.nb10, pc.nb11, pc.nb12, pc.nb13 = 1, count, count, count
    pc.ne20, pc.ne21, pc.ne22, pc.ne23 = embed_dim, count, 1, 1
    pc.nb20, pc.nb21, pc.nb22, pc.nb23 = 1, embed_dim, embed_dim * count, embed_dim * count
    return pc


def value_column_push_constants(kv_dim, head_dim, max_seq, position):
    """CopyValueColumnExecute (src/FullModel.cpp:376-420): v[kvh][c] -> cache[kvh][c][pos]."""
    pc = LlamaCopyPushConstants()
    pc.ne = kv_dim
    pc.ne00, pc.ne01, pc.ne02, pc.ne03, pc.nb00 = kv_dim, 1, 1, 1, 1
    pc.ne10, pc.ne11, pc.ne12, pc.ne13 = head_dim, max_seq, 1, 1
    pc.nb10, pc.nb11 = max_seq, head_dim * max_seq
    pc.misalignOffsets = position
    mp0, l0 = init_fastdiv(pc.ne11)
    mp1, l1 = init_fastdiv(pc.ne11 * pc.ne10)
    mp2, l2 = init_fastdiv(pc.ne12 * pc.ne11 * pc.ne10)
    pc.ne1_0mp, pc.ne1_01mp, pc.ne1_012mp = mp0, mp1, mp2
    pc.ne1_Ls = l2 | (l1 << 8) | (l0 << 16)
    s0mp, s0 = init_fastdiv(pc.ne00)
    s1mp, s1 = init_fastdiv(pc.ne01 * pc.ne00)
    s2mp, s2 = init_fastdiv(pc.ne02 * pc.ne01 * pc.ne00)
    pc.ne0_0mp, pc.ne0_01mp, pc.ne0_012mp = s0mp, s1mp, s2mp
    pc.ne0_Ls = s2 | (s1 << 8) | (s0 << 16)
    return pc


def contract_bytes(struct_value) -> bytes:
    return bytes(memoryview(struct_value).cast("B"))


def qwen2_config(layers, hidden, ffn, heads, kv_heads, head_dim, vocab, max_seq, eps=1e-6, rope_base=1e6,
                 untied_output=False):
    c = MuyoQwen2Config()
    c.layers, c.hidden, c.feedForward, c.heads, c.kvHeads = layers, hidden, ffn, heads, kv_heads
    c.headDim, c.vocab, c.maxSeq, c.rmsEps, c.ropeBase = head_dim, vocab, max_seq, eps, rope_base
    c.untiedOutput = 1 if untied_output else 0
    return c


QWEN25_05B = dict(layers=24, hidden=896, ffn=4864, heads=14, kv_heads=2, head_dim=64, vocab=151936, max_seq=2048)
QWEN25_7B = dict(layers=28, hidden=3584, ffn=18944, heads=28, kv_heads=4, head_dim=128, vocab=152064, max_seq=2048)


class Gguf:
    """A mapped GGUF file (muyo_gguf_* in include/muyo_hip.h)."""

    def __init__(self, path):
        self.lib = load()
        handle = vp()
        check(self.lib.muyo_gguf_open(os.fsencode(path), ctypes.byref(handle)))
        self.handle = handle

    def close(self):
        if self.handle:
            self.lib.muyo_gguf_close(self.handle)
            self.handle = vp()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def version(self) -> int:
        return int(self.lib.muyo_gguf_version(self.handle))

    @property
    def data_offset(self) -> int:
        return int(self.lib.muyo_gguf_data_offset(self.handle))

    def tensors(self) -> list[tuple[str, int, list[int], int]]:
        """(name, ggml type, dims fastest-varying first, offset) per table entry."""
        out = []
        for i in range(int(self.lib.muyo_gguf_tensor_count(self.handle))):
            name, typ, nd = ctypes.c_char_p(), u32(), u32()
            dims, off = (ctypes.c_uint64 * 4)(), ctypes.c_uint64()
            check(self.lib.muyo_gguf_tensor_info(self.handle, i, ctypes.byref(name), ctypes.byref(typ),
                                                 ctypes.byref(nd), dims, ctypes.byref(off)))
            out.append((name.value.decode(), typ.value, list(dims)[:nd.value], off.value))
        return out

    def uint_or(self, key: str, fallback: int) -> int:
        return int(self.lib.muyo_gguf_uint_or(self.handle, key.encode(), fallback))

    def float_or(self, key: str, fallback: float) -> float:
        return float(self.lib.muyo_gguf_float_or(self.handle, key.encode(), fallback))

    def string_or(self, key: str, fallback: str) -> str:
        return self.lib.muyo_gguf_string_or(self.handle, key.encode(), fallback.encode()).decode()

    def string_array_size(self, key: str) -> int:
        return int(self.lib.muyo_gguf_string_array_size(self.handle, key.encode()))

    def string_array_at(self, key: str, index: int) -> str | None:
        v = self.lib.muyo_gguf_string_array_at(self.handle, key.encode(), index)
        return None if v is None else v.decode()

    def tensor_bytes(self, name: str) -> bytes:
        data, n = vp(), ctypes.c_uint64()
        check(self.lib.muyo_gguf_tensor_data(self.handle, name.encode(), ctypes.byref(data), ctypes.byref(n)))
        return ctypes.string_at(data, n.value)

    def qwen2_config(self, max_seq: int) -> MuyoQwen2Config:
        c = MuyoQwen2Config()
        check(self.lib.muyo_gguf_qwen2_config(self.handle, max_seq, ref(c)))
        return c


class Tokenizer:
    """Owner of a MuyoTokenizer (muyo_tokenizer_* in include/muyo_hip.h), with the reference's
    Tokenizer methods (src/Tokenizer.h:22-88). Host code: no device is needed."""

    def __init__(self, gguf: Gguf):
        self.lib = load()
        handle = vp()
        check(self.lib.muyo_tokenizer_create(gguf.handle, ctypes.byref(handle)))
        self.handle = handle

    def close(self):
        if self.handle:
            self.lib.muyo_tokenizer_destroy(self.handle)
            self.handle = vp()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def vocab_size(self) -> int:
        return int(self.lib.muyo_tokenizer_vocab_size(self.handle))

    def token_for(self, id: int) -> str:
        """The vocabulary string of `id` ("" out of range), as UTF-8 text."""
        return self.lib.muyo_tokenizer_token_text(self.handle, id).decode("utf-8", "surrogateescape")

    def is_special(self, id: int) -> bool:
        return bool(self.lib.muyo_tokenizer_is_special(self.handle, id))

    def encode(self, text: str | bytes, parse_special: bool = True) -> list[int]:
        data = text.encode("utf-8", "surrogateescape") if isinstance(text, str) else bytes(text)
        cap = 3 * len(data) + 1
        ids, n = (i32 * cap)(), ctypes.c_uint64()
        check(self.lib.muyo_tokenizer_encode(self.handle, data, len(data), int(parse_special), ids, cap,
                                             ctypes.byref(n)))
        return list(ids[:n.value])

    def _text(self, call) -> bytes:
        """Bytes from a call(buffer, capacity, &length) entry point, growing the buffer once when
        the first one is too small."""
        n = ctypes.c_uint64()
        cap = 256
        while True:
            buf = ctypes.create_string_buffer(cap)
            status = call(buf, cap, ctypes.byref(n))
            if status == MUYO_OK:
                return buf.raw[:n.value]
            if n.value <= cap:
                check(status)
            cap = int(n.value)

    def decode_bytes(self, ids) -> bytes:
        arr = (i32 * max(1, len(ids)))(*ids)
        return self._text(lambda buf, cap, n: self.lib.muyo_tokenizer_decode(self.handle, arr, len(ids), buf, cap, n))

    def decode(self, ids) -> str:
        return self.decode_bytes(ids).decode("utf-8", "replace")

    def token_bytes(self, id: int) -> bytes:
        return self._text(lambda buf, cap, n: self.lib.muyo_tokenizer_token_bytes(self.handle, id, buf, cap, n))


# Qwen2.5's ChatML framing (the reference's src/ChatTemplate.h:9-29, src/ChatTemplate.cpp).
QWEN2_DEFAULT_SYSTEM = "You are Qwen, created by Alibaba Cloud. You are a helpful assistant."


def qwen2_system_start(system: str) -> str:
    return "<|im_start|>system\n" + system + "<|im_end|>\n"


def qwen2_user_turn(user: str) -> str:
    return "<|im_start|>user\n" + user + "<|im_end|>\n<|im_start|>assistant\n"


def qwen2_chat_start(system: str, user: str) -> str:
    return qwen2_system_start(system) + qwen2_user_turn(user)


class Decoder:
    """Owner of a MuyoDecoder (muyo_decoder_* in include/muyo_hip.h)."""

    def __init__(self, config: MuyoQwen2Config):
        self.lib = load()
        self.config = config
        handle = vp()
        check(self.lib.muyo_decoder_create(ref(config), ctypes.byref(handle)))
        self.handle = handle

    def close(self):
        if self.handle:
            self.lib.muyo_decoder_destroy(self.handle)
            self.handle = vp()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def tensor(self, kind: str, layer: int = 0) -> tuple[int, int]:
        ptr, nbytes = vp(), ctypes.c_uint64()
        check(self.lib.muyo_decoder_tensor(self.handle, TENSOR[kind], layer, ctypes.byref(ptr), ctypes.byref(nbytes)))
        return ptr.value or 0, nbytes.value

    def upload(self, kind: str, layer: int, array) -> None:
        check(self.lib.muyo_decoder_upload(self.handle, TENSOR[kind], layer, array.ctypes.data, array.nbytes))

    def download(self, kind: str, layer: int, array) -> None:
        check(self.lib.muyo_decoder_download(self.handle, TENSOR[kind], layer, array.ctypes.data, array.nbytes))

    def fill_random(self, seed: int) -> None:
        check(self.lib.muyo_decoder_fill_random(self.handle, seed))

    def fill_kv_random(self, positions: int, seed: int) -> None:
        check(self.lib.muyo_decoder_fill_kv_random(self.handle, positions, seed))

    def step(self, token: int, position: int) -> int:
        nxt = i32()
        check(self.lib.muyo_decoder_step(self.handle, token, position, ctypes.byref(nxt)))
        return nxt.value

    def prefill(self, tokens, position: int = 0) -> int:
        """Feed a prompt at cache rows position.. in one batched pass; returns the next token."""
        import numpy as np

        arr = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32))
        nxt = i32()
        check(self.lib.muyo_decoder_prefill(self.handle, arr.ctypes.data, arr.size, position, ctypes.byref(nxt)))
        return nxt.value

    def generate(self, token: int, position: int, count: int, stream: int = 0) -> list[int]:
        ids = (i32 * max(count, 1))()
        check(self.lib.muyo_decoder_generate(self.handle, token, position, count, ids, stream))
        return list(ids)[:count]

    def generate_async(self, token: int, position: int, count: int, stream: int = 0) -> None:
        check(self.lib.muyo_decoder_generate_async(self.handle, token, position, count, stream))

    def generated_ids(self, count: int) -> list[int]:
        ids = (i32 * max(count, 1))()
        check(self.lib.muyo_decoder_generated_ids(self.handle, ids, count))
        return list(ids)[:count]

    def launches_per_step(self) -> int:
        return int(self.lib.muyo_decoder_launches_per_step(self.handle))

    def set_state(self, token: int, position: int, stream: int = 0) -> None:
        check(self.lib.muyo_decoder_set_state(self.handle, token, position, stream))

    def load_gguf(self, gguf: "Gguf") -> None:
        check(self.lib.muyo_decoder_load_gguf(self.handle, gguf.handle))

    def set_sampler(self, **params) -> None:
        """Sampler::Sample after every step (sampler_params' keywords); no keywords: greedy."""
        p = sampler_params(**params) if params else None
        check(self.lib.muyo_decoder_set_sampler(self.handle, ref(p) if p is not None else None))

    def set_history(self, tokens) -> None:
        arr = (i32 * max(len(tokens), 1))(*[int(t) for t in tokens])
        check(self.lib.muyo_decoder_set_history(self.handle, arr, len(tokens)))

    def enqueue_kernel(self, kernel: str, layer: int = 0, stream: int = 0) -> None:
        check(self.lib.muyo_decoder_enqueue_kernel(self.handle, KERNEL[kernel], layer, stream))


def tensor_seed(seed: int, kind: str, layer: int) -> int:
    return int(load().muyo_tensor_seed(seed, TENSOR[kind], layer))


def _self_check_sizes() -> None:
    for cls, words in CONTRACT_WORDS.items():
        assert ctypes.sizeof(cls) == 4 * words, cls.__name__
    assert ctypes.sizeof(MuyoSamplerParams) == 32


_self_check_sizes()
__all__ = [n for n in dir() if not n.startswith("_")]
del struct, math
