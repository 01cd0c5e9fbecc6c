"""The C-ABI boundary, checked on the CPU: the library loads, exports every symbol the header
declares, the contract structs have the reference's sizes, and argument errors are reported
before anything touches a GPU."""
import ctypes
import os
import pathlib
import re
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "muyo_hip.h"
CONTRACTS = ROOT / "include" / "muyo" / "LlamaContracts.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(muyo_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(mh):
    lib_path = mh.LIB_PATH
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib_path)], capture_output=True, text=True, check=True)
    exported = set(re.findall(r" T (muyo_\w+)", out.stdout))
    missing = [s for s in declared_symbols() if s not in exported]
    assert not missing, missing
    lib = mh.load()
    for name in declared_symbols():
        assert hasattr(lib, name)
    assert set(mh.exported_symbols()) == set(declared_symbols())


def test_header_compiles_as_c_and_sizes_match(tmp_path, mh):
    """The contract header is plain C (for cgo/JNI/ctypes) and its sizes are the reference's."""
    probe = tmp_path / "probe.c"
    probe.write_text(
        '#include <stdio.h>\n#include "muyo_hip.h"\nint main(void){printf("%zu %zu %zu %zu %zu %zu %zu\\n",'
        "sizeof(LlamaAddPushConstants), sizeof(LlamaMatVecPushConstants), sizeof(LlamaRopePushConstants),"
        "sizeof(LlamaGluPushConstants), sizeof(LlamaGenericHeadPushConstants), sizeof(LlamaSoftMaxPushConstants),"
        "sizeof(LlamaCopyPushConstants)); return 0;}\n")
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", str(ROOT / "include"), str(probe), "-o", str(exe)],
                   check=True)
    sizes = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    # src/LlamaContracts.h:41,87,156,202,235,277 and src/FullModel.cpp:364.
    assert sizes == [29 * 4, 13 * 4, 30 * 4, 27 * 4, 6 * 4, 17 * 4, 30 * 4]
    for cls, words in mh.CONTRACT_WORDS.items():
        assert ctypes.sizeof(cls) == 4 * words


def test_fastdiv_magic_is_exact_division(mh):
    """init_fastdiv_values (src/Swiglu.cpp:46-54): (mulhi(n, mp) + n) >> L == n / d for n < 2^31."""
    for d in (1, 2, 3, 7, 64, 600, 896, 2048, 4864, 131072, 4096 * 4864):
        mp, shift = mh.init_fastdiv(d)
        for n in (0, 1, d - 1, d, d + 1, 12345, 2**20 + 7, 2**31 - 1):
            assert ((((n * mp) >> 32) + n) >> shift) == n // d, (d, n)


def test_value_column_packing_order(mh):
    """src/FullModel.cpp:398-408: shifts packed outermost divisor first (Finding F12)."""
    pc = mh.value_column_push_constants(128, 64, 2048, 5)
    _, l012 = mh.init_fastdiv(64 * 2048)
    _, l0 = mh.init_fastdiv(2048)
    assert pc.ne1_Ls & 0xFF == l012 and (pc.ne1_Ls >> 16) & 0xFF == l0
    assert pc.misalignOffsets == 5


def test_argument_errors_without_a_gpu(mh):
    lib = mh.load()
    pc = mh.mat_vec_push_constants(8, 8)
    assert lib.muyo_mul_mat_vec_f16_f32_f32(mh.ref(pc), None, None, None, None, None, None, 8, 1, 1, 0) == mh.MUYO_E_NULL
    assert b"required" in lib.muyo_last_error()
    assert lib.muyo_rms_norm_f32(None, 1, None, None, None, None, 1, 1, 1, 0) == mh.MUYO_E_NULL
    # rms_norm's dispatch is (rows, channels, samples): past the tensor it is refused, not read.
    rows = mh.rows_push_constants(896, 4096, 1e-6)
    fake = ctypes.c_void_p(16)
    assert lib.muyo_rms_norm_f32(mh.ref(rows), 1, fake, fake, fake, None, 512, 8, 1, 0) == mh.MUYO_E_DISPATCH
    assert lib.muyo_rms_norm_f32(mh.ref(rows), 1, fake, fake, fake, None, 4097, 1, 1, 0) == mh.MUYO_E_DISPATCH
    glu = mh.glu_push_constants(600)
    glu.ne2_012mp ^= 1
    fake = ctypes.c_void_p(16)
    assert lib.muyo_swiglu_f32(mh.ref(glu), fake, fake, fake, 1, 2, 1, 0) == mh.MUYO_E_CONTRACT
    glu = mh.glu_push_constants(600)
    assert lib.muyo_swiglu_f32(mh.ref(glu), fake, fake, fake, 2, 2, 1, 0) == mh.MUYO_E_DISPATCH
    cfg = mh.qwen2_config(1, 896, 4864, 14, 2, 96, 1000, 64)
    handle = ctypes.c_void_p()
    assert lib.muyo_decoder_create(mh.ref(cfg), ctypes.byref(handle)) == mh.MUYO_E_UNSUPPORTED
    assert not handle.value


def test_step_bytes_match_the_published_derivation():
    """BASELINE.md section 2 (derived, not published): 987,922,432 B of fp16 weights at the
    0.5B shape and 12,288 B of fp16 KV per position."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("bench", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    import muyo_hip as mh

    s = dict(mh.QWEN25_05B)
    b1, b2 = bench.step_bytes(s, 1024), bench.step_bytes(s, 1025)
    assert b2 - b1 == 12_288
    weights = s["layers"] * 2 * (1152 * 896 + 896 * 896 + 2 * 4864 * 896 + 896 * 4864) + 2 * 151936 * 896
    assert weights == 987_922_432
    # + KV rows 0..1024 (12.6 MB) + f32 activations, biases, norms and logits (2.6 MB)
    assert 987_922_432 + 12_288 * 1025 < b1 < 987_922_432 + 12_288 * 1025 + 3_000_000
    s7 = dict(mh.QWEN25_7B)
    w7 = s7["layers"] * 2 * (4608 * 3584 + 3584 * 3584 + 3 * 18944 * 3584) + 2 * 152064 * 3584
    assert w7 == 14_140_571_648


def test_node_factories_fill_like_the_reference(tmp_path, mh):
    """include/muyo/Nodes.h compiles as C++ and its Make* fills equal the Python mirror's word for
    word (the fills the GPU parity tests use, each citing the reference factory it restates)."""
    probe = tmp_path / "nodes.cpp"
    probe.write_text(r'''
#include <cstdio>
#include "muyo/Nodes.h"
using namespace muyo_llm::hip;
template <typename T> void Dump(const char* name, const T& pc) {
    const unsigned char* p = reinterpret_cast<const unsigned char*>(&pc);
    std::printf("%s ", name);
    for (size_t i = 0; i < sizeof(T); ++i) std::printf("%02x", p[i]);
    std::printf("\n");
}
int main() {
    Dump("matvec", MakeMatVec(896, 1152, LLAMA_MAT_VEC_FUSION_BIAS0));
    Dump("rows", MakeRows(896, 4, 1e-6F));
    Dump("add", MakeAdd(1000));
    Dump("swiglu", MakeSwiglu(600));
    Dump("rope", MakeRopeNeox(2, 64, 1e6F, 64 * 2048, 1234 * 64));
    Dump("softmax", MakeSoftMax(14, 2048, 0.125F));
    Dump("argmax", MakeArgmax(151936));
    Dump("getrows", MakeGetRows(896, 151936));
    Dump("valuecol", MakeValueColumn(128, 64, 2048, 5));
    return 0;
}
''')
    exe = tmp_path / "nodes"
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-I", str(ROOT / "include"), str(probe), "-o", str(exe)],
                   check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                       check=True).stdout.splitlines())
    want = {
        "matvec": mh.mat_vec_push_constants(896, 1152, fusion_flags=mh.FUSION_BIAS0),
        "rows": mh.rows_push_constants(896, 4, 1e-6),
        "add": mh.add_push_constants(1000),
        "swiglu": mh.glu_push_constants(600),
        "rope": mh.rope_push_constants(2, 64, 1e6, output_row_stride=64 * 2048, destination_offset=1234 * 64),
        "softmax": mh.soft_max_push_constants(14, 2048, 0.125),
        "argmax": mh.argmax_push_constants(151936),
        "getrows": mh.get_rows_push_constants(896, 151936),
        "valuecol": mh.value_column_push_constants(128, 64, 2048, 5),
    }
    for name, pc in want.items():
        assert got[name] == mh.contract_bytes(pc).hex(), name


def test_sampler_header_compiles_and_mirrors_sampler_params(tmp_path):
    """include/muyo/Sampler.h (the device-backed mirror of src/Sampler.h) compiles as C++, and
    MuyoSamplerParams is the C layout the bindings assume (32 bytes, seed at offset 24)."""
    probe = tmp_path / "sampler.cpp"
    probe.write_text(r'''
#include <cstddef>
#include <cstdio>
#include "muyo/Sampler.h"
static_assert(sizeof(MuyoSamplerParams) == 32, "MuyoSamplerParams layout");
static_assert(offsetof(MuyoSamplerParams, seed) == 24, "seed offset");
int Use(float* logits) {
    muyo_llm::hip::SamplerParams params;
    params.temperature = 0.7F;
    muyo_llm::hip::Sampler sampler(params, 151936);
    return sampler.Sample(logits, 151936, {1, 2, 3});
}
''')
    subprocess.run(["/opt/rocm/bin/hipcc", "-std=c++17", "-Wall", "-Werror", "-Wno-unused-command-line-argument",
                    "-fsyntax-only", "-I", str(ROOT / "include"), str(probe)], check=True)


def test_tokenizer_and_chat_headers_work_as_the_reference_classes(tmp_path, mh):
    """include/muyo/Tokenizer.h and include/muyo/ChatTemplate.h (mirrors of src/Tokenizer.h and
    src/ChatTemplate.h) compile as C++ and, linked to the library, encode the ChatML prompt as the
    Python binding does and decode it back (the tokenizer is host code: no device)."""
    if os.environ.get("MUYO_HIP_LIBRARY"):
        pytest.skip("links a g++ program against the library; the run over the product build covers it")
    import json

    import gguf_writer as gw

    vocab = json.loads((ROOT / "tests" / "golden" / "bpe_vocab.json").read_text(encoding="utf-8"))
    gguf = tmp_path / "tok.gguf"
    gw.tokenizer_file(gguf, vocab, "qwen2")
    probe = tmp_path / "tok.cpp"
    probe.write_text(r'''
#include <cstdio>
#include "muyo/ChatTemplate.h"
#include "muyo/Tokenizer.h"
int main(int argc, char** argv) {
    MuyoGguf* g = nullptr;
    if (muyo_gguf_open(argv[1], &g) != MUYO_OK) return 3;
    muyo_llm::hip::Tokenizer tok(g);
    muyo_gguf_close(g);
    namespace ct = muyo_llm::hip::chat_template;
    const std::string text = ct::Qwen2ChatStart(ct::QWEN2_DEFAULT_SYSTEM, "Hi there");
    const std::vector<int32_t> ids = tok.Encode(text);
    for (int32_t id : ids) std::printf("%d ", id);
    std::printf("\n%d %d %zu\n", tok.Decode(ids) == text ? 1 : 0, tok.IsSpecial(ids[0]) ? 1 : 0, tok.VocabSize());
    try { tok.Encode("\xf4\x90\x80\x80"); } catch (const std::invalid_argument&) { std::printf("threw\n"); }
    return 0;
}
''')
    exe = tmp_path / "tok"
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-I", str(ROOT / "include"), str(probe), "-o", str(exe),
                    "-L", str(mh.LIB_PATH.parent), "-lmuyo_hip", f"-Wl,-rpath,{mh.LIB_PATH.parent}"], check=True)
    out = subprocess.run([str(exe), str(gguf)], capture_output=True, text=True, check=True).stdout.splitlines()
    with mh.Gguf(gguf) as g, mh.Tokenizer(g) as tok:
        want = tok.encode(mh.qwen2_chat_start(mh.QWEN2_DEFAULT_SYSTEM, "Hi there"))
    assert [int(x) for x in out[0].split()] == want
    assert out[1] == f"1 1 {len(vocab['tokens'])}" and out[2] == "threw"
