"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer, as the reference runs
every mode of its build under ASan/UBSan (CMakeLists.txt:42-45, scripts/sanity.sh:75-87).

`make -C muyo-llm_amd/csrc san` rebuilds the library and the CLI with the host code
instrumented (the device code as usual). This test reruns the CPU tests of the host parts
against that build:
- the GGUF reader, including every truncation and seeded corruptions of a file's tables;
- the tokenizer and its CLI mode;
- the --forward flag parsing;
- the C-ABI argument checks;
- the host sampler.

It preloads clang's ASan runtime and fails on any report. No GPU."""
import os
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
SAN = ROOT / "muyo-llm_amd" / "_build" / "san"
CLANG = pathlib.Path("/opt/rocm/llvm/bin/clang")
SUITES = ["tests/test_gguf.py", "tests/test_tokenizer.py", "tests/test_forward_cli.py", "tests/test_abi.py",
          "tests/test_sampler.py"]


def asan_runtime() -> pathlib.Path | None:
    if not CLANG.exists():
        return None
    out = subprocess.run([str(CLANG), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                         text=True).stdout.strip()
    path = pathlib.Path(out)
    return path if path.is_absolute() and path.exists() else None


@pytest.mark.timeout(900)
def test_host_code_under_asan_and_ubsan():
    lib, cli = SAN / "libmuyo_hip.so", SAN / "muyo_llm"
    runtime = asan_runtime()
    if not lib.exists() or not cli.exists():
        pytest.skip("the sanitizer build is absent (make -C muyo-llm_amd/csrc san)")
    if runtime is None:
        pytest.skip("clang's ASan runtime was not found")
    env = dict(os.environ, MUYO_HIP_LIBRARY=str(lib), MUYO_LLM_CLI=str(cli), LD_PRELOAD=str(runtime),
               ASAN_OPTIONS="detect_leaks=0:alloc_dealloc_mismatch=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    p = subprocess.run([sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider", *SUITES],
                       cwd=ROOT, env=env, capture_output=True, timeout=850)
    out = p.stdout.decode(errors="replace") + p.stderr.decode(errors="replace")
    assert p.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert " passed" in out
