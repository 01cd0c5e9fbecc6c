"""`muyo_llm --forward` flag handling (src/main.cpp:353-414's options), which runs before any
device is touched: unknown flags are usage errors (exit 2), a flag without its value or with a
malformed number fails with exit 1 and says which. No GPU."""
import os
import pathlib
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
CLI = pathlib.Path(os.environ.get("MUYO_LLM_CLI") or ROOT / "muyo-llm_amd" / "muyo_llm")

pytestmark = pytest.mark.skipif(not CLI.exists(), reason="the muyo_llm CLI is not built")


def forward(*args):
    p = subprocess.run([str(CLI), "--forward", *args], capture_output=True, timeout=60)
    return p.returncode, p.stderr.decode()


def test_usage_without_a_model():
    code, err = forward()
    assert code == 2 and "usage:" in err


@pytest.mark.parametrize("flag", ["--bogus", "-x", "--Temp", "-pp"])
def test_unknown_flags_are_usage_errors(flag):
    code, err = forward("model.gguf", "-n", "3", flag)
    assert code == 2 and f"unknown --forward option: {flag}" in err


@pytest.mark.parametrize("flag,name", [("-n", "--n-predict"), ("--temp", "--temp"), ("-p", "--prompt"),
                                       ("--tokens", "--tokens"), ("--seed", "--seed"), ("--system", "--system")])
def test_a_flag_without_its_value(flag, name):
    code, err = forward("model.gguf", "--chat", flag)
    assert code == 1 and f"[fail] {name} needs a value" in err


@pytest.mark.parametrize("flag,value", [("-n", "many"), ("--top-k", ""), ("--seed", "x1"), ("--ctx", "-")])
def test_malformed_numbers_fail(flag, value):
    code, err = forward("model.gguf", flag, value)
    assert code == 1 and err.startswith("[fail]")
