"""Shared fixtures. GPU tests are marked `gpu`; everything else runs on the CPU."""
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for sub in ("muyo-llm_amd", "oracle"):
    path = str(ROOT / sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu on the GPU box)")


def pytest_report_header(config):
    return f"muyo root: {ROOT}"


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.load()
    return oracle


@pytest.fixture(scope="session")
def mh():
    import muyo_hip

    muyo_hip.load()
    return muyo_hip


@pytest.fixture(scope="session")
def gpu(mh):
    """torch on cuda:0 with the HIP library loaded; the kernels never fall back to the CPU."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("a GPU test ran without a visible GPU")
    torch.cuda.set_device(0)
    return torch


def close(actual, expected, tol):
    """The reference's mixed tolerance |a - e| <= tol * (1 + |e|) (src/RmsNorm.cpp:52-55)."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    bad = np.abs(actual - expected) > tol * (1.0 + np.abs(expected))
    return int(bad.sum())


def worst(actual, expected):
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    return float(np.max(np.abs(actual - expected) / (1.0 + np.abs(expected)))) if actual.size else 0.0
