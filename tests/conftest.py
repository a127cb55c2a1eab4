"""Shared test setup: the ``gpu`` marker, repo-root imports, and fixtures for
the native library and the CUDA (HIP) device."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_addoption(parser):
    parser.addoption("--gemm-random-cases", type=int, default=20,
                     help="seeded random GEMM shapes per input type in test_gpu_gemm_random.py (default 20)")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libmi355bench.so")


@pytest.fixture(scope="session")
def torch_gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu-marked test ran without a visible GPU")
    torch.cuda.set_device(0)
    return torch


@pytest.fixture(scope="session")
def lib(torch_gpu):
    """libmi355bench.so, loaded; a missing or stale build FAILS (never skips) GPU tests."""
    from teamredbench_amd.native import capi

    return capi.load_library()


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import clib

    return clib.load()


@pytest.fixture
def tune(lib):
    """Force plan knobs (mb_set_tuning) for one test: ``tune(gemm_splits=2)``. Every knob the test
    touched is restored when it ends, so the overrides never leak into later tests."""
    saved: dict[str, int | None] = {}

    def set_knobs(**knobs: int | None) -> None:
        for name, value in knobs.items():
            saved.setdefault(name, lib.get_tuning(name))
            lib.set_tuning(name, value)

    yield set_knobs
    for name, value in saved.items():
        lib.set_tuning(name, value)
