"""Shared fixtures.  GPU tests are marked `gpu`; everything else runs on the CPU.

torch is imported before libg4.so is loaded, so the process has a single HIP
runtime (torch's and ROCm's libamdhip64 share one soname).
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402

MODEL_SEED = 20261201


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def pkg():
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def image(pkg):
    """The synthetic E2B model image (exporter layout, ~5.0 GB, seeded)."""
    return pkg.Image.synthetic(seed=MODEL_SEED)


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import binding
    return binding


@pytest.fixture(scope="session")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.fixture(scope="session")
def g4lib(pkg, torch_gpu):
    return pkg.lib()


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def random_weight(gen: np.random.Generator, n: int, k: int):
    """Packed int8 weight U[-127, 127] with fp16 scales log-uniform in
    [1e-3, 1e-2] per (row, 64-group): the matmul workload's distributions."""
    w = gen.integers(-127, 128, size=(n, k), dtype=np.int8)
    s = np.exp(gen.uniform(np.log(1e-3), np.log(1e-2), size=(n, k // 64))).astype(np.float16)
    return w, s
