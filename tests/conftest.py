"""Shared test setup: import paths, the `gpu` marker, and fixtures for the library, the oracle and device buffers.

CPU tests (-m "not gpu") check the oracle against golden data, the host logic and the C ABI surface. GPU tests
(-m gpu) call libgen9blas.so through its C ABI (ctypes, via gen9blas.py or directly) and compare with the oracle.
"""
import os
import sys

import numpy as np
import pytest

try:
    # torch's HIP runtime first: libgen9blas.so, loaded later by any test, then binds to the same runtime (two HIP
    # runtimes in one process leave the second without a device)
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.realpath(__file__)))
PKG = os.path.join(ROOT, "gen9-gpu-blas_amd")
for p in (PKG, os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _torch_gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def g9():
    """The gen9blas module with an initialized GPU. Skips without a GPU; fails if a GPU is there but the library does
    not initialize (the HIP path must be the one that runs)."""
    if not _torch_gpu():
        pytest.skip("no GPU visible to torch")
    import gen9blas
    rc = gen9blas._lib.gen9blas_init()
    assert rc == 0, f"libgen9blas failed to initialize on a GPU box: {gen9blas._lib.gen9blas_error().decode()}"
    return gen9blas


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def seeded(seed):
    return np.random.default_rng(seed)
