"""Shared test setup.

* registers the ``gpu`` marker (tests that launch HIP kernels);
* imports the package directory ``kunlunxin-fft_amd`` as ``kunlunxin_fft_amd``;
* puts ``oracle/`` on the path (the CPU checker; tests are allowed to use it).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libmfft.so")


@pytest.fixture(scope="session")
def pkg():
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    return np.load(os.path.join(ROOT, "tests", "golden", "kat.npz"))


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a ROCm GPU")
    from kunlunxin_fft_amd import native

    native.load()
    return torch.device("cuda:0")
