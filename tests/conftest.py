"""Shared pytest setup: markers, import paths, the oracle and (for gpu tests) the engine."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "cosyvoice.cpp_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def orc():
    from oracle.oracle import oracle

    return oracle()


@pytest.fixture(scope="session")
def eng():
    """The engine library; on a GPU run a missing build is an error, not a skip."""
    import cvattn

    return cvattn.lib()


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test collected but no GPU is visible")
    torch.cuda.init()
    return torch.device("cuda:0")


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
