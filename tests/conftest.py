"""Shared fixtures.  GPU tests carry @pytest.mark.gpu; everything else runs on CPU."""
from __future__ import annotations

import pathlib
import sys

import pytest

REPO = pathlib.Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

import __graft_entry__ as entry  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def race():
    """The package (race-attention-kernel_amd/) imported as race_attention_kernel_amd."""
    return entry.load_package()


@pytest.fixture(scope="session")
def oracle():
    """The CPU oracle (oracle/oracle.py); built on first use if needed."""
    mod = entry.load_oracle()
    mod.build()
    return mod


@pytest.fixture(scope="session")
def ext(race):
    from race_attention_kernel_amd import _lib

    return _lib.ext()


@pytest.fixture(scope="session")
def cuda():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return torch.device("cuda:0")
