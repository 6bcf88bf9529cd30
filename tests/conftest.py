"""Shared test setup. Tests marked `gpu` need an MI355X; everything else runs on the CPU.

GPU tests fail (they do not skip) when no HIP device is visible, so a GPU run can never pass
without the kernels having run.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and liblema_hip.so")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def hip():
    """The built library on a visible GPU; builds it first if it is missing or stale."""
    import torch
    from latest_exact_match_attention_amd import build, _lib
    assert torch.cuda.is_available(), "GPU tests need a visible HIP device"
    build.ensure_built()
    _lib.lib()
    torch.cuda.init()
    return _lib


@pytest.fixture
def dev(hip):
    import torch
    return torch.device("cuda", 0)
