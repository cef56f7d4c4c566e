"""Test setup: the package path, the ``gpu`` marker, and device helpers.

CPU tests (``-m "not gpu"``) pin the oracle and the host logic and check that the C-ABI library loads and exports
every declared symbol. GPU tests (``-m gpu``) run the HIP kernels through that C ABI and compare them with the
oracle on the same seeded inputs.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "lean-vllm_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def gpu_ready() -> bool:
    import torch

    if not torch.cuda.is_available():
        return False
    from lvattn import MI355XAttention

    return MI355XAttention.is_available()


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; fails (not skips) on a machine with a GPU whose library is missing, so nothing passes
    silently."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from lvattn import _capi

    _capi.load()  # raises if liblvattn.so is missing
    return torch.device("cuda:0")
