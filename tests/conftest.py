"""pytest setup: import paths, the `gpu` marker and shared fixtures.

`-m "not gpu"` runs on any host (oracle checks, host logic, C-ABI loading);
`-m gpu` needs a ROCm device and fails -- never skips -- without one.
"""

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO / "diff-gpt_amd", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libdgattn.so")


@pytest.fixture(scope="session")
def dev():
    import torch

    assert torch.cuda.is_available(), "gpu-marked test run without a visible ROCm device"
    from diff_gpt import _native

    _native.lib()  # loud failure when the HIP library is missing
    return torch.device("cuda:0")
