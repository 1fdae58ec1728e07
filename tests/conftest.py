"""Test configuration: the `gpu` marker, import paths and shared fixtures.

`-m "not gpu"` runs here (no GPU): the oracle against golden vectors and closed forms, the host
logic, and the C ABI library's exports.  `-m gpu` runs on an MI355X: parity of the HIP path
against the oracle through the C ABI.
"""
import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO, REPO / "forge-gpu_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) HIP device")


@pytest.fixture(scope="session")
def oracle():
    import oracle.oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def fh():
    import forge_hip
    forge_hip.load()
    return forge_hip


@pytest.fixture(scope="session")
def gpu_ctx(fh):
    """One context for the GPU tests: room for the largest configuration's sort (c1)."""
    import torch
    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    ctx = fh.Context(max_n=16_777_216, max_cells=1_000_000)
    yield ctx
    ctx.sync()
    ctx.close()
