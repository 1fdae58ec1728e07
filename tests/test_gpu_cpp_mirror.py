"""The C++ host mirror (include/forge_hip.hpp) running the reference's hash-grid and radix-sort
tests, a pipeline step, graph replay, resident substeps, CSR cell ranges from sorted keys, the
standalone force pass and the streaming frames on the GPU (binary built by
__graft_entry__.build())."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu
BIN = Path(__file__).resolve().parent.parent / "forge-gpu_amd" / "_build" / "test_mirror"


def test_cpp_mirror_reference_tests():
    assert BIN.exists(), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("PASS ") == 11
