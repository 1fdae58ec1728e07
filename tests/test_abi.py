"""The C ABI library: it loads, exports every entry point include/forge_hip.h declares, the
ctypes signatures cover exactly those, and host-side argument errors come back as status codes
(no GPU needed: nothing here launches a kernel)."""
import ctypes
import re

import pytest


def declared_symbols():
    from forge_hip import _lib
    text = _lib.HEADER_PATH.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(fh):
    lib = fh.load()
    names = declared_symbols()
    assert len(names) >= 20
    for nm in names:
        assert hasattr(lib, nm), nm


def test_ctypes_signatures_match_header(fh):
    from forge_hip import _lib
    assert sorted(_lib.SIGNATURES) == declared_symbols()


def test_abi_version(fh):
    assert fh.load().fh_abi_version() == 3


def test_null_context_is_an_argument_error(fh):
    lib = fh.load()
    assert lib.fh_sync(None) == fh.FH_EINVAL
    assert b"null context" in lib.fh_last_error()
    assert lib.fh_sort_pairs(None, None, None, 0, 8) == fh.FH_EINVAL


def test_create_argument_errors(fh):
    lib = fh.load()
    out = ctypes.c_void_p()
    assert lib.fh_create(0, 0, 10, None, ctypes.byref(out)) == fh.FH_EINVAL
    assert lib.fh_create(0, 10, 10, None, None) == fh.FH_EINVAL
    assert lib.fh_create(0, (1 << 30) + 1, 10, None, ctypes.byref(out)) == fh.FH_ERANGE


def test_create_without_gpu_reports_nodev(fh):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present")
    out = ctypes.c_void_p()
    rc = fh.load().fh_create(0, 16, 16, None, ctypes.byref(out))
    assert rc == fh.FH_ENODEV and not out.value
    with pytest.raises(fh.ForgeError) as e:
        fh.Context(16, 16)
    assert e.value.code == fh.FH_ENODEV


def test_product_path_has_no_oracle_dependency():
    """The package and the library never reference the CPU oracle (no fallback path)."""
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent / "forge-gpu_amd"
    for p in list(root.rglob("*.py")) + list(root.rglob("*.hip")) + list(root.rglob("*.hpp")):
        text = p.read_text()
        assert "oracle" not in text.lower() or p.name == "build.py", p


def test_sort_digit_layout(fh):
    """Digit layout of a sort (the library's digits_for): two 10-bit passes for 17..20-bit keys
    below 8,388,608 pairs, 8-bit passes otherwise; bench.py counts passes with it."""
    lay = fh.RadixSorter.digit_layout
    assert lay(20, 1 << 20) == (10, 2)       # c3: 10^6 cells
    assert lay(17, 100) == (10, 2)
    assert lay(20, (1 << 22) - 1) == (10, 2)
    assert lay(20, 1 << 22) == (10, 2)        # c2: 82^3 cells, 4,194,304 points
    assert lay(20, (1 << 23) - 1) == (10, 2)
    assert lay(20, 1 << 23) == (8, 3)         # larger sorts keep 8-bit digits
    assert lay(16, 1 << 20) == (8, 2)         # c0: 40^3 cells
    assert lay(21, 1 << 20) == (8, 3)
    assert lay(32, 1 << 24) == (8, 4)         # c1
    assert lay(1, 10) == (8, 1)
