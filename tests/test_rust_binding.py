"""The Rust binding (forge-gpu_amd/rust/) against the C ABI it declares.

No Rust toolchain is in this image, so the crate is not compiled here; this test pins its raw
declarations to include/forge_hip.h instead: every function of the header is declared in
forge-hip-sys with the same parameter names in the same order and the same constness of every
pointer, nothing else is declared, the #define constants have the same values, and the two
#[repr(C)] structs list the header's fields in the header's order.  The safe crate must only
call declared functions.
"""
import re
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "forge_hip.h"
RUST = REPO / "forge-gpu_amd" / "rust"
SYS = RUST / "forge-hip-sys" / "src" / "lib.rs"


def _strip_c_comments(s: str) -> str:
    return re.sub(r"/\*.*?\*/", "", s, flags=re.S)


def c_functions():
    src = _strip_c_comments(HEADER.read_text())
    out = {}
    for m in re.finditer(r"\b([A-Za-z_][\w \*]*?)\s*\b(fh_\w+)\s*\(([^;{]*?)\)\s*;", src):
        name, params = m.group(2), m.group(3).strip()
        plist = []
        if params and params != "void":
            for p in params.split(","):
                p = p.strip()
                arr = p.endswith("]")
                p = re.sub(r"\[\d*\]$", "", p).strip()
                pname = re.findall(r"(\w+)$", p)[0]
                ptype = p[: -len(pname)].strip()
                is_ptr = "*" in ptype or arr
                is_const = is_ptr and ptype.startswith("const") and ptype.count("*") <= 1
                plist.append((pname, is_ptr, is_const))
        out[name] = plist
    return out


def rust_functions():
    src = SYS.read_text()
    block = re.search(r'extern "C" \{(.*?)\n\}', src, flags=re.S).group(1)
    out = {}
    for m in re.finditer(r"pub fn (fh_\w+)\s*\((.*?)\)\s*(->[^;]*)?;", block, flags=re.S):
        name, params = m.group(1), " ".join(m.group(2).split())
        plist = []
        for p in filter(None, (q.strip() for q in params.split(","))):
            pname, ptype = (q.strip() for q in p.split(":", 1))
            is_ptr = ptype.startswith("*")
            is_const = ptype.startswith("*const")
            plist.append((pname, is_ptr, is_const))
        out[name] = plist
    return out


def test_every_header_function_is_declared_with_the_same_parameters():
    c, r = c_functions(), rust_functions()
    assert len(c) >= 30, sorted(c)
    assert sorted(c) == sorted(r), (set(c) ^ set(r))
    for name, cp in c.items():
        rp = r[name]
        assert [p[0] for p in cp] == [p[0] for p in rp], name
        # pointer-ness and constness of every parameter (fixed-size C arrays are pointers)
        assert [(p[1], p[2]) for p in cp] == [(p[1], p[2]) for p in rp], name


def test_constants_match_the_header():
    defs = dict(re.findall(r"#define (FH_\w+) (-?\d+)u?\b", HEADER.read_text()))
    src = SYS.read_text()
    rs = dict(re.findall(r"pub const (FH_\w+): \w+ = (-?[\d_]+);", src))
    assert set(defs) == set(rs), set(defs) ^ set(rs)
    for k, v in defs.items():
        assert int(rs[k].replace("_", "")) == int(v), k


def test_structs_match_the_header():
    hdr = _strip_c_comments(HEADER.read_text())
    src = SYS.read_text()
    for name in ("fh_sph_params", "fh_epilogue"):
        body = re.search(r"typedef struct %s \{(.*?)\}" % name, hdr, flags=re.S).group(1)
        cf = re.findall(r"(\w+)(?:\[\d+\])?;", body)
        rbody = re.search(r"pub struct %s \{(.*?)\}" % name, src, flags=re.S).group(1)
        rf = re.findall(r"pub (\w+):", rbody)
        assert cf == rf, name
    assert "#[repr(C)]\n#[derive(Clone, Copy, Debug, Default, PartialEq)]\npub struct fh_sph_params" in src


def test_safe_crate_calls_only_declared_functions():
    declared = set(rust_functions())
    called = set()
    for f in (RUST / "forge-hip" / "src").glob("*.rs"):
        called |= set(re.findall(r"sys::(fh_\w+)\s*\(", f.read_text()))
    assert called, "the safe crate calls the C ABI"
    assert called <= declared, called - declared
    # the reference's wrappers are all there
    lib = (RUST / "forge-hip" / "src" / "lib.rs").read_text()
    for name in ("HashGrid", "RadixSorter", "find_cell_boundaries", "FieldSet", "SimModule",
                 "Pipeline", "SphFusedModule", "SphDensityModule", "SphPressureModule",
                 "SphViscosityModule", "GravityModule", "IntegrateModule", "BoxColliderModule",
                 "ForgeError", "fuse_epilogue"):
        assert re.search(r"\b%s\b" % name, lib), name
