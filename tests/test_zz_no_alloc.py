"""fh_sort_pairs_noalloc (no counterpart in the reference: fh_sort_pairs for callers that
cannot allocate) against the existing entry point fh_sort_pairs, bit for bit, on two calls in
a row -- the second with a smaller input, so it runs on the scratch the first one left -- and
against numpy's stable argsort; captured into a graph and replayed on fresh inputs; its
argument errors; and its device-side status (fh_noalloc_status), including a look-back
failure forced from the host with a one-poll spin limit (no fault: the scatter stays in
bounds, the output is wrong and the status says so)."""
import ctypes
import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _sort_noalloc(fh, keys, vals, n, bits):
    lib = fh.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.fh_sort_pairs_noalloc(stream, ctypes.c_void_p(keys.data_ptr()),
                                   ctypes.c_void_p(vals.data_ptr()), n, bits)
    assert rc == fh.FH_OK, lib.fh_last_error()
    torch.cuda.current_stream().synchronize()


def _sort_ctx(fh, ctx, keys, vals, n, bits):
    torch.cuda.synchronize()
    fh.RadixSorter(n, ctx=ctx).sort(keys, vals, n, bits)


@pytest.mark.parametrize("first,second", [((1_048_576, 32), (70_001, 20)),
                                          ((300_000, 24), (12_345, 7)),
                                          ((1_048_576, 20), (4097, 18))])
def test_noalloc_sort_equals_fh_sort_pairs(fh, gpu_ctx, first, second):
    lib = fh.load()
    max_n = 1_048_576
    rng = np.random.default_rng(first[0] + second[0])
    for n, bits in (first, second):
        print(f"no-alloc sort n={n} bits={bits}", flush=True)
        keys = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
        keys[: n // 3] &= np.uint32(0xFF)  # runs of equal low digits: stability matters
        vals = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
        k1 = torch.from_numpy(keys.view(np.int32)).cuda()
        v1 = torch.from_numpy(vals.view(np.int32)).cuda()
        k2, v2 = k1.clone(), v1.clone()
        torch.cuda.synchronize()
        _sort_noalloc(fh, k1, v1, n, bits)
        _sort_ctx(fh, gpu_ctx, k2, v2, n, bits)
        assert torch.equal(k1, k2) and torch.equal(v1, v2)
        mask = np.uint32(0xFFFFFFFF if bits == 32 else (1 << bits) - 1)
        order = np.argsort(keys & mask, kind="stable")
        assert np.array_equal(fh.to_u32(k1), keys[order])
        assert np.array_equal(fh.to_u32(v1), vals[order])
    # no look-back gave up in these sorts
    assert lib.fh_noalloc_status(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == fh.FH_OK


def test_noalloc_sort_arguments(fh, gpu_ctx):
    lib = fh.load()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    k = torch.zeros(8, dtype=torch.int32, device="cuda")
    p = ctypes.c_void_p(k.data_ptr())
    assert lib.fh_sort_pairs_noalloc(s, p, p, 1_048_577, 32) == fh.FH_ERANGE  # MAX_N + 1
    assert b"exceeds" in lib.fh_last_error()
    assert lib.fh_sort_pairs_noalloc(s, p, p, 2**32 - 1, 32) == fh.FH_ERANGE
    assert lib.fh_sort_pairs_noalloc(s, p, p, 8, 0) == fh.FH_EINVAL
    assert lib.fh_sort_pairs_noalloc(s, p, p, 8, 33) == fh.FH_EINVAL
    assert lib.fh_sort_pairs_noalloc(s, None, None, 8, 32) == fh.FH_EINVAL
    assert lib.fh_sort_pairs_noalloc(s, None, None, 0, 32) == fh.FH_OK
    assert lib.fh_sort_pairs_noalloc(s, p, p, 1, 32) == fh.FH_OK


def test_noalloc_sort_captured_and_replayed(fh, gpu_ctx):
    """One warm call resolves the device's scratch; a second call is captured into a torch CUDA
    graph (global capture mode: any allocating or synchronising HIP call fails the capture) and
    the graph is replayed on fresh inputs, with eager work and synchronisations in between;
    every replay equals fh_sort_pairs on the same input."""
    lib = fh.load()
    n, bits = 200_003, 24
    rng = np.random.default_rng(77)
    k_in = torch.zeros(n, dtype=torch.int32, device="cuda")
    v_in = torch.zeros(n, dtype=torch.int32, device="cuda")
    warm_k = torch.from_numpy(rng.integers(0, 2**31, n).astype(np.int32)).cuda()
    warm_v = warm_k.clone()
    _sort_noalloc(fh, warm_k, warm_v, n, bits)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=s):
        rc = lib.fh_sort_pairs_noalloc(ctypes.c_void_p(s.cuda_stream),
                                       ctypes.c_void_p(k_in.data_ptr()),
                                       ctypes.c_void_p(v_in.data_ptr()), n, bits)
    assert rc == fh.FH_OK, lib.fh_last_error()
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"no-alloc graph replay {rep}", flush=True)
        keys = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
        keys[: n // 4] &= np.uint32(0xFFF)
        vals = np.arange(n, dtype=np.uint32) * np.uint32(3)
        k_in.copy_(torch.from_numpy(keys.view(np.int32)))
        v_in.copy_(torch.from_numpy(vals.view(np.int32)))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        k2 = torch.from_numpy(keys.view(np.int32)).cuda()
        v2 = torch.from_numpy(vals.view(np.int32)).cuda()
        _sort_ctx(fh, gpu_ctx, k2, v2, n, bits)
        assert torch.equal(k_in, k2) and torch.equal(v_in, v2), rep
    assert lib.fh_noalloc_status(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == fh.FH_OK


_FORCED = r"""
import ctypes, json, sys
import numpy as np, torch
sys.path.insert(0, sys.argv[1])
import forge_hip as fh
lib = fh.load()
n = 1_048_576
rng = np.random.default_rng(5)
keys = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
k = torch.from_numpy(keys.view(np.int32)).cuda()
v = torch.arange(n, dtype=torch.int32, device="cuda")
s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
out = {"sort": lib.fh_sort_pairs_noalloc(s, ctypes.c_void_p(k.data_ptr()),
                                         ctypes.c_void_p(v.data_ptr()), n, 32)}
out["status"] = lib.fh_noalloc_status(s)
out["message"] = lib.fh_last_error().decode()
out["status_again"] = lib.fh_noalloc_status(s)
out["sorted"] = bool(np.array_equal(fh.to_u32(k), np.sort(keys)))
print(json.dumps(out), flush=True)
"""


def test_noalloc_status_reports_a_forced_lookback_failure(fh):
    """A look-back that gives up is reported by fh_noalloc_status (once), not hidden behind
    FH_OK.  The failure is forced from the host: FH_DEBUG_SPIN_LIMIT=1 lets every look-back poll
    once before giving up, in a process of its own (the limit is set when that process resolves
    its scratch)."""
    pkg = str(Path(__file__).resolve().parent.parent / "forge-gpu_amd")
    env = dict(os.environ, FH_DEBUG_SPIN_LIMIT="1")
    print("forced look-back failure: subprocess, 1,048,576 pairs, spin limit 1", flush=True)
    r = subprocess.run([sys.executable, "-c", _FORCED, pkg], env=env, capture_output=True,
                       text=True, timeout=180)
    assert r.returncode == 0, r.stderr[-2000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["sort"] == fh.FH_OK  # queued fine: the failure happens on the device
    assert out["status"] == fh.FH_ESTATE, out
    assert "gave up" in out["message"]
    assert out["status_again"] == fh.FH_OK  # reported once, then cleared
    print(f"forced failure: output sorted = {out['sorted']} (expected wrong)", flush=True)
