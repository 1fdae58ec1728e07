"""fh_sort_pairs_noalloc (no counterpart in the reference: fh_sort_pairs for callers that
cannot allocate) against the existing entry point fh_sort_pairs, bit for bit, on two calls in
a row -- the second with a smaller input, so it runs on the scratch the first one left -- and
against numpy's stable argsort; plus its argument errors."""
import ctypes

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
    assert max_n == 1_048_576  # FH_NOALLOC_MAX_N


def test_noalloc_sort_arguments(fh, gpu_ctx):
    lib = fh.load()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    k = torch.zeros(8, dtype=torch.int32, device="cuda")
    p = ctypes.c_void_p(k.data_ptr())
    assert lib.fh_sort_pairs_noalloc(s, p, p, 1_048_577, 32) == fh.FH_ERANGE
    assert b"exceeds" in lib.fh_last_error()
    assert lib.fh_sort_pairs_noalloc(s, p, p, 8, 0) == fh.FH_EINVAL
    assert lib.fh_sort_pairs_noalloc(s, p, p, 8, 33) == fh.FH_EINVAL
    assert lib.fh_sort_pairs_noalloc(s, None, None, 8, 32) == fh.FH_EINVAL
    assert lib.fh_sort_pairs_noalloc(s, None, None, 0, 32) == fh.FH_OK
    assert lib.fh_sort_pairs_noalloc(s, p, p, 1, 32) == fh.FH_OK
