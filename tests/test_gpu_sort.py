"""GPU parity of the radix sort and cell boundaries (C ABI fh_sort_pairs,
fh_find_cell_boundaries) against the oracle and the reference's known answers.
Bar: bit-exact keys and values (stable order), tests/radix_sort_test.rs as the model."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def xorshift32(seed, n, mask):
    out = np.empty(n, np.uint32)
    s = seed
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = s & mask
    return out


def expected_plan(keys, digit_bits, passes):
    """The passes an in-place sort runs: those whose digit is not the same for every key; when
    that is exactly one of two or more passes, its neighbour runs as well (a copy), so the
    second of the two writes the caller's arrays (sort_plan in fh_sort.hip)."""
    m = (1 << digit_bits) - 1
    plan = sum(1 << p for p in range(passes)
               if np.unique((keys >> (digit_bits * p)) & m).size > 1)
    if bin(plan).count("1") == 1 and passes >= 2:
        p = plan.bit_length() - 1
        plan |= 1 << (p - 1 if p > 0 else 1)
    return plan


def gpu_sort(fh, ctx, keys, vals, bits):
    k = fh.from_u32(keys)
    v = fh.from_u32(vals)
    torch.cuda.synchronize()
    fh.RadixSorter(max(len(keys), 1), ctx=ctx).sort(k, v, len(keys), bits)
    return fh.to_u32(k), fh.to_u32(v)


def test_radix_sort_small(fh, gpu_ctx):
    kat = KATS["radix_sort_small"]
    k, v = gpu_sort(fh, gpu_ctx, kat["keys"], kat["vals"], kat["num_bits"])
    assert k.tolist() == kat["sorted_keys"]
    assert v.tolist() == kat["sorted_vals"]


@pytest.mark.parametrize("name", ["radix_sort_medium", "radix_sort_compare_cpu"])
def test_radix_sort_xorshift_streams(fh, gpu_ctx, oracle, name):
    kat = KATS[name]
    keys = xorshift32(kat["xorshift_seed"], kat["n"], kat["mask"])
    assert keys[:8].tolist() == kat["first_keys"]
    vals = np.arange(kat["n"], dtype=np.uint32)
    k, v = gpu_sort(fh, gpu_ctx, keys, vals, kat["num_bits"])
    ok, ov = oracle.stable_sort_pairs(keys, vals, kat["num_bits"])
    assert np.array_equal(k, ok) and np.array_equal(v, ov)
    assert np.all(keys[v] == k)  # key/value correspondence (radix_sort_test.rs:84-88)


@pytest.mark.parametrize("n,bits", [(0, 8), (1, 32), (2, 1), (3, 5), (4095, 12), (4096, 16),
                                    (4097, 20), (65537, 8), (100_000, 7), (100_000, 32),
                                    (1 << 20, 20), (1_000_003, 24), (2_500_000, 31),
                                    (1 << 22, 32), (5_000_011, 19),
                                    # 10-bit digits (17..20 bits below 8,388,608 keys; first
                                    # pass without look-back up to 4,194,304 keys)
                                    (8192, 17), (8193, 18), (70_000, 17), (300_000, 19),
                                    (1_000_003, 20), (4_194_303, 20), (4_194_304, 20),
                                    (4_194_305, 20), (8_388_607, 20), (8_388_608, 20)])
def test_sort_matches_oracle(fh, gpu_ctx, oracle, n, bits):
    rng = np.random.default_rng(n * 131 + bits)
    keys = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)  # high bits beyond num_bits too
    vals = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    print(f"sort n={n} bits={bits}", flush=True)
    k, v = gpu_sort(fh, gpu_ctx, keys, vals, bits)
    ok, ov = oracle.stable_sort_pairs(keys, vals, bits)
    assert np.array_equal(k, ok)
    assert np.array_equal(v, ov)


def test_sort_heavy_duplicates_is_stable(fh, gpu_ctx):
    n = 300_000
    rng = np.random.default_rng(7)
    keys = rng.integers(0, 4, n).astype(np.uint32)
    vals = np.arange(n, dtype=np.uint32)
    k, v = gpu_sort(fh, gpu_ctx, keys, vals, 32)
    exp = np.argsort(keys, kind="stable").astype(np.uint32)  # library stable sort
    assert np.array_equal(v, exp)
    assert np.array_equal(k, keys[exp])


@pytest.mark.parametrize("case", ["all_equal", "one_moving_pass", "trivial_middle_passes",
                                  "trivial_first_pass", "two_values", "only_last_pass",
                                  "only_middle_pass"])
def test_sort_skips_identity_passes(fh, gpu_ctx, oracle, case):
    """Passes whose digit is the same for every key are skipped on the device; the result must
    still be the stable sort, in place, whatever number of passes actually moved keys."""
    n = 50_000
    rng = np.random.default_rng(11)
    r = rng.integers(0, 256, n).astype(np.uint32)
    keys = {"all_equal": np.full(n, 0xA5A5A5A5, np.uint32),
            "one_moving_pass": r,                                  # bytes 1..3 are zero
            "trivial_middle_passes": r | (r[::-1] << 24),          # bytes 1, 2 zero
            "trivial_first_pass": (r << 8) | 7,                    # byte 0 constant
            "two_values": np.where(r < 128, 3, 0x70000).astype(np.uint32),
            "only_last_pass": (r << 24) | 0x00123456,              # bytes 0..2 constant
            "only_middle_pass": (r << 16) | 0x9F0000FF & 0xFF00FFFF}[case]
    vals = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    print(f"sort skip case {case}", flush=True)
    k, v = gpu_sort(fh, gpu_ctx, keys, vals, 32)
    ok, ov = oracle.stable_sort_pairs(keys, vals, 32)
    assert np.array_equal(k, ok) and np.array_equal(v, ov)
    # the device's pass plan (fh_sort_plan)
    want = expected_plan(keys, 8, 4)
    assert gpu_ctx.sort_plan() == want, (case, gpu_ctx.sort_plan(), want)


@pytest.mark.parametrize("case", ["all_equal", "low_digit_constant", "high_digit_constant",
                                  "two_values", "low_only"])
def test_sort_skips_identity_passes_wide(fh, gpu_ctx, oracle, case):
    """The same for 20-bit sorts, which run two 10-bit passes: an identity pass is skipped and
    the other one (in place) still leaves the stable sort in the caller's arrays."""
    n = 200_000
    rng = np.random.default_rng(13)
    r = rng.integers(0, 1024, n).astype(np.uint32)
    keys = {"all_equal": np.full(n, 0xBEEF5, np.uint32),
            "low_digit_constant": (r << 10) | 0x155,
            "high_digit_constant": r | (0x2AB << 10),
            "two_values": np.where(r < 512, 0x3FF, 0xFFC00).astype(np.uint32),
            "low_only": r}[case]
    keys = keys | (rng.integers(0, 4096, n).astype(np.uint32) << 20)  # bits above num_bits
    vals = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    print(f"sort wide skip case {case}", flush=True)
    k, v = gpu_sort(fh, gpu_ctx, keys, vals, 20)
    ok, ov = oracle.stable_sort_pairs(keys, vals, 20)
    assert np.array_equal(k, ok) and np.array_equal(v, ov)
    want = expected_plan(keys & 0xFFFFF, 10, 2)
    assert gpu_ctx.sort_plan() == want, (case, gpu_ctx.sort_plan(), want)


def test_sort_back_to_back_sizes(fh, gpu_ctx, oracle):
    """Consecutive sorts of different sizes on one context (look-back words are re-zeroed)."""
    rng = np.random.default_rng(5)
    for n, bits in [(1_000_000, 24), (10_000, 32), (4_200_000, 32), (300_000, 16), (8193, 9),
                    (4_194_304, 17), (1_000_000, 20), (2_000_000, 24), (50_000, 18),
                    (1_000_000, 24)]:
        keys = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
        vals = np.arange(n, dtype=np.uint32)
        k, v = gpu_sort(fh, gpu_ctx, keys, vals, bits)
        ok, ov = oracle.stable_sort_pairs(keys, vals, bits)
        assert np.array_equal(k, ok) and np.array_equal(v, ov), (n, bits)


def test_sort_config1_full(fh, gpu_ctx):
    """c1: 16,777,216 pairs of cell keys, full 32-bit stable sort, vs numpy's stable argsort."""
    from forge_hip import workloads
    keys, vals = workloads.config1()
    print("c1 sort", flush=True)
    k, v = gpu_sort(fh, gpu_ctx, keys, vals, 32)
    exp = np.argsort(keys, kind="stable").astype(np.uint32)
    assert np.array_equal(v, exp)
    assert np.array_equal(k, keys[exp])
    assert np.all(np.diff(k.astype(np.int64)) >= 0)


def test_sort_errors(fh, gpu_ctx):
    k = fh.u32_empty(16)
    v = fh.u32_empty(16)
    sorter = fh.RadixSorter(16, ctx=gpu_ctx)
    with pytest.raises(fh.ForgeError) as e:
        sorter.sort(k, v, 16, 0)
    assert e.value.code == fh.FH_EINVAL
    with pytest.raises(fh.ForgeError) as e:
        sorter.sort(k, v, 16, 33)
    assert e.value.code == fh.FH_EINVAL
    small = fh.Context(max_n=8, max_cells=8)
    with pytest.raises(fh.ForgeError) as e:
        fh.RadixSorter(1 << 20, ctx=small).sort(k, v, 16, 8)
    assert e.value.code == fh.FH_ERANGE
    small.close()


def test_find_cell_boundaries_kat(fh, gpu_ctx):
    kat = KATS["find_cell_boundaries"]
    ids = fh.from_u32(kat["sorted"])
    s = fh.u32_empty(kat["num_cells"])
    e = fh.u32_empty(kat["num_cells"])
    torch.cuda.synchronize()
    fh.find_cell_boundaries(ids, s, e, len(kat["sorted"]), kat["num_cells"], ctx=gpu_ctx)
    assert fh.to_u32(s).tolist() == kat["start"]
    assert fh.to_u32(e).tolist() == kat["end"]


def test_find_cell_boundaries_vs_oracle(fh, gpu_ctx, oracle):
    rng = np.random.default_rng(3)
    C = 50_000
    keys = np.sort(rng.integers(0, C + 100, 200_000).astype(np.uint32))  # some keys >= C
    s = fh.u32_empty(C)
    e = fh.u32_empty(C)
    ids = fh.from_u32(keys)
    torch.cuda.synchronize()
    fh.find_cell_boundaries(ids, s, e, keys.size, C, ctx=gpu_ctx)
    os_, oe = oracle.find_cell_boundaries(keys, C)
    assert np.array_equal(fh.to_u32(s), os_) and np.array_equal(fh.to_u32(e), oe)
