"""Writes tests/golden/reference_kats.json: the known-answer vectors of the reference's own tests
for this path, transcribed as data (inputs and the outputs those tests assert), plus the brute-
force answers that the reference tests leave implicit.

Sources (huaying/forge-gpu, read as text):
  tests/radix_sort_test.rs:14-48     test_radix_sort_small      (16 keys, 4 bits)
  tests/radix_sort_test.rs:51-91     test_radix_sort_medium     (xorshift32 seed 12345, 20 bits)
  tests/radix_sort_test.rs:94-137    test_radix_sort_compare_cpu_reference (seed 42, 16 bits)
  tests/radix_sort_test.rs:139-171   test_find_cell_boundaries
  tests/hashgrid_test.rs:6-36        test_hashgrid_basic
  tests/hashgrid_test.rs:38-88       test_hashgrid_uniform_distribution
Run: python tests/golden/make_golden.py   (numpy only; nothing from the reference is executed)
"""
import json
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "reference_kats.json"
S = 0xFFFFFFFF


def xorshift32_keys(seed, n, mask):
    """The key stream of radix_sort_test.rs:60-66 / :102-108."""
    s = seed
    out = []
    for _ in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out.append(s & mask)
    return out


def brute_neighbors(pos, q, r):
    p = np.asarray(pos, np.float32)
    q = np.asarray(q, np.float32)
    d = p - q
    dist = (d[:, 0] * d[:, 0] + d[:, 1] * d[:, 1]) + d[:, 2] * d[:, 2]
    return [int(i) for i in np.nonzero(dist <= np.float32(r) * np.float32(r))[0]]


def main():
    small_keys = [15, 3, 7, 1, 9, 0, 12, 5, 8, 2, 14, 6, 11, 4, 13, 10]
    order = sorted(range(16), key=lambda i: small_keys[i])
    kats = {
        "radix_sort_small": {
            "source": "tests/radix_sort_test.rs:20-28",
            "keys": small_keys, "vals": list(range(16)), "num_bits": 4,
            "sorted_keys": sorted(small_keys), "sorted_vals": order,
        },
        "radix_sort_medium": {
            "source": "tests/radix_sort_test.rs:57-73",
            "xorshift_seed": 12345, "n": 10000, "mask": 0xFFFFF, "num_bits": 20,
            "first_keys": xorshift32_keys(12345, 8, 0xFFFFF),
        },
        "radix_sort_compare_cpu": {
            "source": "tests/radix_sort_test.rs:100-120",
            "xorshift_seed": 42, "n": 5000, "mask": 0xFFFF, "num_bits": 16,
            "first_keys": xorshift32_keys(42, 8, 0xFFFF),
        },
        "find_cell_boundaries": {
            "source": "tests/radix_sort_test.rs:145-168",
            "sorted": [0, 0, 1, 1, 1, 3, 3, 5], "num_cells": 8,
            "start": [0, 2, S, 5, S, 7, S, S], "end": [2, 5, 0, 7, 0, 8, 0, 0],
            "asserted_by_reference": {"start": [0, 1, 2, 3, 5], "end": [0, 1, 2, 3, 5]},
        },
    }
    basic_pos = [[5.0, 5.0, 5.0], [5.1, 5.0, 5.0], [5.5, 5.5, 5.5], [9.0, 9.0, 9.0]]
    kats["hashgrid_basic"] = {
        "source": "tests/hashgrid_test.rs:9-33",
        "cell_size": 1.0, "dims": [10, 10, 10], "origin": [0.0, 0.0, 0.0],
        "positions": basic_pos, "query": basic_pos[0], "radius": 1.0,
        "must_contain": [0, 1, 2], "must_not_contain": [3],
        "neighbors": brute_neighbors(basic_pos, basic_pos[0], 1.0),
    }
    uni = [[(i % 10) + 0.5, ((i // 10) % 10) + 0.5, (i // 100) + 0.5] for i in range(1000)]
    nb = brute_neighbors(uni, [5.0, 5.0, 5.0], 1.5)
    kats["hashgrid_uniform"] = {
        "source": "tests/hashgrid_test.rs:42-85",
        "cell_size": 2.0, "dims": [5, 5, 5], "origin": [0.0, 0.0, 0.0],
        "positions": "lattice (i%10+0.5, (i/10)%10+0.5, i/100+0.5), i < 1000",
        "query": [5.0, 5.0, 5.0], "radius": 1.5, "reference_asserts_at_least": 4,
        "neighbors_sorted": sorted(nb), "count": len(nb),
    }
    OUT.write_text(json.dumps(kats, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
