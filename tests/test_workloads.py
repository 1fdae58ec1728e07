"""Deterministic input generation (forge_hip/workloads.py): same seed -> same bytes, pinned
digests, the lattice layouts and ranges the configurations describe.  CPU only."""
import numpy as np

from forge_hip import workloads


def test_splitmix_known_values():
    # splitmix64 of counter i with seed s: first outputs for seed 0 (published test vector of
    # the generator: 0xE220A8397B1DCDAF for the first draw of a zero-seeded stream)
    z = workloads.splitmix64(0, np.arange(1, dtype=np.uint64))
    assert int(z[0]) == 0xE220A8397B1DCDAF


def test_uniform_is_exact_and_in_range():
    u = workloads.uniform_f32(1, 0, 100_000)
    assert u.dtype == np.float32 and u.min() >= 0.0 and u.max() < 1.0
    assert np.all((u * np.float32(2**24)) == np.floor(u * np.float32(2**24)))


def test_generators_are_deterministic():
    a, b = workloads.config0(), workloads.config0()
    assert a.digest() == b.digest()
    assert a.n == 50_000 and a.mass == float(np.float32(np.float32(1000) / np.float32(50000)) * np.float32(0.001))


def test_config0_lattice_layout():
    c = workloads.config0()
    # 40 x 40 columns at spacing 0.0125, jitter 1e-3: every point inside [0, 0.5) x [0, 0.5)
    assert c.x.min() > 0 and c.x.max() < 0.5 and c.y.min() > 0 and c.y.max() < 0.5
    assert c.z.max() < 0.4  # 31 full layers + 400 points
    ix = np.floor(c.x / 0.0125).astype(int)
    assert np.array_equal(ix, np.arange(c.n) % 40)


def test_config3_shape():
    c = workloads.config3(n=1 << 16)
    assert np.array_equal(np.floor(c.x / 0.005).astype(int), np.arange(c.n) % 128)


def test_config1_keys_below_2_24():
    k, v = workloads.config1(n=1 << 16)
    assert k.max() < 2**24 and np.array_equal(v, np.arange(1 << 16, dtype=np.uint32))


def test_config4_mixture_in_unit_cube():
    c = workloads.config4(n=1 << 16, chunk=1 << 14)
    for a in (c.x, c.y, c.z):
        assert a.min() >= 0.0 and a.max() < 1.0
    cells = (np.floor(c.x / 0.01) + 100 * np.floor(c.y / 0.01) + 1e4 * np.floor(c.z / 0.01)).astype(int)
    occ = np.bincount(cells)
    assert occ.max() > 20  # skewed occupancy
