"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker of the HIP path.

Every oracle function is checked against something other than a retyping of its own formula:
the reference's known-answer tests (tests/golden/reference_kats.json), library routines (numpy's
stable argsort, searchsorted, bincount), brute force over all pairs, and closed forms of the SPH
kernels (Mueller et al. 2003: poly6 density, spiky pressure gradient, viscosity Laplacian).  The
checks are chosen so that plausible slips (a dropped self term, `<=` for `<`, a sign, a swapped
operand, an off-by-one cell) fail at least one of them.  CPU only.
"""
import json
import math
from pathlib import Path

import numpy as np
import pytest

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
PI = math.pi


def xorshift32(seed, n, mask):
    out = np.empty(n, np.uint32)
    s = seed
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = s & mask
    return out


# ---- hashing (hashgrid.rs:128-139) -----------------------------------------------------------

def test_f32_as_i32_matches_rust_semantics(oracle):
    assert oracle.f32_as_i32(float("nan")) == 0
    assert oracle.f32_as_i32(float("inf")) == 2**31 - 1
    assert oracle.f32_as_i32(float("-inf")) == -(2**31)
    assert oracle.f32_as_i32(3e9) == 2**31 - 1
    assert oracle.f32_as_i32(-3e9) == -(2**31)
    assert oracle.f32_as_i32(-2.0) == -2
    assert oracle.f32_as_i32(7.0) == 7


def test_position_to_cell_closed_forms(oracle):
    dims, o = (10, 20, 30), (0.0, 0.0, 0.0)
    # cell centres of a power-of-two cell size are exact: cell (i, j, k) -> i + 10 j + 200 k
    cs = 0.125
    for (i, j, k) in [(0, 0, 0), (9, 19, 29), (3, 7, 11), (5, 0, 29)]:
        p = ((i + 0.5) * cs, (j + 0.5) * cs, (k + 0.5) * cs)
        assert oracle.position_to_cell(p, cs, o, dims) == i + 10 * j + 200 * k
    # exact lower faces belong to the cell
    assert oracle.position_to_cell((3 * cs, 4 * cs, 5 * cs), cs, o, dims) == 3 + 40 + 1000
    # below the grid / NaN -> 0, above -> dim - 1 (clamp after the saturating cast)
    assert oracle.position_to_cell((-5.0, float("nan"), -0.0), cs, o, dims) == 0
    assert oracle.position_to_cell((1e30, float("inf"), 100.0), cs, o, dims) == 9 + 10 * 19 + 200 * 29
    assert oracle.position_to_cell((float("-inf"), 1e-30, 2.0), cs, o, dims) == 0 + 0 + 200 * 16
    # origin is subtracted before dividing
    assert oracle.position_to_cell((1.0 + 0.3, 2.0, 3.0), 0.25, (1.0, 2.0, 3.0), dims) == 1


def test_hash_of_config1_points_is_exact(oracle):
    """c1: cs = 1/256, so floor(x / cs) = floor(256 x) exactly; checked on the 24-bit mantissas."""
    from forge_hip import workloads
    n = 100_000
    m = [workloads.u32_stream(7, a, n) >> np.uint32(8) for a in range(3)]
    x, y, z = [(mm.astype(np.float64) * 2.0**-24).astype(np.float32) for mm in m]
    keys, vals = oracle.hash_cells(x, y, z, 1.0 / 256.0, (0, 0, 0), (256, 256, 256))
    exp = (m[0] >> 16) + (m[1] >> 16) * 256 + (m[2] >> 16) * 65536
    assert np.array_equal(keys, exp.astype(np.uint32))
    assert np.array_equal(vals, np.arange(n, dtype=np.uint32))


# ---- sorting (radix_sort.rs:79-220 contract) ------------------------------------------------

def test_sort_known_answer(oracle):
    kat = KATS["radix_sort_small"]
    k, v = oracle.stable_sort_pairs(kat["keys"], kat["vals"], kat["num_bits"])
    assert k.tolist() == kat["sorted_keys"] and v.tolist() == kat["sorted_vals"]


@pytest.mark.parametrize("name", ["radix_sort_medium", "radix_sort_compare_cpu"])
def test_sort_reference_streams_vs_numpy_stable(oracle, name):
    kat = KATS[name]
    keys = xorshift32(kat["xorshift_seed"], kat["n"], kat["mask"])
    assert keys[:8].tolist() == kat["first_keys"]
    vals = np.arange(kat["n"], dtype=np.uint32)
    k, v = oracle.stable_sort_pairs(keys, vals, kat["num_bits"])
    order = np.argsort(keys, kind="stable")
    assert np.array_equal(v, order.astype(np.uint32)) and np.array_equal(k, keys[order])


@pytest.mark.parametrize("bits", [1, 5, 12, 16, 31, 32])
def test_sort_masked_keys_vs_numpy(oracle, bits):
    rng = np.random.default_rng(bits)
    keys = rng.integers(0, 2**32, 20_000, dtype=np.uint64).astype(np.uint32)
    vals = rng.integers(0, 2**32, 20_000, dtype=np.uint64).astype(np.uint32)
    mask = np.uint32(0xFFFFFFFF if bits == 32 else (1 << bits) - 1)
    order = np.argsort(keys & mask, kind="stable")
    k, v = oracle.stable_sort_pairs(keys, vals, bits)
    assert np.array_equal(k, keys[order]) and np.array_equal(v, vals[order])


# ---- cell ranges ----------------------------------------------------------------------------

def test_find_cell_boundaries_known_answer(oracle):
    kat = KATS["find_cell_boundaries"]
    s, e = oracle.find_cell_boundaries(kat["sorted"], kat["num_cells"])
    assert s.tolist() == kat["start"] and e.tolist() == kat["end"]


def test_cell_ranges_vs_searchsorted(oracle):
    rng = np.random.default_rng(2)
    C = 5000
    keys = np.sort(rng.integers(0, C + 50, 40_000).astype(np.uint32))  # some keys >= C
    csr = oracle.cell_start_csr(keys, C)
    assert np.array_equal(csr, np.searchsorted(keys, np.arange(C + 1), side="left").astype(np.uint32)
                          .clip(max=int(np.searchsorted(keys, C))))
    s, e = oracle.find_cell_boundaries(keys, C)
    nonempty = csr[1:] > csr[:-1]
    assert np.array_equal(s[nonempty], csr[:-1][nonempty]) and np.array_equal(e[nonempty], csr[1:][nonempty])
    assert np.all(s[~nonempty] == 0xFFFFFFFF) and np.all(e[~nonempty] == 0)


def test_hashgrid_build_vs_library_counting_sort(oracle):
    rng = np.random.default_rng(4)
    p = rng.uniform(-0.1, 1.1, (30_000, 3)).astype(np.float32)
    cs, dims = 0.05, (20, 22, 24)
    start, sidx, cell = oracle.hashgrid_build(p[:, 0], p[:, 1], p[:, 2], cs, (0, 0, 0), dims)
    keys, _ = oracle.hash_cells(p[:, 0], p[:, 1], p[:, 2], cs, (0, 0, 0), dims)
    assert np.array_equal(cell, keys)
    C = dims[0] * dims[1] * dims[2]
    counts = np.bincount(keys, minlength=C)
    assert start[0] == 0 and np.array_equal(np.diff(start.astype(np.int64)), counts)
    assert np.array_equal(sidx, np.argsort(keys, kind="stable").astype(np.uint32))


# ---- neighbour queries (hashgrid.rs:145-193) ------------------------------------------------

def test_query_neighbors_known_answers(oracle):
    kat = KATS["hashgrid_basic"]
    p = np.asarray(kat["positions"], np.float32)
    st, si, _ = oracle.hashgrid_build(p[:, 0], p[:, 1], p[:, 2], kat["cell_size"], kat["origin"], kat["dims"])
    nb = oracle.query_neighbors(kat["query"], kat["radius"], p[:, 0], p[:, 1], p[:, 2],
                                kat["cell_size"], kat["origin"], kat["dims"], st, si)
    assert nb.tolist() == kat["neighbors"]
    kat = KATS["hashgrid_uniform"]
    i = np.arange(1000)
    p = np.stack([(i % 10) + 0.5, ((i // 10) % 10) + 0.5, (i // 100) + 0.5], 1).astype(np.float32)
    st, si, _ = oracle.hashgrid_build(p[:, 0], p[:, 1], p[:, 2], kat["cell_size"], kat["origin"], kat["dims"])
    nb = oracle.query_neighbors(kat["query"], kat["radius"], p[:, 0], p[:, 1], p[:, 2],
                                kat["cell_size"], kat["origin"], kat["dims"], st, si)
    assert sorted(nb.tolist()) == kat["neighbors_sorted"] and len(nb) == kat["count"] == 8


def brute_counts(p, r):
    d = p[None, :, :] - p[:, None, :]
    dist = (d[..., 0] * d[..., 0] + d[..., 1] * d[..., 1]) + d[..., 2] * d[..., 2]
    return dist, dist <= np.float32(r) * np.float32(r)


def test_neighbor_counts_vs_brute_force(oracle):
    rng = np.random.default_rng(8)
    n, cs, dims = 2000, 0.1, (10, 10, 10)
    p = rng.uniform(0, 1, (n, 3)).astype(np.float32)
    st, si, _ = oracle.hashgrid_build(p[:, 0], p[:, 1], p[:, 2], cs, (0, 0, 0), dims)
    r = 0.1
    cnt, w = oracle.neighbor_counts(p[:, 0], p[:, 1], p[:, 2], cs, (0, 0, 0), dims, st, si, r)
    dist, hit = brute_counts(p, r)
    assert np.array_equal(cnt, hit.sum(1).astype(np.uint32))
    c = 315.0 / (64.0 * PI * r**9)
    w64 = np.where(hit, c * (r * r - dist.astype(np.float64)) ** 3, 0.0).sum(1)
    assert np.allclose(w, w64, rtol=2e-5, atol=0)
    for q in (0, 17, 999):  # per-query lists equal the brute-force sets
        nb = oracle.query_neighbors(p[q], r, p[:, 0], p[:, 1], p[:, 2], cs, (0, 0, 0), dims, st, si)
        assert sorted(nb.tolist()) == np.nonzero(hit[q])[0].tolist()


# ---- SPH (sph_density.rs:401-461, sph_fused.rs:542-638) -------------------------------------

# parameters are float32 in the reference; the closed forms use their exact float32 values
H, MASS, K, RHO0, MU = (float(np.float32(v)) for v in (0.025, 2e-5, 2000.0, 1000.0, 0.01))


def prm(oracle, dims=(40, 40, 40)):
    return oracle.sph_params(H, H, dims, MASS, K, RHO0, MU)


def grid(oracle, x, y, z, dims=(40, 40, 40)):
    st, si, _ = oracle.hashgrid_build(x, y, z, H, (0, 0, 0), dims)
    return st, si


def poly6(r):
    return 315.0 / (64.0 * PI * H**9) * (H * H - r * r) ** 3 if r < H else 0.0


def test_density_closed_forms(oracle):
    # isolated particle: rho = m * W(0) = m * 315 / (64 pi h^3)
    x, y, z = (np.array([0.5], np.float32),) * 3
    st, si = grid(oracle, x, y, z)
    rho = oracle.sph_density(prm(oracle), x, y, z, st, si)
    assert rho[0] == pytest.approx(MASS * 315.0 / (64.0 * PI * H**3), rel=2e-6)
    # two particles at distance d in neighbouring cells: rho = m (W(0) + W(d)) each
    d = 0.6 * H
    x = np.array([0.5 - 0.01, 0.5 - 0.01 + d], np.float32)
    y = z = np.array([0.5, 0.5], np.float32)
    st, si = grid(oracle, x, y, z)
    rho = oracle.sph_density(prm(oracle), x, y, z, st, si)
    dd = float(x[1]) - float(x[0])
    assert rho == pytest.approx([MASS * (poly6(0) + poly6(dd))] * 2, rel=2e-6)
    # at distance >= h the neighbour contributes nothing (strict r^2 < h^2)
    x = np.array([0.5, 0.5 + H], np.float32)
    st, si = grid(oracle, x, y, z)
    rho = oracle.sph_density(prm(oracle), x, y, z, st, si)
    assert rho == pytest.approx([MASS * poly6(0)] * 2, rel=2e-6)


def test_density_vs_brute_force(oracle):
    rng = np.random.default_rng(12)
    p = rng.uniform(0.2, 0.5, (3000, 3)).astype(np.float32)
    st, si = grid(oracle, p[:, 0], p[:, 1], p[:, 2])
    rho = oracle.sph_density(prm(oracle), p[:, 0], p[:, 1], p[:, 2], st, si)
    d = p[None, :, :].astype(np.float64) - p[:, None, :]
    r2 = (d * d).sum(-1)
    c = 315.0 / (64.0 * PI * H**9)
    rho64 = MASS * c * np.where(r2 < H * H, (H * H - r2) ** 3, 0.0).sum(1)
    assert np.allclose(rho, rho64, rtol=5e-5)


def pair_accel(xi, xj, vi, vj, rho_i, rho_j):
    """Mueller 2003 forms as the reference applies them: pressure with the spiky gradient
    grad W = -45/(pi h^6) (h - r)^2 r_hat, symmetrised as -(m (p_i + p_j) / (2 rho_j)) grad W;
    viscosity mu m (v_j - v_i) / rho_j * lap W with lap W = 45/(pi h^6) (h - r); both / rho_i."""
    rv = np.asarray(xi, np.float64) - np.asarray(xj, np.float64)
    r = np.linalg.norm(rv)
    if not (r < H and r * r > 1e-12):
        return np.zeros(3)
    grad = -45.0 / (PI * H**6) * (H - r) ** 2 * rv / r
    pi_, pj = K * (rho_i - RHO0), K * (rho_j - RHO0)
    a_p = -MASS * (pi_ + pj) / (2.0 * rho_j) * grad
    a_v = MU * MASS * (np.asarray(vj, np.float64) - vi) / rho_j * 45.0 / (PI * H**6) * (H - r)
    return (a_p + a_v) / rho_i


def test_force_closed_forms(oracle):
    p = prm(oracle)
    # isolated particle: no force
    x = y = z = np.array([0.5], np.float32)
    st, si = grid(oracle, x, y, z)
    rho = oracle.sph_density(p, x, y, z, st, si)
    _, acc = oracle.sph_force(p, x, y, z, x * 0 + 1, y * 0, z * 0, rho, st, si, 1e-4)
    assert np.all(acc == 0)
    # two particles with velocities: against the textbook pair terms
    x = np.array([0.5, 0.512], np.float32)
    y = np.array([0.4, 0.405], np.float32)
    z = np.array([0.3, 0.296], np.float32)
    vx, vy, vz = (np.array([0.1, -0.3], np.float32), np.array([0.0, 0.2], np.float32),
                  np.array([0.5, 0.5], np.float32))
    st, si = grid(oracle, x, y, z)
    rho = oracle.sph_density(p, x, y, z, st, si)
    vout, acc = oracle.sph_force(p, x, y, z, vx, vy, vz, rho, st, si, 1e-4)
    a64, s64, _ = oracle.sph_force_f64(p, x, y, z, vx, vy, vz, rho, st, si)
    for i, j in ((0, 1), (1, 0)):
        exp = pair_accel((x[i], y[i], z[i]), (x[j], y[j], z[j]), (vx[i], vy[i], vz[i]),
                         (vx[j], vy[j], vz[j]), float(rho[i]), float(rho[j]))
        assert np.allclose(acc[:, i], exp, rtol=1e-5, atol=0)
        assert np.allclose(a64[:, i], exp, rtol=1e-12, atol=0)
        # attraction: rho << rho0 makes p negative, so particle i accelerates towards j
        # (pressure part only: compare with zero velocities)
    _, acc0 = oracle.sph_force(p, x, y, z, vx * 0, vy * 0, vz * 0, rho, st, si, 1e-4)
    d01 = np.array([x[1] - x[0], y[1] - y[0], z[1] - z[0]], np.float64)
    assert np.dot(acc0[:, 0], d01) > 0 and np.dot(acc0[:, 1], d01) < 0
    # v_out = v + a dt
    assert np.allclose(vout[0], vx + acc[0] * np.float32(1e-4), rtol=0, atol=1e-7)


def test_force_viscosity_closed_form_without_pressure(oracle):
    """gas_constant = 0 removes the pressure term, so the fused force is the viscosity term
    alone: a_i = sum_j mu m (v_j - v_i) / rho_j * 45 / (pi h^6) (h - r) / rho_i
    (sph_fused.rs:617-623).  With the reference constants the pressure term is ~10^6 times
    larger, so only this configuration pins the viscosity half of or_sph_force: a dropped
    term, a flipped sign, (v_i - v_j) for (v_j - v_i), rho_i for rho_j or a missing (h - r)
    each move every particle's acceleration by far more than rtol 1e-6."""
    p0 = oracle.sph_params(H, H, (40, 40, 40), MASS, 0.0, RHO0, MU)
    x = np.array([0.5, 0.512, 0.495, 0.507, 0.53], np.float32)
    y = np.array([0.4, 0.405, 0.391, 0.414, 0.40], np.float32)
    z = np.array([0.3, 0.296, 0.309, 0.288, 0.3], np.float32)
    vx = np.array([0.1, -0.3, 0.25, 0.7, -0.2], np.float32)
    vy = np.array([0.0, 0.2, -0.45, 0.15, 0.33], np.float32)
    vz = np.array([0.5, 0.6, -0.1, 0.05, 0.9], np.float32)
    st, si = grid(oracle, x, y, z)
    # densities chosen apart from the poly6 sums, so rho_i and rho_j cannot be exchanged
    rho = np.array([3.0, 7.5, 11.25, 5.5, 9.0], np.float32)
    _, acc = oracle.sph_force(p0, x, y, z, vx, vy, vz, rho, st, si, 1e-4)
    a64, s64, _ = oracle.sph_force_f64(p0, x, y, z, vx, vy, vz, rho, st, si)
    lap = 45.0 / (PI * H**6)
    P = np.stack([x, y, z], 1).astype(np.float64)
    V = np.stack([vx, vy, vz], 1).astype(np.float64)
    for i in range(5):
        exp = np.zeros(3)
        scale = np.zeros(3)  # sum of the terms' magnitudes (float32 rounding is relative to it)
        pairs = 0
        for j in range(5):
            r = np.linalg.norm(P[i] - P[j])
            if j != i and r < H:
                t = MU * MASS * (V[j] - V[i]) / float(rho[j]) * lap * (H - r) / float(rho[i])
                exp += t
                scale += np.abs(t)
                pairs += 1
        assert pairs >= 1
        # every component is at least 1e-3 of its scale, so flipping its sign (an error of
        # 2 |exp|), or dropping or mis-scaling a term (an error of a term's size), exceeds the
        # bound below by more than 10^3
        assert np.all(np.abs(exp) >= 1e-3 * scale), (i, exp, scale)
        assert np.all(np.abs(acc[:, i] - exp) <= 1e-6 * scale), (i, acc[:, i], exp)
        assert np.all(np.abs(a64[:, i] - exp) <= 1e-12 * scale), i
        # the fp64 error scale is the sum of the viscosity terms' magnitudes alone
        assert np.allclose(s64[:, i], scale, rtol=1e-9), i


def test_force_vs_brute_force_and_f64(oracle):
    rng = np.random.default_rng(14)
    n = 2500
    P = rng.uniform(0.3, 0.45, (n, 3)).astype(np.float32)
    V = rng.uniform(-1, 1, (n, 3)).astype(np.float32)
    p = prm(oracle)
    st, si = grid(oracle, P[:, 0], P[:, 1], P[:, 2])
    rho = oracle.sph_density(p, P[:, 0], P[:, 1], P[:, 2], st, si)
    _, acc = oracle.sph_force(p, *P.T, *V.T, rho, st, si, 1e-4)
    a64, s64, _ = oracle.sph_force_f64(p, *P.T, *V.T, rho, st, si)
    bf = np.zeros((3, n))
    for i in range(0, n, 97):  # brute force over all particles for a sample of i
        for j in range(n):
            if j != i:
                bf[:, i] += pair_accel(P[i], P[j], V[i], V[j], float(rho[i]), float(rho[j]))
        assert np.all(np.abs(bf[:, i] - a64[:, i]) <= 1e-9 * s64[:, i] + 1e-12)
        assert np.all(np.abs(acc[:, i] - a64[:, i]) <= 1e-5 * s64[:, i] + 1e-12)


def test_subset_passes_equal_the_full_passes(oracle):
    """sph_density_at / sph_force_f64_at (used where the full pass is too slow, c4) give the
    full passes' values for the listed particles, bit for bit, in any order, repeats included."""
    rng = np.random.default_rng(15)
    n = 3000
    P = rng.uniform(0.3, 0.45, (n, 3)).astype(np.float32)
    V = rng.uniform(-1, 1, (n, 3)).astype(np.float32)
    p = prm(oracle)
    st, si = grid(oracle, P[:, 0], P[:, 1], P[:, 2])
    rho = oracle.sph_density(p, *P.T, st, si)
    a64, s64, e64 = oracle.sph_force_f64(p, *P.T, *V.T, rho, st, si)
    which = np.concatenate([rng.permutation(n)[:400], [0, n - 1, 7, 7]]).astype(np.uint32)
    assert np.array_equal(oracle.sph_density_at(p, *P.T, st, si, which), rho[which])
    b64, t64, f64 = oracle.sph_force_f64_at(p, *P.T, *V.T, rho, st, si, which)
    assert np.array_equal(b64, a64[:, which]) and np.array_equal(t64, s64[:, which])
    assert np.array_equal(f64, e64[:, which])


def test_force_distance_rounding_sensitivity(oracle):
    """The third output of or_sph_force_f64: per pair, |d term / dr| * 8 * 2^-24 * r / rho_i
    with d/dr of the pressure factor (h - r)^2 / r * d taken at fixed direction d
    (-2 (h - r) / r * d) and of the viscosity factor (h - r) (-1).  Checked against the
    textbook terms of pair_accel for a two-particle pair, then as a bound: on sparse random
    particles (a few neighbours each, some near r = h, where h - r cancels), the float32
    oracle is within 1e-5 sum|terms| + sens of the fp64 values for every particle, while
    without the sensitivity some particles are not."""
    p = prm(oracle)
    u = 8.0 * 2.0**-24
    x = np.array([0.5, 0.512], np.float32)
    y = np.array([0.4, 0.405], np.float32)
    z = np.array([0.3, 0.296], np.float32)
    vx, vy, vz = (np.array([0.1, -0.3], np.float32), np.array([0.0, 0.2], np.float32),
                  np.array([0.5, 0.5], np.float32))
    st, si = grid(oracle, x, y, z)
    rho = oracle.sph_density(p, x, y, z, st, si)
    _, _, e64 = oracle.sph_force_f64(p, x, y, z, vx, vy, vz, rho, st, si)
    for i, j in ((0, 1), (1, 0)):
        d = np.array([x[i], y[i], z[i]], np.float64) - np.array([x[j], y[j], z[j]], np.float64)
        dv = np.array([vx[j], vy[j], vz[j]], np.float64) - np.array([vx[i], vy[i], vz[i]])
        r = np.linalg.norm(d)
        ri, rj = float(rho[i]), float(rho[j])
        pij = K * (ri - RHO0) + K * (rj - RHO0)
        dp = np.abs(MASS * pij / (2 * rj) * 45.0 / (PI * H**6) * 2 * (H - r) / r) * np.abs(d)
        dvv = MU * MASS / rj * 45.0 / (PI * H**6) * np.abs(dv)
        assert np.allclose(e64[:, i], (dp + dvv) * u * r / ri, rtol=1e-12, atol=0)
    # as a bound on float32 rounding
    rng = np.random.default_rng(71)
    n = 50_000
    P = (rng.uniform(0, 1, (n, 3)) * [1.0, 2.0, 0.5]).astype(np.float32)
    V = rng.uniform(-1, 1, (n, 3)).astype(np.float32)
    p2 = oracle.sph_params(H, 2 * H, (40, 80, 20), MASS, K, RHO0, MU)
    st, si, _ = oracle.hashgrid_build(*P.T, 2 * H, (0, 0, 0), (40, 80, 20))
    rho = oracle.sph_density(p2, *P.T, st, si)
    _, acc = oracle.sph_force(p2, *P.T, *V.T, rho, st, si, 1e-4)
    a64, s64, e64 = oracle.sph_force_f64(p2, *P.T, *V.T, rho, st, si)
    err = np.abs(acc - a64)
    assert np.all(err <= 1e-5 * s64 + e64)
    assert np.any(err > 1e-5 * s64)


def test_epilogue_closed_forms(oracle):
    vx, vy, vz = (np.array([1.0, np.nan, -2.0], np.float32), np.array([0.0, 1.0, np.inf], np.float32),
                  np.array([3.0, -1.0, 0.5], np.float32))
    g, dt = (0.5, -9.81, 0.0), 0.01
    v = oracle.gravity(vx, vy, vz, g, dt)
    assert v[0][0] == np.float32(1.0) + np.float32(0.5) * np.float32(dt)
    assert v[1][0] == np.float32(-9.81) * np.float32(dt)
    x = np.array([0.5, 0.5, 0.5], np.float32)
    s = oracle.integrate(x, x, x, vx, vy, vz, dt)
    assert s[3][1] == 0.0 and s[0][1] == 0.5           # NaN velocity zeroed, no motion
    assert s[4][2] == 0.0 and s[1][2] == 0.5           # inf likewise
    assert s[0][0] == np.float32(0.5) + np.float32(1.0) * np.float32(dt)
    b = oracle.box_collider(np.array([-0.1, 1.2, 0.5], np.float32), x, x,
                            np.array([-2.0, 3.0, 1.0], np.float32), vy, vz, (0, 0, 0), (1, 1, 1), 0.3)
    assert b[0].tolist() == [0.0, 1.0, 0.5]
    assert b[3][0] == np.float32(2.0) * np.float32(0.3) and b[3][1] == -np.float32(3.0) * np.float32(0.3)


def test_sph_step_is_the_module_sequence(oracle):
    from forge_hip import workloads
    cfg = workloads.small_sph(n=3000, cols=16)
    rng = np.random.default_rng(3)
    V = [rng.uniform(-1, 1, cfg.n).astype(np.float32) for _ in range(3)]
    p = oracle.sph_params(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                          cfg.rest_density, cfg.viscosity)
    out = oracle.sph_step(p, 7, cfg.gravity, cfg.box_min, cfg.box_max, cfg.restitution,
                          cfg.x, cfg.y, cfg.z, *V, cfg.dt)
    st, si = grid(oracle, cfg.x, cfg.y, cfg.z, cfg.dims)
    rho = oracle.sph_density(p, cfg.x, cfg.y, cfg.z, st, si)
    vout, acc = oracle.sph_force(p, cfg.x, cfg.y, cfg.z, *V, rho, st, si, cfg.dt)
    v = oracle.gravity(*vout, cfg.gravity, cfg.dt)
    s = oracle.integrate(cfg.x, cfg.y, cfg.z, *v, cfg.dt)
    s = oracle.box_collider(*s, cfg.box_min, cfg.box_max, cfg.restitution)
    for a, b in zip(out[:6], s):
        assert np.array_equal(a, b)
    assert np.array_equal(out[6], rho) and np.array_equal(out[7], acc)


# ---- unfused SphPressureModule / SphViscosityModule (sph_pressure.rs:28-112,
# sph_viscosity.rs:27-106) --------------------------------------------------------------------
def pair_parts(xi, xj, vi, vj, rho_i, rho_j):
    """(pressure, viscosity) accelerations of i due to j, textbook forms in float64 (Mueller
    2003: spiky gradient for pressure, viscosity Laplacian), each divided by rho_i."""
    rv = np.asarray(xi, np.float64) - np.asarray(xj, np.float64)
    r = np.linalg.norm(rv)
    if not (r < H and r * r > 1e-12):
        return np.zeros(3), np.zeros(3)
    grad = -45.0 / (PI * H**6) * (H - r) ** 2 * rv / r
    a_p = -MASS * (K * (rho_i - RHO0) + K * (rho_j - RHO0)) / (2.0 * rho_j) * grad
    a_v = MU * MASS * (np.asarray(vj, np.float64) - vi) / rho_j * 45.0 / (PI * H**6) * (H - r)
    return a_p / rho_i, a_v / rho_i


DT = float(np.float32(1e-4))


def test_unfused_closed_forms(oracle):
    p = prm(oracle)
    # isolated particle: both passes leave the velocity bit-identical
    x = y = z = np.array([0.5], np.float32)
    v = (np.array([0.25], np.float32), np.array([-1.5], np.float32), np.array([3.0], np.float32))
    st, si = grid(oracle, x, y, z)
    rho = oracle.sph_density(p, x, y, z, st, si)
    for fn in (oracle.sph_pressure, oracle.sph_viscosity):
        out = fn(p, x, y, z, *v, rho, st, si, DT)
        assert [out[c][0] for c in range(3)] == [v[c][0] for c in range(3)]
    # two particles: the velocity change over dt is the textbook pair term of each module
    x = np.array([0.5, 0.512], np.float32)
    y = np.array([0.4, 0.405], np.float32)
    z = np.array([0.3, 0.296], np.float32)
    V = np.array([[0.1, -0.3], [0.0, 0.2], [0.5, 0.5]], np.float32)
    st, si = grid(oracle, x, y, z)
    rho = oracle.sph_density(p, x, y, z, st, si)
    vp = oracle.sph_pressure(p, x, y, z, *V, rho, st, si, DT)
    vv = oracle.sph_viscosity(p, x, y, z, *V, rho, st, si, DT)
    for i, j in ((0, 1), (1, 0)):
        ep, ev = pair_parts((x[i], y[i], z[i]), (x[j], y[j], z[j]), V[:, i], V[:, j],
                            float(rho[i]), float(rho[j]))
        # v + a dt rounds to float32: compare the change against a dt within a few ulp of v
        tol = 4 * np.spacing(np.abs(V[:, i]).astype(np.float32)).astype(np.float64)
        assert np.all(np.abs((vp[:, i].astype(np.float64) - V[:, i]) - ep * DT) <= tol + 1e-6 * np.abs(ep * DT))
        assert np.all(np.abs((vv[:, i].astype(np.float64) - V[:, i]) - ev * DT) <= tol + 1e-6 * np.abs(ev * DT))
    # equal densities (symmetric pair): pressure changes are opposite, viscosity pulls together
    assert rho[0] == rho[1]
    dp = vp.astype(np.float64) - V
    assert np.allclose(dp[:, 0], -dp[:, 1], rtol=1e-3, atol=1e-12)
    dv = vv.astype(np.float64) - V
    assert np.all(dv[:, 0] * (V[:, 1] - V[:, 0]) >= 0)
    # uniform velocity field: viscosity changes nothing (v_j - v_i = 0 exactly)
    U = np.ones((3, 2), np.float32) * np.float32(0.7)
    out = oracle.sph_viscosity(p, x, y, z, *U, rho, st, si, DT)
    assert np.array_equal(out, U)
    # a neighbour whose density is below 1e-6 is skipped, and such a particle is left untouched
    rho0 = rho.copy()
    rho0[1] = 0.0
    for fn in (oracle.sph_pressure, oracle.sph_viscosity):
        out = fn(p, x, y, z, *V, rho0, st, si, DT)
        assert np.array_equal(out[:, 0], V[:, 0]) and np.array_equal(out[:, 1], V[:, 1])


def test_unfused_vs_brute_force_and_fused(oracle):
    rng = np.random.default_rng(15)
    n = 2000
    P = rng.uniform(0.3, 0.44, (n, 3)).astype(np.float32)
    V = rng.uniform(-1, 1, (n, 3)).astype(np.float32)
    p = prm(oracle)
    st, si = grid(oracle, P[:, 0], P[:, 1], P[:, 2])
    rho = oracle.sph_density(p, P[:, 0], P[:, 1], P[:, 2], st, si)
    vp = oracle.sph_pressure(p, *P.T, *V.T, rho, st, si, DT)
    vv = oracle.sph_viscosity(p, *P.T, *V.T, rho, st, si, DT)
    vf, _ = oracle.sph_force(p, *P.T, *V.T, rho, st, si, DT)
    a64, s64, _ = oracle.sph_force_f64(p, *P.T, *V.T, rho, st, si)
    # bound of a velocity change: f32 rounding of v + a dt plus 1e-5 of the term magnitudes
    vt = V.T.astype(np.float64)
    ulp = 2 * np.spacing(np.abs(V.T)).astype(np.float64)
    for i in range(0, n, 89):
        bp, bv = np.zeros(3), np.zeros(3)
        for j in range(n):
            if j != i:
                a, b = pair_parts(P[i], P[j], V[i], V[j], float(rho[i]), float(rho[j]))
                bp += a
                bv += b
        tol = ulp[:, i] + 1e-5 * s64[:, i] * DT
        assert np.all(np.abs((vp[:, i] - vt[:, i]) - bp * DT) <= tol)
        assert np.all(np.abs((vv[:, i] - vt[:, i]) - bv * DT) <= tol)
    # from the same state the two unfused changes add up to the fused pass's change
    tot = (vp.astype(np.float64) - vt) + (vv.astype(np.float64) - vt)
    assert np.all(np.abs(tot - (vf.astype(np.float64) - vt)) <= 3 * ulp + 1e-5 * s64 * DT)
