"""GPU parity of the SPH modules (C ABI fh_sph_fused, fh_sph_density, fh_gravity,
fh_integrate, fh_box_collider) against the oracle, one Pipeline::step from identical inputs.
Bar: densities and positions within rel 1e-4; accelerations
("forces") within 1e-4 * sum_j |pair terms| per component plus the terms' sensitivity to a
float32 rounding of the pair distances, with the reference acceleration and both scales
computed in fp64 (or_sph_force_f64)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
REL = 1e-4


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def fields_from(fh, cfg, vel=None):
    f = fh.FieldSet(cfg.n)
    for nm, a in (("pos_x", cfg.x), ("pos_y", cfg.y), ("pos_z", cfg.z)):
        f.f32_fields[nm] = dev(a)
    for q, nm in enumerate(("vel_x", "vel_y", "vel_z")):
        f.f32_fields[nm] = dev(vel[q]) if vel is not None else torch.zeros(cfg.n, device="cuda")
    return f


def sph_pipeline(fh, cfg, fuse=True, accel=None):
    p = fh.Pipeline(fuse_epilogue=fuse)
    m = fh.SphFusedModule(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                          cfg.rest_density, cfg.viscosity)
    m.accel = accel
    p.add(m)
    p.add(fh.GravityModule(*cfg.gravity))
    p.add(fh.IntegrateModule())
    p.add(fh.BoxColliderModule(*cfg.box_min, *cfg.box_max, cfg.restitution))
    return p


def rel_err(a, b):
    return np.abs(a - b) / np.maximum(np.abs(b), 1e-30)


def set_mode(fh, f, cfg, mode):
    """fast: default work split (below 2^18 particles: items of more than 32 candidates per
    particle split into 8 parts); fastlarge: the default split of larger systems (192
    candidates, 4 parts) at any size; heavy: every (sub-tile, slab) item split into 4
    single-wave parts whose partials are added afterwards; light: none of them (one wavefront per item, shared
    stream); heavy8: as heavy, with 8 parts per item (FH_OPT_HEAVY_PARTS) instead of 4; spill,
    spill8: as heavy and heavy8 with 5 partial-sum slots (FH_OPT_HEAVY_SLOTS), so nearly every
    item is walked without slots (k_density_pass's part-0 wave, k_force_spill); subcell, subcell2, subcell8: as fast with the cells
    ordered by 4, 2 or 8 sub-cells per axis (FH_OPT_SUBCELL), so that heavy items skip far
    candidate chunks and compact the others to their near candidates;
    subheavy: every item heavy, with 4 sub-cells per axis; subspill: as subheavy with 5
    partial-sum slots (the slot-less walks with chunk culling); direct: every item walked lane by
    lane; exact: the bit-exact passes."""
    ctx = f.context(cfg.num_cells)
    heavy = {"heavy": 1, "heavy8": 1, "spill": 1, "spill8": 1, "subheavy": 1, "subspill": 1}
    ctx.set_option(fh.FH_OPT_SPH_EXACT, 1 if mode == "exact" else 0)
    ctx.set_option(fh.FH_OPT_HEAVY_WORK, heavy.get(mode, 1 << 30 if mode == "light" else
                                                   192 if mode == "fastlarge" else 0))
    ctx.set_option(fh.FH_OPT_DIRECT_ITEMS,
                   0 if mode in heavy or mode == "light" else 2 if mode == "direct" else 1)
    ctx.set_option(fh.FH_OPT_HEAVY_PARTS, 8 if mode in ("heavy8", "spill8") else
                   4 if mode in heavy or mode == "fastlarge" else 0)
    ctx.set_option(fh.FH_OPT_HEAVY_SLOTS, 5 if mode in ("spill", "spill8", "subspill") else 0)
    ctx.set_option(fh.FH_OPT_SUBCELL,
                   {"subcell": 4, "subcell2": 2, "subcell8": 8, "subheavy": 4,
                    "subspill": 4}.get(mode, 0))


def check_step(fh, oracle, cfg, vel=None, fuse=True, mode="fast", visible=None):
    """One step through the pipeline against the oracle.  visible: particle indices whose
    acceleration must be resolvable by the bound (median |a64| >= 100 x 1e-4 sum|terms|, over
    all particles and over these), so that the term under test cannot hide in the tolerance."""
    accel = torch.zeros((3, cfg.n), dtype=torch.float32, device="cuda")
    f = fields_from(fh, cfg, vel)
    set_mode(fh, f, cfg, mode)
    p = sph_pipeline(fh, cfg, fuse=fuse, accel=accel)
    torch.cuda.synchronize()
    p.step(f, cfg.dt)
    set_mode(fh, f, cfg, "fast")
    got = {k: f.f32_fields[k].cpu().numpy() for k in f.f32_fields}
    return assert_oracle_step(oracle, cfg, (cfg.x, cfg.y, cfg.z), vel, got,
                              accel.cpu().numpy(), exact=mode == "exact", visible=visible)


def assert_oracle_step(oracle, cfg, pos, vel, got, gacc, exact=False, visible=None):
    """`got` (fields after one substep) and `gacc` (its accelerations) against one oracle step
    (or_sph_step) from positions `pos` and velocities `vel`, particle by particle:
      density            |d - d_ref| <= 1e-4 |d_ref|
      acceleration       |a - a64| <= 1e-4 sum_j |pair terms| + sens  (fp64 reference)
      velocity           |v - v_ref| <= 1e-4 |v_ref| + dt * (the acceleration bound)
      position           |x - x_ref| <= 1e-4 |x_ref| + dt^2 * (the acceleration bound)
    sens (or_sph_force_f64) is the change of the pair terms under a float32 rounding of the pair
    distances: a pair near r = h has a factor h - r that cancels, so any float32 evaluation of
    it (the float32 oracle's included) is off by more than 1e-4 of the term, and a particle
    whose only neighbours sit there has nothing else in its sum.
    v = v0 + a dt + g dt and x = x0 + v dt, hence the dt and dt^2 terms.  A particle whose
    unclamped position lies within that bound of a box wall has an ill-conditioned clamp
    decision (reflected or not) and is left out of the field checks (the count is returned).
    exact: every output bit-identical to the oracle."""
    x, y, z = (np.ascontiguousarray(a, dtype=np.float32) for a in pos)
    v0 = [np.ascontiguousarray(a, dtype=np.float32) for a in vel] if vel is not None \
        else [np.zeros(cfg.n, np.float32)] * 3
    prm = oracle.sph_params(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                            cfg.rest_density, cfg.viscosity)
    args = (cfg.gravity, cfg.box_min, cfg.box_max, cfg.restitution, x, y, z, *v0, cfg.dt)
    ox, oy, oz, ovx, ovy, ovz, orho, oacc = oracle.sph_step(prm, 7, *args)
    assert rel_err(got["density"], orho).max() <= REL
    ocs, osi, _ = oracle.hashgrid_build(x, y, z, cfg.cell_size, (0, 0, 0), cfg.dims)
    a64, s64, e64 = oracle.sph_force_f64(prm, x, y, z, *v0, orho, ocs, osi)
    ga = gacc.astype(np.float64)
    atol = REL * s64 + e64 + 1e-30
    bad = np.abs(ga - a64) > atol
    assert not bad.any(), (int(bad.any(0).sum()), float((np.abs(ga - a64) / atol).max()))
    if visible is not None:
        ratio = np.abs(a64) / atol
        assert np.median(ratio) >= 100 and np.median(ratio[:, visible]) >= 100, \
            (np.median(ratio), np.median(ratio[:, visible]))
    pre = oracle.sph_step(prm, 3, *args)  # the same step without the box
    amb = np.zeros(cfg.n, bool)
    for a, o in enumerate(pre[:3]):
        ptol = REL * np.abs(o) + cfg.dt * cfg.dt * atol[a]
        amb |= (np.abs(o - cfg.box_min[a]) <= ptol) | (np.abs(o - cfg.box_max[a]) <= ptol)
    ok = ~amb
    for a, (k, o) in enumerate((("pos_x", ox), ("pos_y", oy), ("pos_z", oz))):
        tol = REL * np.abs(o) + cfg.dt * cfg.dt * atol[a]
        assert np.all((np.abs(got[k] - o) <= tol)[ok]), k
    for a, (k, o) in enumerate((("vel_x", ovx), ("vel_y", ovy), ("vel_z", ovz))):
        tol = REL * np.abs(o) + cfg.dt * atol[a]
        assert np.all((np.abs(got[k] - o) <= tol)[ok]), k
    fr = {k: float(np.mean(got[k] == o)) for k, o in
          (("density", orho), ("pos_x", ox), ("pos_y", oy), ("pos_z", oz), ("vel_x", ovx),
           ("vel_y", ovy), ("vel_z", ovz))}
    fr["accel"] = float(np.mean(gacc == oacc))
    fr["ambiguous_clamps"] = int(amb.sum())
    if exact:
        # reference float expressions in the reference order: bit-identical to the oracle
        assert all(fr[k] == 1.0 for k in fr if k != "ambiguous_clamps"), fr
    return fr


@pytest.mark.parametrize("mode", ["fast", "exact"])
def test_c0_step1_matches_oracle(fh, gpu_ctx, oracle, mode):
    from forge_hip import workloads
    cfg = workloads.config0()
    print(f"c0 step 1 ({mode})", flush=True)
    exact = check_step(fh, oracle, cfg, mode=mode)
    print("bit-exact fractions", exact)


@pytest.mark.parametrize("mode", ["fast", "fastlarge", "exact", "heavy", "heavy8", "spill",
                                  "subcell", "subheavy", "light", "direct"])
def test_step_with_velocities_matches_oracle(fh, gpu_ctx, oracle, mode):
    """v != 0 exercises the viscosity term (zero at c0's initial state)."""
    from forge_hip import workloads
    cfg = workloads.small_sph(n=20_000, cols=24)
    rng = np.random.default_rng(5)
    vel = [rng.uniform(-0.5, 0.5, cfg.n).astype(np.float32) for _ in range(3)]
    exact = check_step(fh, oracle, cfg, vel, mode=mode)
    print("bit-exact fractions", exact)


def test_c3_step1_matches_oracle(fh, gpu_ctx, oracle):
    """configs[3] at full size (1,048,576 particles), first substep, fast passes."""
    from forge_hip import workloads
    cfg = workloads.config3()
    print("c3 step 1", flush=True)
    exact = check_step(fh, oracle, cfg)
    print("bit-exact fractions", exact)


@pytest.mark.parametrize("mode", ["fast", "fastlarge", "heavy", "heavy8", "spill", "spill8",
                                  "subcell", "subcell2", "subcell8", "subheavy", "subspill",
                                  "light", "direct"])
def test_dense_clumps_match_oracle(fh, gpu_ctx, oracle, mode):
    """Hundreds of particles per cell and particles pinned to the walls (the state c3 reaches
    after a few substeps): many staging chunks per row and empty / skipped rows."""
    from forge_hip import workloads
    cfg = workloads.small_sph(n=30_000, cols=24)
    rng = np.random.default_rng(21)
    k = cfg.n // 3
    cfg.x[:k] = rng.uniform(0.0, 0.03, k).astype(np.float32)
    cfg.y[:k] = 0.0
    cfg.z[:k] = rng.uniform(0.0, 0.05, k).astype(np.float32)
    cfg.x[k:k + 500] = 1.0
    cfg.y[k:k + 500] = 1.0
    cfg.z[k:k + 500] = 1.0
    vel = [rng.uniform(-1, 1, cfg.n).astype(np.float32) for _ in range(3)]
    print(f"dense clumps ({mode})", flush=True)
    exact = check_step(fh, oracle, cfg, vel, mode=mode)
    print("bit-exact fractions", exact)


def colocated_cfg(n=40_000, seed=33):
    """Clumps of particles at bitwise-identical positions (the box corners of c3 hold ~5600
    each): cells of >= 64 such particles are computed once by their first particle."""
    from forge_hip import workloads
    cfg = workloads.small_sph(n=n, cols=24)
    rng = np.random.default_rng(seed)
    spots = [((0.0, 0.0, 0.0), 5600), ((1.0, 1.0, 1.0), 1000), ((0.3, 0.41, 0.27), 200),
             ((0.6, 0.2, 0.7), 65), ((0.62, 0.52, 0.12), 64), ((0.2, 0.8, 0.5), 63)]
    at = 0
    for (x, y, z), k in spots:
        cfg.x[at:at + k] = x
        cfg.y[at:at + k] = y
        cfg.z[at:at + k] = z
        at += k
    # 200 particles at one point but one of them 1 ulp away: that cell must not be collapsed
    cfg.x[at:at + 200] = 0.45
    cfg.y[at:at + 200] = 0.55
    cfg.z[at:at + 200] = 0.65
    cfg.x[at + 137] = np.nextafter(np.float32(0.45), np.float32(1.0))
    at += 200
    # shuffle so clump members are spread over the particle order
    perm = rng.permutation(cfg.n)
    for a in ("x", "y", "z"):
        setattr(cfg, a, np.ascontiguousarray(getattr(cfg, a)[perm]))
    # A cell of 1000 (in an empty part of the box) whose sorted run holds one point at both
    # ends and 271 distinct points in the middle (run slots 250..520): the middle sample and
    # the middle slot are not in the group, which is found from another sample.  The run
    # order is the particle order (stable sort), so the 1000 are taken in index order from
    # former lattice particles.
    idx = np.nonzero(perm >= at)[0][:1000]
    mid = np.zeros(1000, bool)
    mid[250:521] = True
    cfg.x[idx] = np.float32(0.905)
    cfg.y[idx] = np.float32(0.505)
    cfg.z[idx] = np.float32(0.305)
    cfg.x[idx[mid]] = np.float32(0.905) + np.arange(1, 272, dtype=np.float32) * np.float32(1e-5)
    vel =[rng.uniform(-1, 1, cfg.n).astype(np.float32) for _ in range(3)]
    return cfg, vel


@pytest.mark.parametrize("mode", ["fast", "fastlarge", "heavy", "heavy8", "spill", "spill8",
                                  "subcell", "subcell8", "subheavy", "subspill", "light",
                                  "direct"])
def test_colocated_cells_match_oracle(fh, gpu_ctx, oracle, mode):
    cfg, vel = colocated_cfg()
    print(f"co-located cells ({mode})", flush=True)
    exact = check_step(fh, oracle, cfg, vel, mode=mode)
    print("bit-exact fractions", exact)


def outside_cfg():
    """Particles the grid does not hold as they are: NaN / +inf / -inf coordinates, a clump of
    50 at x ~ -0.2 (clamped into the cells of x = 0, within h of each other and of no particle
    inside), one at x = -0.004 within h of an inside particle, and two beyond the far corner of
    the grid (x, y, z ~ 1.4)."""
    from forge_hip import workloads
    cfg = workloads.small_sph(n=20_000, cols=24)
    rng = np.random.default_rng(41)
    cfg.x[0] = np.nan
    cfg.y[1] = np.inf
    cfg.z[2] = -np.inf
    cfg.x[3:53] = (-0.2 + rng.uniform(-0.004, 0.004, 50)).astype(np.float32)
    cfg.y[3:53] = (0.3 + rng.uniform(-0.004, 0.004, 50)).astype(np.float32)
    cfg.z[3:53] = (0.2 + rng.uniform(-0.004, 0.004, 50)).astype(np.float32)
    inside = int(np.argmin(cfg.x[60:])) + 60  # the particle nearest the x = 0 face
    cfg.x[53] = np.float32(-0.004)
    cfg.y[53] = cfg.y[inside]
    cfg.z[53] = cfg.z[inside] + np.float32(0.003)
    cfg.x[54:56] = np.float32(1.4)
    cfg.y[54:56] = np.float32(1.41)
    cfg.z[54:56] = np.array([1.4, 1.405], np.float32)
    vel = [rng.uniform(-0.5, 0.5, cfg.n).astype(np.float32) for _ in range(3)]
    return cfg, vel


@pytest.mark.parametrize("mode", ["fast", "exact", "subcell", "subheavy", "heavy", "light",
                                  "direct"])
def test_nonfinite_and_outside_positions_match_oracle(fh, gpu_ctx, oracle, mode):
    """One fused step over outside_cfg against the oracle: every output field has NaN and
    +-inf in the same places as the oracle's; the three non-finite particles have no neighbour
    (density 0, no force); the particles with finite inputs meet the one-step bar of
    assert_oracle_step (densities rel 1e-4, accelerations against the fp64 sums, velocities and
    positions except where the box's clamp decision is ill-conditioned); exact: every finite
    output bit-identical."""
    cfg, vel = outside_cfg()
    print(f"non-finite and outside positions ({mode})", flush=True)
    accel = torch.zeros((3, cfg.n), dtype=torch.float32, device="cuda")
    f = fields_from(fh, cfg, vel)
    set_mode(fh, f, cfg, mode)
    p = sph_pipeline(fh, cfg, accel=accel)
    torch.cuda.synchronize()
    try:
        p.step(f, cfg.dt)
    finally:
        set_mode(fh, f, cfg, "fast")
    got = {k: f.f32_fields[k].cpu().numpy() for k in f.f32_fields}
    gacc = accel.cpu().numpy()
    prm = oracle.sph_params(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                            cfg.rest_density, cfg.viscosity)
    out = oracle.sph_step(prm, 7, cfg.gravity, cfg.box_min, cfg.box_max, cfg.restitution,
                          cfg.x, cfg.y, cfg.z, *vel, cfg.dt)
    names = ("pos_x", "pos_y", "pos_z", "vel_x", "vel_y", "vel_z", "density")
    ref = dict(zip(names, out[:7]))
    for k in names:
        assert np.array_equal(np.isnan(got[k]), np.isnan(ref[k])), k
        assert np.array_equal(np.isinf(got[k]), np.isinf(ref[k])), k
    assert np.array_equal(np.isnan(gacc), np.isnan(out[7]))
    fin = np.isfinite(cfg.x) & np.isfinite(cfg.y) & np.isfinite(cfg.z)
    assert (~fin).sum() == 3
    # the non-finite particles: no neighbours, so density 0 and no force, as in the oracle
    assert np.all(got["density"][~fin] == 0.0) and np.all(ref["density"][~fin] == 0.0)
    assert np.all(gacc[:, ~fin] == 0.0)
    assert rel_err(got["density"][fin], ref["density"][fin]).max() <= REL
    ocs, osi, _ = oracle.hashgrid_build(cfg.x, cfg.y, cfg.z, cfg.cell_size, (0, 0, 0), cfg.dims)
    a64, s64, e64 = oracle.sph_force_f64(prm, cfg.x, cfg.y, cfg.z, *vel, ref["density"], ocs, osi)
    atol = REL * s64 + e64 + 1e-30
    ga = gacc.astype(np.float64)
    assert np.all((np.abs(ga - a64) <= atol)[:, fin])
    # the outside clump and the particle beside the x = 0 face do have neighbours
    assert np.all(got["density"][3:54] > 0.0)
    pre = oracle.sph_step(prm, 3, cfg.gravity, cfg.box_min, cfg.box_max, cfg.restitution,
                          cfg.x, cfg.y, cfg.z, *vel, cfg.dt)  # the same step without the box
    ok = fin.copy()
    for a, o in enumerate(pre[:3]):
        ptol = REL * np.abs(o) + cfg.dt * cfg.dt * atol[a]
        ok &= ~((np.abs(o - cfg.box_min[a]) <= ptol) | (np.abs(o - cfg.box_max[a]) <= ptol))
    for a, k in enumerate(("pos_x", "pos_y", "pos_z")):
        tol = REL * np.abs(ref[k]) + cfg.dt * cfg.dt * atol[a]
        assert np.all((np.abs(got[k] - ref[k]) <= tol)[ok]), k
    for a, k in enumerate(("vel_x", "vel_y", "vel_z")):
        tol = REL * np.abs(ref[k]) + cfg.dt * atol[a]
        assert np.all((np.abs(got[k] - ref[k]) <= tol)[ok]), k
    print(f"finite particles checked {int(ok.sum())} of {int(fin.sum())} (ambiguous clamps "
          f"{int((fin & ~ok).sum())})", flush=True)
    if mode == "exact":
        for k in names:
            assert np.array_equal(got[k][fin], ref[k][fin]), k
        assert np.array_equal(gacc[:, fin], out[7][:, fin])


def interior_groups_cfg(seed=36):
    """Co-located groups inside the lattice block (x, y in [0, 0.3), z in [0, 0.87)): every
    group's 27 cells hold lattice particles, the z +-1 slabs included, and every member has a
    velocity of its own.  Returns the config, the velocities and the members' indices."""
    from forge_hip import workloads
    cfg = workloads.small_sph(n=40_000, cols=24)
    rng = np.random.default_rng(seed)
    spots = [((0.1, 0.15, 0.3), 400), ((0.2, 0.08, 0.55), 120), ((0.13, 0.22, 0.7), 64)]
    at = cfg.n
    members = []
    for (x, y, z), k in spots:  # taken from the top layers, so the block below stays whole
        cfg.x[at - k:at], cfg.y[at - k:at], cfg.z[at - k:at] = x, y, z
        members.append(np.arange(at - k, at))
        at -= k
    perm = rng.permutation(cfg.n)
    for a in ("x", "y", "z"):
        setattr(cfg, a, np.ascontiguousarray(getattr(cfg, a)[perm]))
    members = np.argsort(perm)[np.concatenate(members)]
    vel = [rng.uniform(-1, 1, cfg.n).astype(np.float32) for _ in range(3)]
    return cfg, vel, members


def viscosity_cfg(case):
    """gas_constant = 0: the pressure term vanishes and the acceleration is the viscosity term
    alone (with the reference's constants the pressure term is ~10^4 times larger, so the
    viscosity term is invisible within the force bound)."""
    from forge_hip import workloads
    if case == "lattice":
        cfg = workloads.small_sph(n=20_000, cols=24)
        rng = np.random.default_rng(5)
        vel = [rng.uniform(-0.5, 0.5, cfg.n).astype(np.float32) for _ in range(3)]
        visible = np.arange(cfg.n)
    elif case == "groups":
        cfg, vel, visible = interior_groups_cfg()
    else:  # the corner and stand-alone groups, members with distinct velocities
        cfg, vel = colocated_cfg(seed=37)
        visible = np.arange(cfg.n)
    cfg.gas_constant = 0.0
    return cfg, vel, visible


@pytest.mark.parametrize("case", ["lattice", "groups", "colocated"])
@pytest.mark.parametrize("mode", ["fast", "fastlarge", "exact", "heavy", "heavy8", "subheavy",
                                  "light", "direct"])
def test_viscosity_without_pressure_matches_oracle(fh, gpu_ctx, oracle, case, mode):
    """The fused force's viscosity half (sph_fused.rs:617-623) on its own, in every work split:
    plain lattice particles, and members of co-located groups, which are finished from their
    representative with the viscosity weight of all three z-slabs."""
    cfg, vel, visible = viscosity_cfg(case)
    print(f"viscosity without pressure: {case} ({mode})", flush=True)
    exact = check_step(fh, oracle, cfg, vel, mode=mode, visible=visible)
    print("bit-exact fractions", exact)


def test_colocated_density_module_matches_oracle(fh, gpu_ctx, oracle):
    cfg, _ = colocated_cfg(seed=34)
    f = fields_from(fh, cfg, None)
    p = fh.Pipeline()
    p.add(fh.SphDensityModule(cfg.h, cfg.cell_size, cfg.dims, cfg.mass))
    torch.cuda.synchronize()
    p.step(f, cfg.dt)
    prm = oracle.sph_params(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                            cfg.rest_density, cfg.viscosity)
    ocs, osi, _ = oracle.hashgrid_build(cfg.x, cfg.y, cfg.z, cfg.cell_size, (0, 0, 0), cfg.dims)
    orho = oracle.sph_density(prm, cfg.x, cfg.y, cfg.z, ocs, osi)
    assert rel_err(f.f32_fields["density"].cpu().numpy(), orho).max() <= REL


def test_fused_epilogue_equals_separate_modules(fh, gpu_ctx):
    from forge_hip import workloads
    cfg = workloads.small_sph(n=8192)
    rng = np.random.default_rng(9)
    vel = [rng.uniform(-1, 1, cfg.n).astype(np.float32) for _ in range(3)]
    outs = []
    for fuse in (True, False):
        f = fields_from(fh, cfg, vel)
        p = sph_pipeline(fh, cfg, fuse=fuse)
        torch.cuda.synchronize()
        for _ in range(3):
            p.step(f, cfg.dt)
        outs.append({k: v.cpu().numpy() for k, v in f.f32_fields.items()})
    for k in outs[0]:
        assert np.array_equal(outs[0][k], outs[1][k]), k


@pytest.mark.parametrize("resident,case", [(True, "small"), (False, "small"), (True, "c3"),
                                           (True, "c3_subcell")])
def test_graph_replay_matches_eager(fh, gpu_ctx, resident, case):
    """10 captured substeps replayed twice == the same 10 substeps run eagerly twice, bit for
    bit; each replay is checked after eager work and synchronisation in between (graph nodes
    must not go stale).  resident: one fh_sph_fused_steps call of 10 substeps; otherwise 10
    fh_sph_fused calls.  c3: the full 1M-particle dam break (co-located corner groups, heavy
    and transposed items, both streams), whose heavy-list order varies from run to run while
    every item's sums must not.  c3_subcell: the same with 4 sub-cells per axis."""
    from forge_hip import workloads
    cfg = workloads.small_sph(n=16384, cols=32) if case == "small" else workloads.config3()
    print(f"graph replay {case} resident={resident}", flush=True)
    f_e = fields_from(fh, cfg)
    f_g = fields_from(fh, cfg)
    p_e = sph_pipeline(fh, cfg)
    p_g = sph_pipeline(fh, cfg)
    p_e.resident = p_g.resident = resident
    ctx = f_g.context(cfg.num_cells)
    ctx.set_option(fh.FH_OPT_SUBCELL, 4 if case == "c3_subcell" else 0)
    try:
        torch.cuda.synchronize()
        p_g.capture(f_g, cfg.dt, 10)
        for rep in range(2):
            p_e.run(f_e, cfg.dt, 10)
            p_g.replay(1)
            f_g.context().sync()
            for k in f_e.f32_fields:
                assert torch.equal(f_e.f32_fields[k], f_g.f32_fields[k]), (rep, k)
    finally:
        ctx.set_option(fh.FH_OPT_SUBCELL, 0)


def test_density_module_matches_oracle(fh, gpu_ctx, oracle):
    from forge_hip import workloads
    cfg = workloads.config0()
    f = fields_from(fh, cfg)
    m = fh.SphDensityModule(cfg.h, cfg.cell_size, cfg.dims, cfg.mass)
    torch.cuda.synchronize()
    m.execute(f, cfg.dt)
    f.context().sync()
    ocs, osi, _ = oracle.hashgrid_build(cfg.x, cfg.y, cfg.z, cfg.cell_size, (0, 0, 0), cfg.dims)
    prm = oracle.sph_params(cfg.h, cfg.cell_size, cfg.dims, cfg.mass)
    orho = oracle.sph_density(prm, cfg.x, cfg.y, cfg.z, ocs, osi)
    assert rel_err(f.f32_fields["density"].cpu().numpy(), orho).max() <= REL


def test_standalone_modules_match_oracle(fh, gpu_ctx, oracle):
    rng = np.random.default_rng(1)
    n = 10_000
    s = [rng.uniform(-0.2, 1.2, n).astype(np.float32) for _ in range(3)] + \
        [rng.uniform(-3, 3, n).astype(np.float32) for _ in range(3)]
    s[3][:7] = [np.nan, np.inf, -np.inf, np.nan, 1.0, 0.0, -0.0]  # integrate's non-finite guard
    f = fh.FieldSet(n)
    names = ["pos_x", "pos_y", "pos_z", "vel_x", "vel_y", "vel_z"]
    for nm, a in zip(names, s):
        f.f32_fields[nm] = dev(a)
    g, dt = (0.5, -9.81, 0.25), 1e-3
    mn, mx, e = (0.0, 0.05, 0.0), (1.0, 0.95, 0.9), 0.3
    torch.cuda.synchronize()
    fh.GravityModule(*g).execute(f, dt)
    fh.IntegrateModule().execute(f, dt)
    fh.BoxColliderModule(*mn, *mx, e).execute(f, dt)
    f.context().sync()
    v = oracle.gravity(s[3], s[4], s[5], g, dt)
    st = oracle.integrate(s[0], s[1], s[2], v[0], v[1], v[2], dt)
    st = oracle.box_collider(*st, mn, mx, e)
    for nm, o in zip(names, st):
        gpu = f.f32_fields[nm].cpu().numpy()
        assert np.array_equal(gpu, o), nm


@pytest.mark.parametrize("parts,sub,work", [(4, 0, 0), (8, 0, 0), (8, 4, 0), (8, 8, 384)])
def test_c4_skewed_density_and_force_match_oracle(fh, gpu_ctx, oracle, parts, sub, work):
    """configs[4] at full size (8,388,608 particles, 64 Gaussian clumps + 10 % uniform, cells of
    0 to ~27,000 particles): one HashGrid build (bit-exact), then one fused SPH pass.  The full
    CPU passes would take ~1.3e11 candidate tests each, so the oracle evaluates a sample: 4096
    random particles, 512 of the densest cell and 512 of the sparsest occupied cells.  Density
    is checked against or_sph_density_at (rel 1e-4); the acceleration against
    or_sph_force_f64_at evaluated on the GPU's densities (themselves checked on the sample),
    within 1e-4 * sum|pair terms|.  Random velocities make the viscosity term non-zero.
    parts: wavefronts per heavy item (FH_OPT_HEAVY_PARTS); sub: sub-cells per axis
    (FH_OPT_SUBCELL); work: candidates per particle above which an item is split
    (FH_OPT_HEAVY_WORK, 0: the default); (8, 8, 384) is the bench's setting, which also gives
    every item a partial-sum slot (FH_OPT_HEAVY_SLOTS); the others keep the default slots, one
    per 8 items, so that most heavy items of this clumped workload are walked without one."""
    from forge_hip import workloads
    cfg = workloads.config4()
    n = cfg.n
    print("c4 build", flush=True)
    grid = fh.HashGrid(cfg.cell_size, cfg.dims, (0.0, 0.0, 0.0), n, ctx=gpu_ctx)
    P = (dev(cfg.x), dev(cfg.y), dev(cfg.z))
    grid.build(P)
    ocs, osi, _ = oracle.hashgrid_build(cfg.x, cfg.y, cfg.z, cfg.cell_size, (0, 0, 0), cfg.dims)
    assert np.array_equal(fh.to_u32(grid.cell_start), ocs)
    assert np.array_equal(fh.to_u32(grid.sorted_indices), osi)
    del grid, P
    occ = np.diff(ocs.astype(np.int64))
    rng = np.random.default_rng(44)
    vel = [rng.uniform(-1, 1, n).astype(np.float32) for _ in range(3)]
    accel = torch.zeros((3, n), dtype=torch.float32, device="cuda")
    f = fields_from(fh, cfg, vel)
    p = fh.Pipeline()
    m = fh.SphFusedModule(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                          cfg.rest_density, cfg.viscosity)
    m.accel = accel
    p.add(m)
    torch.cuda.synchronize()
    print(f"c4 fused pass ({parts} parts, {sub} sub-cells, work {work}): max occupancy "
          f"{occ.max()}, p99 {np.percentile(occ, 99):.0f}", flush=True)
    ctx = f.context(cfg.num_cells)
    ctx.set_option(fh.FH_OPT_HEAVY_PARTS, parts)
    ctx.set_option(fh.FH_OPT_SUBCELL, sub)
    ctx.set_option(fh.FH_OPT_HEAVY_WORK, work)
    ctx.set_option(fh.FH_OPT_HEAVY_SLOTS, 2**31 - 1 if work == 384 else 0)
    try:
        p.step(f, cfg.dt)
    finally:
        ctx.set_option(fh.FH_OPT_HEAVY_PARTS, 0)
        ctx.set_option(fh.FH_OPT_SUBCELL, 0)
        ctx.set_option(fh.FH_OPT_HEAVY_WORK, 0)
        ctx.set_option(fh.FH_OPT_HEAVY_SLOTS, 0)
    rho = f.f32_fields["density"].cpu().numpy()
    acc = accel.cpu().numpy().astype(np.float64)
    dense = int(np.argmax(occ))
    sparse_cells = np.nonzero(occ == 1)[0][:512]
    which = np.unique(np.concatenate([
        rng.choice(n, 4096, replace=False),
        osi[ocs[dense]:ocs[dense] + 512],
        osi[ocs[sparse_cells]]])).astype(np.uint32)
    prm = oracle.sph_params(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                            cfg.rest_density, cfg.viscosity)
    orho = oracle.sph_density_at(prm, cfg.x, cfg.y, cfg.z, ocs, osi, which)
    assert rel_err(rho[which], orho).max() <= REL
    a64, s64, e64 = oracle.sph_force_f64_at(prm, cfg.x, cfg.y, cfg.z, *vel, rho, ocs, osi,
                                            which)
    assert np.all(np.abs(acc[:, which] - a64) <= REL * s64 + e64 + 1e-30)
    print(f"c4: {which.size} particles checked, density max rel "
          f"{rel_err(rho[which], orho).max():.3g}")


def test_wide_rows_light_streams_match_oracle(fh, gpu_ctx, oracle):
    """Light items whose candidate streams may span more than 65,536 sorted slots: a 2048 x 4 x 4
    grid with ~20 uniform particles per cell (655,360), so the rows y - 1 and y + 1 of a slab lie
    ~82,000 sorted slots apart and the plan's bound on every stream (its first particle's cell
    - 1 - nx to its last one's + 1 + nx) exceeds the 16-bit offsets: no stream is kept, and each
    pass rebuilds its own.  One fused pass against the oracle on a sample: 4096 random particles
    and the 1024 first of a middle row (densities rel 1e-4; accelerations against the fp64
    sums, as for configs[4])."""
    from forge_hip import workloads
    nx, ny, nz, per = 2048, 4, 4, 20
    n = nx * ny * nz * per
    h = 0.01
    rng = np.random.default_rng(58)
    x = rng.uniform(0.0, nx * h, n).astype(np.float32)
    y = rng.uniform(0.0, ny * h, n).astype(np.float32)
    z = rng.uniform(0.0, nz * h, n).astype(np.float32)
    cfg = workloads.SphConfig("wide", n, x, y, z, h=h, cell_size=h, dims=(nx, ny, nz), mass=1e-3)
    vel = [rng.uniform(-1, 1, n).astype(np.float32) for _ in range(3)]
    accel = torch.zeros((3, n), dtype=torch.float32, device="cuda")
    f = fields_from(fh, cfg, vel)
    p = fh.Pipeline()
    m = fh.SphFusedModule(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                          cfg.rest_density, cfg.viscosity)
    m.accel = accel
    p.add(m)
    torch.cuda.synchronize()
    print("wide rows: fused pass", flush=True)
    p.step(f, cfg.dt)
    rho = f.f32_fields["density"].cpu().numpy()
    acc = accel.cpu().numpy().astype(np.float64)
    ocs, osi, _ = oracle.hashgrid_build(x, y, z, cfg.cell_size, (0, 0, 0), cfg.dims)
    row = nx // 2 + nx * (1 + ny * 2)  # cell (nx / 2, 1, 2): a middle row of a middle plane
    which = np.unique(np.concatenate([rng.choice(n, 4096, replace=False),
                                      osi[ocs[row]:ocs[row] + 1024]])).astype(np.uint32)
    prm = oracle.sph_params(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                            cfg.rest_density, cfg.viscosity)
    orho = oracle.sph_density_at(prm, x, y, z, ocs, osi, which)
    assert rel_err(rho[which], orho).max() <= REL
    a64, s64, e64 = oracle.sph_force_f64_at(prm, x, y, z, *vel, rho, ocs, osi, which)
    assert np.all(np.abs(acc[:, which] - a64) <= REL * s64 + e64 + 1e-30)
    print(f"wide rows: {which.size} particles checked", flush=True)


@pytest.mark.parametrize("case", ["small", "colocated"])
def test_one_resident_substep_is_fh_sph_fused(fh, gpu_ctx, case):
    """fh_sph_fused_steps with steps = 1 is fh_sph_fused, bit for bit."""
    from forge_hip import workloads
    if case == "small":
        cfg = workloads.small_sph(n=20_000, cols=24)
        rng = np.random.default_rng(8)
        vel = [rng.uniform(-0.5, 0.5, cfg.n).astype(np.float32) for _ in range(3)]
    else:
        cfg, vel = colocated_cfg(seed=35)
    f1, f2 = fields_from(fh, cfg, vel), fields_from(fh, cfg, vel)
    m = sph_pipeline(fh, cfg)._fused_plan()[0]
    torch.cuda.synchronize()
    m.execute(f1, cfg.dt)
    m.execute_steps(f2, cfg.dt, 1)
    f1.context().sync()
    for k in f1.f32_fields:
        assert torch.equal(f1.f32_fields[k], f2.f32_fields[k]), k


def resident_case(case):
    from forge_hip import workloads
    if case == "small":
        cfg = workloads.small_sph(n=20_000, cols=24)
        rng = np.random.default_rng(8)
        return cfg, [rng.uniform(-0.5, 0.5, cfg.n).astype(np.float32) for _ in range(3)], 4
    if case == "colocated":
        cfg, vel = colocated_cfg(seed=35)
        return cfg, vel, 3
    if case == "c0":
        return workloads.config0(), None, 2
    if case == "c3":
        return workloads.config3(), None, 2
    cfg, vel, _ = viscosity_cfg("groups" if case == "groups_k0" else "lattice")
    return cfg, vel, 4


@pytest.mark.parametrize("case,mode", [("small", "fast"), ("colocated", "fast"), ("c0", "fast"),
                                       ("lattice_k0", "fast"), ("groups_k0", "fast"),
                                       ("c3", "fast"), ("small", "subheavy"),
                                       ("colocated", "subcell"), ("groups_k0", "subheavy"),
                                       ("c3", "subcell")])
def test_resident_substeps_match_oracle(fh, gpu_ctx, oracle, case, mode):
    """Resident substeps (fh_sph_fused_steps: the state stays in sorted order on the device
    between substeps, sorted by the previous substep's slots) against the oracle, particle by
    particle.  A call of k substeps repeats the first k - 1 substeps of the call of k - 1
    bit for bit, so substep k is checked as one oracle step (or_sph_step) from the fields the
    (k-1)-substep call returned, at the one-step bar, for k = 1 .. K.  Every substep after the
    first runs resident.  c3: the full 1,048,576-particle dam break, whose second substep
    (resident) already moves most particles to other cells.  _k0 cases: gas_constant = 0 (the viscosity term alone, non-chaotic
    motion), where the K-substep result is also compared with K chained oracle steps from the
    initial fields, within K times the one-step bound.  mode: the work split (set_mode); the
    sub-cell modes carry the sub-cell order from substep to substep in the resident keys."""
    cfg, vel, K = resident_case(case)
    print(f"resident substeps vs oracle: {case} ({mode}) n={cfg.n} K={K}", flush=True)
    states = [({"pos_x": cfg.x, "pos_y": cfg.y, "pos_z": cfg.z}, vel)]
    for k in range(1, K + 1):
        acc = torch.zeros((3, cfg.n), dtype=torch.float32, device="cuda")
        f = fields_from(fh, cfg, vel)
        p = sph_pipeline(fh, cfg, accel=acc)
        p.resident = True
        set_mode(fh, f, cfg, mode)
        torch.cuda.synchronize()
        try:
            p.run(f, cfg.dt, k)
        finally:
            set_mode(fh, f, cfg, "fast")
        got = {nm: t.cpu().numpy() for nm, t in f.f32_fields.items()}
        prev, pvel = states[-1]
        fr = assert_oracle_step(oracle, cfg, (prev["pos_x"], prev["pos_y"], prev["pos_z"]),
                                pvel, got, acc.cpu().numpy())
        print(f"  substep {k}: bit-exact fractions {fr}", flush=True)
        states.append((got, [got["vel_x"], got["vel_y"], got["vel_z"]]))
    if cfg.gas_constant == 0.0:
        prm = oracle.sph_params(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                                cfg.rest_density, cfg.viscosity)
        st = [cfg.x.copy(), cfg.y.copy(), cfg.z.copy()] + [v.copy() for v in vel]
        vtol = np.zeros((3, cfg.n))
        for _ in range(K):
            ocs, osi, _ = oracle.hashgrid_build(*st[:3], cfg.cell_size, (0, 0, 0), cfg.dims)
            out = oracle.sph_step(prm, 7, cfg.gravity, cfg.box_min, cfg.box_max,
                                  cfg.restitution, *st, cfg.dt)
            _, s64, e64 = oracle.sph_force_f64(prm, *st, out[6], ocs, osi)
            vtol += cfg.dt * (REL * s64 + e64)
            st = list(out[:6])
        got = states[-1][0]
        for a, nm in enumerate(("vel_x", "vel_y", "vel_z")):
            tol = K * (REL * np.abs(st[3 + a]) + vtol[a]) + 1e-30
            assert np.all(np.abs(got[nm] - st[3 + a]) <= tol), nm
        for a, nm in enumerate(("pos_x", "pos_y", "pos_z")):
            tol = K * (REL * np.abs(st[a]) + cfg.dt * vtol[a]) + 1e-30
            assert np.all(np.abs(got[nm] - st[a]) <= tol), nm


def test_fused_steps_edge_cases(fh, gpu_ctx):
    """fh_sph_fused_steps: steps = 0 is an error; n = 0 is a no-op; with FH_OPT_SPH_EXACT the
    call is `steps` separate exact substeps, bit for bit."""
    import ctypes
    from forge_hip import _lib, workloads
    from forge_hip.modules import _sph_params
    from forge_hip.runtime import ptr
    cfg = workloads.small_sph(n=6000, cols=16)
    m = sph_pipeline(fh, cfg)._fused_plan()[0]
    f = fields_from(fh, cfg)
    m.prepare(f)
    ctx = f.context(cfg.num_cells)
    lib = _lib.load()
    px, py, pz = f.pos()
    vx, vy, vz = f.vel()
    args = [ctx.handle, ctypes.byref(_sph_params(m)), ctypes.byref(m.epilogue)] + \
        [ptr(t) for t in (px, py, pz, vx, vy, vz, f.f32_fields["density"])] + [None]
    assert lib.fh_sph_fused_steps(*args, cfg.n, cfg.dt, 0) == fh.FH_EINVAL
    assert lib.fh_sph_fused_steps(*args, 0, cfg.dt, 3) == fh.FH_OK
    ctx.sync()
    # exact mode: one call of 3 substeps == 3 calls
    f1, f2 = fields_from(fh, cfg), fields_from(fh, cfg)
    for ff in (f1, f2):
        m.prepare(ff)
        ff.context(cfg.num_cells).set_option(fh.FH_OPT_SPH_EXACT, 1)
    torch.cuda.synchronize()
    m.execute_steps(f1, cfg.dt, 3)
    for _ in range(3):
        m.execute(f2, cfg.dt)
    f1.context().sync()
    f2.context().sync()
    for k in f1.f32_fields:
        assert torch.equal(f1.f32_fields[k], f2.f32_fields[k]), k
    for ff in (f1, f2):
        ff.context(cfg.num_cells).set_option(fh.FH_OPT_SPH_EXACT, 0)


def test_heavy_parts_option(fh, gpu_ctx):
    """FH_OPT_HEAVY_PARTS takes 0 (default), 4 or 8; other values are refused."""
    for v in (0, 4, 8):
        gpu_ctx.set_option(fh.FH_OPT_HEAVY_PARTS, v)
    for bad in (1, 3, 16, -1):
        with pytest.raises(fh.ForgeError):
            gpu_ctx.set_option(fh.FH_OPT_HEAVY_PARTS, bad)
    gpu_ctx.set_option(fh.FH_OPT_HEAVY_PARTS, 0)


def test_subcell_option(fh, gpu_ctx):
    """FH_OPT_SUBCELL takes 0 (default), 2, 4 or 8; other values are refused."""
    for v in (0, 2, 4, 8):
        gpu_ctx.set_option(fh.FH_OPT_SUBCELL, v)
    for bad in (1, 3, 16, -1):
        with pytest.raises(fh.ForgeError):
            gpu_ctx.set_option(fh.FH_OPT_SUBCELL, bad)
    gpu_ctx.set_option(fh.FH_OPT_SUBCELL, 0)


def test_heavy_slots_option(fh, gpu_ctx):
    """FH_OPT_HEAVY_SLOTS: a negative count is refused; more slots than items give every item
    one, a cap shrinks the context's scratch by its partial-sum buffer, and 0 restores the
    default: one slot per 8 items in a context of 2^18 particles or more (24 bytes per particle
    of max_n), one per item below.  A context for 2^20 particles then takes at most 300 bytes
    per particle beside its cells."""
    default = gpu_ctx.scratch_bytes
    with pytest.raises(fh.ForgeError):
        gpu_ctx.set_option(fh.FH_OPT_HEAVY_SLOTS, -1)
    gpu_ctx.set_option(fh.FH_OPT_HEAVY_SLOTS, 2**31 - 1)
    full = gpu_ctx.scratch_bytes
    gpu_ctx.set_option(fh.FH_OPT_HEAVY_SLOTS, 1)
    one = gpu_ctx.scratch_bytes
    items = slots_per_context(gpu_ctx.max_n)
    slot = (full - one) // (items - 1)
    assert (full - one) % (items - 1) == 0 and slot in (4 * 4 * 64 * 4, 8 * 4 * 64 * 4)
    assert default - one == (items // 8 - 1) * slot
    gpu_ctx.set_option(fh.FH_OPT_HEAVY_SLOTS, 3)
    gpu_ctx.set_option(fh.FH_OPT_HEAVY_SLOTS, 0)
    assert gpu_ctx.scratch_bytes == default
    big = fh.Context(max_n=1 << 20, max_cells=1)
    try:
        assert big.scratch_bytes <= 300 * (1 << 20), big.scratch_bytes / (1 << 20)
    finally:
        big.close()
    small = fh.Context(max_n=1 << 17, max_cells=1)
    try:  # every item has a slot (8 parts of 4 KB per 3 items of 64 particles)
        base = small.scratch_bytes
        small.set_option(fh.FH_OPT_HEAVY_SLOTS, 2**31 - 1)
        assert small.scratch_bytes == base
    finally:
        small.close()


def slots_per_context(max_n):
    """Heavy-list entries of a context, a slot each at most: 8 lists of
    3 * 8 * ceil(ceil(max_n / 512) / 8) entries (a plan workgroup of 512 particles lists up to
    24 items, on one of 8 lists)."""
    return 8 * 24 * -(-(-(-max_n // 512)) // 8)


@pytest.mark.parametrize("case", ["colocated", "c3"])
def test_heavy_slot_cap_is_bit_identical(fh, gpu_ctx, case):
    """With a few partial-sum slots (FH_OPT_HEAVY_SLOTS) most heavy items are walked part after
    part without slots (the density pass's part-0 wave, the force pass's spill kernel), the parts
    added in the order the slotted items' are: three
    substeps equal the uncapped ones bit for bit, for the default split, for every item heavy
    with 4 and 8 parts, and for every item heavy with 4 sub-cells per axis (the culling
    instantiations of both kernels).  A graph captured with a cap replays to the eager fields, and a
    later change of the cap drops the context's graph: the replay is refused rather than run on
    the freed buffer.  c3: the 1M-particle dam break (co-located corner groups, transposed
    items)."""
    from forge_hip import workloads
    if case == "c3":
        cfg, vel = workloads.config3(), None
    else:
        cfg, vel = colocated_cfg()
    for mode, cap in (("fast", 3), ("heavy", 1), ("heavy8", 17), ("subheavy", 2)):
        print(f"heavy slot cap {case} {mode} cap={cap}", flush=True)
        outs = []
        for slots in (2**31 - 1, cap):
            f = fields_from(fh, cfg, vel)
            p = sph_pipeline(fh, cfg)
            set_mode(fh, f, cfg, mode)
            f.context(cfg.num_cells).set_option(fh.FH_OPT_HEAVY_SLOTS, slots)
            torch.cuda.synchronize()
            try:
                p.run(f, cfg.dt, 3)
            finally:
                set_mode(fh, f, cfg, "fast")
            outs.append(f.f32_fields)
        for k in outs[0]:
            assert torch.equal(outs[0][k], outs[1][k]), (mode, k)
    print(f"heavy slot cap {case}: graph", flush=True)
    f_e = fields_from(fh, cfg, vel)
    f_g = fields_from(fh, cfg, vel)
    p_e = sph_pipeline(fh, cfg)
    p_g = sph_pipeline(fh, cfg)
    ctx = f_g.context(cfg.num_cells)
    ctx.set_option(fh.FH_OPT_HEAVY_SLOTS, 2)
    try:
        torch.cuda.synchronize()
        p_g.capture(f_g, cfg.dt, 3)
        assert f_g.context(cfg.num_cells) is ctx  # the capped context, not a grown one
        for rep in range(2):
            p_e.run(f_e, cfg.dt, 3)
            p_g.replay(1)
            ctx.sync()
            for k in f_e.f32_fields:
                assert torch.equal(f_e.f32_fields[k], f_g.f32_fields[k]), (rep, k)
    finally:
        ctx.set_option(fh.FH_OPT_HEAVY_SLOTS, 0)
    with pytest.raises(fh.ForgeError) as e:
        p_g.replay(1)
    assert e.value.code == fh.FH_ESTATE
