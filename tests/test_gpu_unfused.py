"""GPU parity of the unfused SPH modules (C ABI fh_sph_pressure, fh_sph_viscosity, and the grid
that fh_sph_density leaves in the FieldSet) against the oracle.  These kernels evaluate the
reference expressions term by term in the reference's neighbour order (sph_pressure.rs:28-112,
sph_viscosity.rs:27-106), so from identical inputs every velocity is bit-identical."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def u32(t):
    return t.cpu().numpy().view(np.uint32)


def state(cfg, seed):
    rng = np.random.default_rng(seed)
    return [rng.uniform(-0.5, 0.5, cfg.n).astype(np.float32) for _ in range(3)]


def clumps():
    """Wall-pinned particles (y = 0), a clump of 300 at one point and 200 at the corner."""
    from forge_hip import workloads
    cfg = workloads.small_sph(n=30_000, cols=24)
    rng = np.random.default_rng(21)
    k = cfg.n // 3
    cfg.x[:k] = rng.uniform(0.0, 0.03, k).astype(np.float32)
    cfg.y[:k] = 0.0
    cfg.z[:k] = rng.uniform(0.0, 0.05, k).astype(np.float32)
    cfg.x[k:k + 300], cfg.y[k:k + 300], cfg.z[k:k + 300] = 0.31, 0.42, 0.27
    cfg.x[k + 300:k + 500], cfg.y[k + 300:k + 500], cfg.z[k + 300:k + 500] = 1.0, 1.0, 1.0
    return cfg


def fieldset(fh, cfg, vel):
    f = fh.FieldSet(cfg.n)
    for nm, a in (("pos_x", cfg.x), ("pos_y", cfg.y), ("pos_z", cfg.z), ("vel_x", vel[0]),
                  ("vel_y", vel[1]), ("vel_z", vel[2])):
        f.f32_fields[nm] = dev(a)
    return f


def modules(fh, cfg):
    d = fh.SphDensityModule(cfg.h, cfg.cell_size, cfg.dims, cfg.mass)
    p = fh.SphPressureModule(cfg.gas_constant, cfg.rest_density, cfg.h, cfg.cell_size, cfg.dims,
                             cfg.mass)
    v = fh.SphViscosityModule(cfg.viscosity, cfg.h, cfg.cell_size, cfg.dims, cfg.mass)
    return d, p, v


@pytest.mark.parametrize("exact", [0, 1])
def test_density_module_leaves_the_hashgrid(fh, gpu_ctx, oracle, exact):
    """cell_start / sorted_indices written by the density module equal HashGrid::build's."""
    from forge_hip import workloads
    cfg = workloads.config0()
    f = fieldset(fh, cfg, state(cfg, 1))
    f.context(cfg.num_cells).set_option(fh.FH_OPT_SPH_EXACT, exact)
    d, _, _ = modules(fh, cfg)
    torch.cuda.synchronize()
    d.execute(f, cfg.dt)
    f.context().sync()
    f.context().set_option(fh.FH_OPT_SPH_EXACT, 0)
    ocs, osi, _ = oracle.hashgrid_build(cfg.x, cfg.y, cfg.z, cfg.cell_size, (0, 0, 0), cfg.dims)
    assert np.array_equal(u32(f.u32_fields["cell_start"]), ocs)
    assert np.array_equal(u32(f.u32_fields["sorted_indices"]), osi)


@pytest.mark.parametrize("which", ["pressure", "viscosity"])
@pytest.mark.parametrize("case", ["c0", "clumps"])
def test_unfused_pass_is_bit_exact(fh, gpu_ctx, oracle, which, case):
    """One pass from the oracle's own density and grid: identical velocities."""
    from forge_hip import workloads
    cfg = workloads.config0() if case == "c0" else clumps()
    print(f"unfused {which} on {case} ({cfg.n} particles)", flush=True)
    vel = state(cfg, 2)
    ocs, osi, _ = oracle.hashgrid_build(cfg.x, cfg.y, cfg.z, cfg.cell_size, (0, 0, 0), cfg.dims)
    prm = oracle.sph_params(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                            cfg.rest_density, cfg.viscosity)
    rho = oracle.sph_density(prm, cfg.x, cfg.y, cfg.z, ocs, osi)
    rho[::97] = 0.0  # particles below the 1e-6 density cut: skipped as i and as j
    f = fieldset(fh, cfg, vel)
    f.f32_fields["density"] = dev(rho)
    f.u32_fields["cell_start"] = fh.from_u32(ocs)
    f.u32_fields["sorted_indices"] = fh.from_u32(osi)
    _, p, v = modules(fh, cfg)
    m = p if which == "pressure" else v
    ref = (oracle.sph_pressure if which == "pressure" else oracle.sph_viscosity)(
        prm, cfg.x, cfg.y, cfg.z, *vel, rho, ocs, osi, cfg.dt)
    f.context(cfg.num_cells)
    torch.cuda.synchronize()
    m.execute(f, cfg.dt)
    f.context().sync()
    for c, nm in enumerate(("vel_x", "vel_y", "vel_z")):
        got = f.f32_fields[nm].cpu().numpy()
        assert np.array_equal(got, ref[c]), nm
    assert not np.array_equal(ref[0], vel[0])  # the pass did change the state


def test_unfused_pipeline_is_bit_exact(fh, gpu_ctx, oracle):
    """density -> pressure -> viscosity -> gravity -> integrate -> box, one Pipeline::step with
    the exact density pass: the viscosity pass sees the velocities the pressure pass wrote."""
    from forge_hip import workloads
    cfg = workloads.small_sph(n=20_000, cols=24)
    vel = state(cfg, 3)
    f = fieldset(fh, cfg, vel)
    f.context(cfg.num_cells).set_option(fh.FH_OPT_SPH_EXACT, 1)
    d, p, v = modules(fh, cfg)
    pipe = fh.Pipeline()
    for m in (d, p, v, fh.GravityModule(*cfg.gravity), fh.IntegrateModule(),
              fh.BoxColliderModule(*cfg.box_min, *cfg.box_max, cfg.restitution)):
        pipe.add(m)
    torch.cuda.synchronize()
    pipe.step(f, cfg.dt)
    f.context().set_option(fh.FH_OPT_SPH_EXACT, 0)
    prm = oracle.sph_params(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                            cfg.rest_density, cfg.viscosity)
    ocs, osi, _ = oracle.hashgrid_build(cfg.x, cfg.y, cfg.z, cfg.cell_size, (0, 0, 0), cfg.dims)
    rho = oracle.sph_density(prm, cfg.x, cfg.y, cfg.z, ocs, osi)
    v1 = oracle.sph_pressure(prm, cfg.x, cfg.y, cfg.z, *vel, rho, ocs, osi, cfg.dt)
    v2 = oracle.sph_viscosity(prm, cfg.x, cfg.y, cfg.z, *v1, rho, ocs, osi, cfg.dt)
    v3 = oracle.gravity(*v2, cfg.gravity, cfg.dt)
    s = oracle.integrate(cfg.x, cfg.y, cfg.z, *v3, cfg.dt)
    s = oracle.box_collider(*s, cfg.box_min, cfg.box_max, cfg.restitution)
    assert np.array_equal(f.f32_fields["density"].cpu().numpy(), rho)
    for nm, o in zip(("pos_x", "pos_y", "pos_z", "vel_x", "vel_y", "vel_z"), s):
        assert np.array_equal(f.f32_fields[nm].cpu().numpy(), o), nm
