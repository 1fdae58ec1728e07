"""GPU parity of the module-level entry points around the fused SPH path, through the C ABI:
the standalone fused force pass over a caller's grid (fh_sph_force, sph_fused.rs:519-639), the
CSR cell_start of already-sorted keys (fh_cell_start_csr, hashgrid.rs:102-106), the binary
position frame of the streaming runner (fh_pack_frame, manifest_runner.rs:145-167 and
serve.rs:43-62), and a dam-break pipeline made by build_pipeline / init_fields
(manifest_runner.rs:192-233,322-544) against the oracle."""
import struct

import numpy as np
import pytest
import torch

from test_gpu_sph import assert_oracle_step, fields_from

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_standalone_force_pass_is_bit_exact(fh, gpu_ctx, oracle):
    """fh_sph_force over the grid and densities the density module left in the field set equals
    or_sph_force on the same inputs bit for bit (velocities and accelerations), with velocities
    so that the viscosity term is present, and with k = 0 (viscosity alone)."""
    from forge_hip import workloads
    for k in (2000.0, 0.0):
        cfg = workloads.small_sph(n=12_000, cols=20)
        cfg.gas_constant = k
        rng = np.random.default_rng(61)
        vel = [rng.uniform(-1, 1, cfg.n).astype(np.float32) for _ in range(3)]
        f = fields_from(fh, cfg, vel)
        dens = fh.SphDensityModule(cfg.h, cfg.cell_size, cfg.dims, cfg.mass)
        force = fh.SphFusedModule(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                                  cfg.rest_density, cfg.viscosity)
        force.accel = torch.zeros((3, cfg.n), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        dens.execute(f, cfg.dt)
        force.execute_force(f, cfg.dt)
        f.context().sync()
        prm = oracle.sph_params(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                                cfg.rest_density, cfg.viscosity)
        ocs, osi, _ = oracle.hashgrid_build(cfg.x, cfg.y, cfg.z, cfg.cell_size, (0, 0, 0),
                                            cfg.dims)
        rho = oracle.sph_density(prm, cfg.x, cfg.y, cfg.z, ocs, osi)
        assert np.array_equal(fh.to_u32(f.u32_fields["cell_start"]), ocs)
        assert np.array_equal(fh.to_u32(f.u32_fields["sorted_indices"]), osi)
        # the force pass reads the density module's (fast-mode) densities: give the oracle those
        grho = f.f32_fields["density"].cpu().numpy()
        assert np.all(np.abs(grho - rho) <= 1e-4 * np.abs(rho))
        vout, acc = oracle.sph_force(prm, cfg.x, cfg.y, cfg.z, *vel, grho, ocs, osi, cfg.dt)
        for a, nm in enumerate(("vel_x", "vel_y", "vel_z")):
            assert np.array_equal(f.f32_fields[nm].cpu().numpy(), vout[a]), (k, nm)
        assert np.array_equal(force.accel.cpu().numpy(), acc), k
        for nm, a in (("pos_x", cfg.x), ("pos_y", cfg.y), ("pos_z", cfg.z)):
            assert np.array_equal(f.f32_fields[nm].cpu().numpy(), a)  # positions untouched
        assert np.abs(acc).max() > 0


@pytest.mark.parametrize("n,C", [(0, 7), (1, 1), (5000, 64), (200_000, 1000), (70_000, 3)])
def test_cell_start_csr_from_sorted_keys(fh, gpu_ctx, oracle, n, C):
    """Bit-exact against the oracle's CSR (or_cell_start_csr), keys >= C included (they count
    in no cell), empty cells and runs longer than a wave's fill."""
    rng = np.random.default_rng(n + C)
    keys = np.sort(rng.integers(0, C + 3, n).astype(np.uint32))
    if n > 10:
        keys[-3:] = 0xFFFFFFFF  # far beyond the grid
        keys = np.sort(keys)
    exp = oracle.cell_start_csr(keys, C)
    got = fh.cell_start_csr(dev(keys.view(np.int32)) if n else torch.empty(0, dtype=torch.int32,
                                                                            device="cuda"),
                            n, C, ctx=gpu_ctx)
    assert np.array_equal(fh.to_u32(got), exp)
    # the same grid as HashGrid.build writes, from sorted cell ids
    if n:
        assert got[0].item() == 0 and fh.to_u32(got)[-1] == np.count_nonzero(keys < C)


def pack_reference(frame, x, y, z):
    """serve.rs:43-62 FrameBuffer::set_frame on the interleaved positions of
    manifest_runner.rs:150-159: u32 LE frame, u32 LE count, f32 LE x0 y0 z0 x1 ..."""
    pos = np.stack([x, y, z], 1).astype("<f4").ravel()
    return struct.pack("<II", frame, len(x)) + pos.tobytes()


@pytest.mark.parametrize("n", [0, 1, 333, 100_003])
def test_pack_frame_bytes(fh, gpu_ctx, n):
    rng = np.random.default_rng(n)
    x, y, z = (rng.uniform(-2, 2, n).astype(np.float32) for _ in range(3))
    if n > 2:
        x[0], y[1], z[2] = np.nan, np.inf, -0.0  # bits travel unchanged
    f = fh.FieldSet(n)
    for nm, a in (("pos_x", x), ("pos_y", y), ("pos_z", z)):
        f.f32_fields[nm] = dev(a)
    torch.cuda.synchronize()
    out = fh.pack_frame(f, 41)
    f.context().sync()
    assert out.numel() == fh.frame_bytes(n) == 8 + 12 * n
    assert out.cpu().numpy().tobytes() == pack_reference(41, x, y, z)


def test_pack_frame_counter_in_a_graph(fh, gpu_ctx):
    """With a device counter the frame number comes from it and advances on every replay of a
    captured graph; each replay is read back after eager work in between."""
    n = 4096
    rng = np.random.default_rng(3)
    x, y, z = (rng.uniform(0, 1, n).astype(np.float32) for _ in range(3))
    f = fh.FieldSet(n)
    for nm, a in (("pos_x", x), ("pos_y", y), ("pos_z", z)):
        f.f32_fields[nm] = dev(a)
    ctx = f.context()
    counter = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    out = torch.empty(fh.frame_bytes(n), dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    ctx.graph_begin()
    ctx.capturing = True
    try:
        fh.pack_frame(f, 0, out, counter)
    finally:
        ctx.capturing = False
        ctx.graph_end()
    for rep in range(3):
        ctx.graph_launch(1)
        ctx.sync()
        assert out.cpu().numpy().tobytes() == pack_reference(7 + rep, x, y, z), rep
        f.f32_fields["pos_x"].add_(0.0)  # eager work between replays
        torch.cuda.synchronize()
    assert counter.item() == 10


DAM_BREAK = dict(  # examples/dam-break.toml
    n=50_000, dt=1e-4, substeps=10,
    fields=[{"name": "position", "type": "vec3f",
             "init": {"type": "random", "min": [0.0, 0.0, 0.0], "max": [1.0, 2.0, 0.5]}},
            {"name": "velocity", "type": "vec3f", "init": {"type": "zero"}}],
    spatial={"type": "hashgrid", "cell_size": 0.05, "grid_dims": [40, 60, 20]},
    forces=[{"type": "sph_density", "smoothing_radius": 0.025},
            {"type": "sph_pressure", "gas_constant": 2000.0, "rest_density": 1000.0},
            {"type": "sph_viscosity", "coefficient": 0.01},
            {"type": "gravity", "value": [0.0, -9.81, 0.0]}],
    constraints=[{"type": "box", "min": [-0.1, 0.0, -0.1], "max": [2.0, 3.0, 0.6],
                  "restitution": 0.3}])


def dam_break_cfg(fh, spatial):
    """The SphConfig the reference's rules give for the dam-break manifest, derived here from
    the manifest (not from the built pipeline): h 0.025, cell size [spatial] or 2h, dims
    [spatial] or 32^3, mass rho0 / N * 0.001 in f32 (manifest_runner.rs:339-367)."""
    from forge_hip import workloads
    m = DAM_BREAK
    n = m["n"]
    arrs = fh.init_field_arrays(m["fields"], n)
    h = float(np.float32(0.025))
    cs = float(np.float32(spatial["cell_size"])) if spatial else float(np.float32(h) * 2)
    dims = tuple(spatial["grid_dims"]) if spatial else (32, 32, 32)
    mass = float(np.float32(np.float32(1000.0) / np.float32(n)) * np.float32(0.001))
    cfg = workloads.SphConfig("dam-break", n, arrs["pos_x"], arrs["pos_y"], arrs["pos_z"], h=h,
                              cell_size=cs, dims=dims, mass=mass, box_min=(-0.1, 0.0, -0.1),
                              box_max=(2.0, 3.0, 0.6), restitution=0.3)
    return cfg, arrs


@pytest.mark.parametrize("with_spatial", [True, False])
def test_build_pipeline_dam_break_step_matches_oracle(fh, gpu_ctx, oracle, with_spatial):
    """examples/dam-break.toml through init_fields + build_pipeline, one Pipeline::step on the
    GPU against or_sph_step with the parameters the reference's rules give; without [spatial]
    the cell size defaults to 2h and the grid to 32^3."""
    m = DAM_BREAK
    spatial = m["spatial"] if with_spatial else None
    cfg, arrs = dam_break_cfg(fh, spatial)
    pipe = fh.build_pipeline(m["forces"], m["constraints"], m["n"], spatial)
    assert [x.name() for x in pipe.modules] == ["sph_fused", "gravity", "integrate",
                                                "box_collider"]
    sph = pipe.modules[0]
    assert (sph.cell_size, tuple(sph.grid_dims), sph.particle_mass) == \
        (pytest.approx(cfg.cell_size), cfg.dims, cfg.mass)
    accel = torch.zeros((3, cfg.n), dtype=torch.float32, device="cuda")
    sph.accel = accel
    f = fh.FieldSet(m["n"])
    fh.init_fields(f, m["fields"])
    for k, a in arrs.items():
        assert np.array_equal(f.f32_fields[k].cpu().numpy(), a), k
    torch.cuda.synchronize()
    pipe.step(f, m["dt"])
    got = {k: t.cpu().numpy() for k, t in f.f32_fields.items()}
    zero = np.zeros(cfg.n, np.float32)
    fr = assert_oracle_step(oracle, cfg, (cfg.x, cfg.y, cfg.z), [zero] * 3, got,
                            accel.cpu().numpy())
    print("dam-break step 1 bit-exact fractions", fr)


def test_run_streaming_frames(fh, gpu_ctx):
    """run_streaming: frames after steps 0, 2, 4 of 5 (interval 2) with consecutive numbers;
    each frame's positions equal the fields after that step, which a separate run of the same
    substeps reproduces bit for bit; the result holds the final interleaved positions.  The
    callback keeps the arrays it is given (no copy): each must stay the frame it was."""
    from forge_hip import workloads
    cfg = workloads.small_sph(n=6000, cols=16)

    def pipeline():
        p = fh.Pipeline()
        p.add(fh.SphFusedModule(cfg.h, cfg.cell_size, cfg.dims, cfg.mass, cfg.gas_constant,
                                cfg.rest_density, cfg.viscosity))
        p.add(fh.GravityModule(*cfg.gravity))
        p.add(fh.IntegrateModule())
        p.add(fh.BoxColliderModule(*cfg.box_min, *cfg.box_max, cfg.restitution))
        return p

    frames = []
    f = fields_from(fh, cfg)
    torch.cuda.synchronize()
    res = fh.run_streaming(pipeline(), f, cfg.dt, total_steps=5, substeps=3, frame_interval=2,
                           on_frame=lambda k, b: frames.append((k, b)))
    assert [k for k, _ in frames] == [0, 1, 2] and res["steps"] == 15 and res["count"] == cfg.n
    g = fields_from(fh, cfg)
    p2 = pipeline()
    torch.cuda.synchronize()
    for step in range(5):
        p2.run(g, cfg.dt, 3)
        if step % 2 == 0:
            k, b = frames[step // 2]
            x, y, z = (g.f32_fields[nm].cpu().numpy() for nm in ("pos_x", "pos_y", "pos_z"))
            assert b.tobytes() == pack_reference(k, x, y, z), step
    assert np.array_equal(res["positions"], np.stack([x, y, z], 1).ravel())
