"""FieldSet / SimModule / Pipeline: host-side mirror of forge-manifest/src/modules/mod.rs and
the builtin modules on the SPH path, dispatching to the C ABI.

  FieldSet                 modules/mod.rs:12-67   (named SoA device arrays in particle order)
  SimModule                modules/mod.rs:70-73   (name(), execute(fields, dt))
  Pipeline                 modules/mod.rs:76-117  (step_async / step / run) + graph capture and
                           replay of substeps as run_manifest does (manifest_runner.rs:53-77)
  SphFusedModule           builtins/sph_fused.rs:14-22,410-733
  SphDensityModule         builtins/sph_density.rs:16-21,385-501
  SphPressureModule        builtins/sph_pressure.rs:9-161 (unfused)
  SphViscosityModule       builtins/sph_viscosity.rs:9-155 (unfused)
  GravityModule            builtins/gravity.rs:5-63
  IntegrateModule          builtins/integrate.rs:5-70
  BoxColliderModule        builtins/box_collider.rs:6-85
  build_pipeline           manifest_runner.rs:322-544 (SPH fusion, parameter defaults, order)
  init_fields              manifest_runner.rs:192-319 (field definitions -> SoA f32 fields)
  run_streaming            manifest_runner.rs:106-181 (substeps, then a binary position frame
                           every frame_interval steps; frame format of serve.rs:7-10,43-62)

Fields stay in original particle order, as the reference keeps them.  The SPH modules create
`density` on first use (sph_fused.rs:420-422); SphDensityModule also leaves its grid in the u32
fields `cell_start` and `sorted_indices`, which the unfused pressure / viscosity modules read.  When a pipeline holds [sph_fused, gravity,
integrate, box_collider] in that order, Pipeline fuses the three epilogue modules into the SPH
force pass (one kernel instead of three); the result equals running them separately.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import FhEpilogue, FhSphParams, check, f3
from .runtime import Context, default_context, ptr


class FieldSet:
    def __init__(self, particle_count: int, device: int = 0):
        self.f32_fields: dict[str, torch.Tensor] = {}
        self.u32_fields: dict[str, torch.Tensor] = {}
        self.particle_count = int(particle_count)
        self.device = int(device)
        self.ctx: Context | None = None

    def add_f32(self, name: str, data) -> None:
        t = torch.as_tensor(np.asarray(data, dtype=np.float32)).to(f"cuda:{self.device}")
        self.f32_fields[name] = t.contiguous()

    def add_f32_zeros(self, name: str, n: int) -> None:
        self.f32_fields[name] = torch.zeros(int(n), dtype=torch.float32,
                                            device=f"cuda:{self.device}")

    def get_f32(self, name: str):
        return self.f32_fields.get(name)

    def context(self, max_cells: int = 1) -> Context:
        """The stream/scratch owner of this field set: the device's default context, grown on
        first need (grow before capturing a graph: a grown context replaces the old one)."""
        self.ctx = default_context(max(self.particle_count, 1), max(int(max_cells), 1),
                                   self.device)
        return self.ctx

    def _f(self, name: str) -> torch.Tensor:
        t = self.f32_fields.get(name)
        if t is None:
            raise _lib.ForgeError(_lib.FH_EINVAL, f"missing field {name}")
        return t

    def pos(self):
        return self._f("pos_x"), self._f("pos_y"), self._f("pos_z")

    def vel(self):
        return self._f("vel_x"), self._f("vel_y"), self._f("vel_z")


class SimModule:
    def name(self) -> str:
        raise NotImplementedError

    def prepare(self, fields: FieldSet) -> None:
        """Create the fields execute() writes but the caller may not have added; this allocates,
        so Pipeline.capture calls it before recording starts."""

    def execute(self, fields: FieldSet, dt: float) -> None:
        raise NotImplementedError


def _sph_params(m) -> FhSphParams:
    p = FhSphParams()
    p.smoothing_radius = m.smoothing_radius
    p.cell_size = m.cell_size
    for q in range(3):
        p.grid_dims[q] = int(m.grid_dims[q])
    p.particle_mass = m.particle_mass
    p.gas_constant = getattr(m, "gas_constant", 0.0)
    p.rest_density = getattr(m, "rest_density", 0.0)
    p.viscosity_coefficient = getattr(m, "viscosity_coefficient", 0.0)
    return p


def _cells(dims) -> int:
    return int(dims[0]) * int(dims[1]) * int(dims[2])


class SphDensityModule(SimModule):
    def __init__(self, smoothing_radius, cell_size, grid_dims, particle_mass):
        self.smoothing_radius = float(smoothing_radius)
        self.cell_size = float(cell_size)
        self.grid_dims = [int(d) for d in grid_dims]
        self.particle_mass = float(particle_mass)

    def name(self) -> str:
        return "sph_density"

    def prepare(self, fields: FieldSet) -> None:
        if "density" not in fields.f32_fields:
            fields.add_f32_zeros("density", fields.particle_count)
        dev = f"cuda:{fields.device}"
        cells = _cells(self.grid_dims) + 1
        cs = fields.u32_fields.get("cell_start")
        if cs is None or cs.numel() != cells:
            fields.u32_fields["cell_start"] = torch.zeros(cells, dtype=torch.int32, device=dev)
        si = fields.u32_fields.get("sorted_indices")
        if si is None or si.numel() != fields.particle_count:
            fields.u32_fields["sorted_indices"] = torch.zeros(fields.particle_count,
                                                              dtype=torch.int32, device=dev)

    def execute(self, fields: FieldSet, dt: float) -> None:
        n = fields.particle_count
        self.prepare(fields)
        ctx = fields.context(_cells(self.grid_dims))
        px, py, pz = fields.pos()
        check(_lib.load().fh_sph_density(ctx.handle, ctypes.byref(_sph_params(self)), ptr(px),
                                         ptr(py), ptr(pz), n, ptr(fields.f32_fields["density"]),
                                         ptr(fields.u32_fields["cell_start"]),
                                         ptr(fields.u32_fields["sorted_indices"])))


class _UnfusedModule(SimModule):
    """Shared body of the unfused pressure / viscosity modules: they read the grid and density
    that SphDensityModule left in the field set (sph_pressure.rs:129-137 take them with
    `.unwrap()`, so a missing field is an error)."""

    _entry = ""

    def execute(self, fields: FieldSet, dt: float) -> None:
        n = fields.particle_count
        for nm in ("cell_start", "sorted_indices"):
            if nm not in fields.u32_fields:
                raise _lib.ForgeError(_lib.FH_EINVAL, f"missing field {nm} (run sph_density first)")
        cs = fields.u32_fields["cell_start"]
        if cs.numel() != _cells(self.grid_dims) + 1:
            raise _lib.ForgeError(_lib.FH_EINVAL, f"{self.name()}: cell_start has {cs.numel()} "
                                  f"entries, the grid needs {_cells(self.grid_dims) + 1}")
        ctx = fields.context(_cells(self.grid_dims))
        px, py, pz = fields.pos()
        vx, vy, vz = fields.vel()
        fn = getattr(_lib.load(), self._entry)
        check(fn(ctx.handle, ctypes.byref(_sph_params(self)), ptr(px), ptr(py), ptr(pz), ptr(vx),
                 ptr(vy), ptr(vz), ptr(fields._f("density")), ptr(cs),
                 ptr(fields.u32_fields["sorted_indices"]), n, float(dt)))


class SphPressureModule(_UnfusedModule):
    """sph_pressure.rs:9-16: v_i += (a_p / rho_i) dt with p = k (rho - rho0)."""

    _entry = "fh_sph_pressure"

    def __init__(self, gas_constant, rest_density, smoothing_radius, cell_size, grid_dims,
                 particle_mass):
        self.gas_constant = float(gas_constant)
        self.rest_density = float(rest_density)
        self.smoothing_radius = float(smoothing_radius)
        self.cell_size = float(cell_size)
        self.grid_dims = [int(d) for d in grid_dims]
        self.particle_mass = float(particle_mass)

    def name(self) -> str:
        return "sph_pressure"


class SphViscosityModule(_UnfusedModule):
    """sph_viscosity.rs:9-15: v_i += (a_v / rho_i) dt, neighbours' velocities before the pass."""

    _entry = "fh_sph_viscosity"

    def __init__(self, coefficient, smoothing_radius, cell_size, grid_dims, particle_mass):
        self.coefficient = float(coefficient)
        self.viscosity_coefficient = self.coefficient
        self.smoothing_radius = float(smoothing_radius)
        self.cell_size = float(cell_size)
        self.grid_dims = [int(d) for d in grid_dims]
        self.particle_mass = float(particle_mass)

    def name(self) -> str:
        return "sph_viscosity"


class SphFusedModule(SimModule):
    def __init__(self, smoothing_radius, cell_size, grid_dims, particle_mass, gas_constant,
                 rest_density, viscosity_coefficient):
        self.smoothing_radius = float(smoothing_radius)
        self.cell_size = float(cell_size)
        self.grid_dims = [int(d) for d in grid_dims]
        self.particle_mass = float(particle_mass)
        self.gas_constant = float(gas_constant)
        self.rest_density = float(rest_density)
        self.viscosity_coefficient = float(viscosity_coefficient)
        self.epilogue: FhEpilogue | None = None  # set by Pipeline fusion
        self.accel: torch.Tensor | None = None   # optional (3, N) output of a_i

    def name(self) -> str:
        return "sph_fused"

    def prepare(self, fields: FieldSet) -> None:
        if "density" not in fields.f32_fields:
            fields.add_f32_zeros("density", fields.particle_count)

    def execute(self, fields: FieldSet, dt: float) -> None:
        self._call(fields, dt, None)

    def execute_force(self, fields: FieldSet, dt: float) -> None:
        """The fused force pass alone (sph_fused.rs:519-639) over the grid and densities already
        in the field set (u32 cell_start / sorted_indices and f32 density, as SphDensityModule
        leaves them): v += a dt in place; a_i into self.accel when set."""
        n = fields.particle_count
        for nm in ("cell_start", "sorted_indices"):
            if nm not in fields.u32_fields:
                raise _lib.ForgeError(_lib.FH_EINVAL, f"missing field {nm} (run sph_density first)")
        cs = fields.u32_fields["cell_start"]
        if cs.numel() != _cells(self.grid_dims) + 1:
            raise _lib.ForgeError(_lib.FH_EINVAL, f"sph_fused: cell_start has {cs.numel()} "
                                  f"entries, the grid needs {_cells(self.grid_dims) + 1}")
        ctx = fields.context(_cells(self.grid_dims))
        px, py, pz = fields.pos()
        vx, vy, vz = fields.vel()
        check(_lib.load().fh_sph_force(ctx.handle, ctypes.byref(_sph_params(self)), ptr(px),
                                       ptr(py), ptr(pz), ptr(vx), ptr(vy), ptr(vz),
                                       ptr(fields._f("density")), ptr(cs),
                                       ptr(fields.u32_fields["sorted_indices"]), ptr(self.accel),
                                       n, float(dt)))

    def execute_steps(self, fields: FieldSet, dt: float, steps: int) -> None:
        """`steps` substeps in one call (fh_sph_fused_steps): the state stays in sorted order on
        the device between them and the fields are written once, after the last."""
        self._call(fields, dt, int(steps))

    def _call(self, fields: FieldSet, dt: float, steps: int | None) -> None:
        n = fields.particle_count
        self.prepare(fields)
        ctx = fields.context(_cells(self.grid_dims))
        px, py, pz = fields.pos()
        vx, vy, vz = fields.vel()
        epi = ctypes.byref(self.epilogue) if self.epilogue is not None else None
        args = (ctx.handle, ctypes.byref(_sph_params(self)), epi, ptr(px), ptr(py), ptr(pz),
                ptr(vx), ptr(vy), ptr(vz), ptr(fields.f32_fields["density"]), ptr(self.accel),
                n, float(dt))
        if steps is None:
            check(_lib.load().fh_sph_fused(*args))
        else:
            check(_lib.load().fh_sph_fused_steps(*args, steps))


class GravityModule(SimModule):
    def __init__(self, gx: float = 0.0, gy: float = -9.81, gz: float = 0.0):
        self.gx, self.gy, self.gz = float(gx), float(gy), float(gz)

    @staticmethod
    def default_earth():
        return GravityModule(0.0, -9.81, 0.0)

    def name(self) -> str:
        return "gravity"

    def execute(self, fields: FieldSet, dt: float) -> None:
        vx, vy, vz = fields.vel()
        ctx = fields.context()
        check(_lib.load().fh_gravity(ctx.handle, ptr(vx), ptr(vy), ptr(vz),
                                     fields.particle_count, self.gx, self.gy, self.gz, float(dt)))


class IntegrateModule(SimModule):
    def name(self) -> str:
        return "integrate"

    def execute(self, fields: FieldSet, dt: float) -> None:
        px, py, pz = fields.pos()
        vx, vy, vz = fields.vel()
        ctx = fields.context()
        check(_lib.load().fh_integrate(ctx.handle, ptr(px), ptr(py), ptr(pz), ptr(vx), ptr(vy),
                                       ptr(vz), fields.particle_count, float(dt)))


class BoxColliderModule(SimModule):
    def __init__(self, min_x, min_y, min_z, max_x, max_y, max_z, restitution):
        self.min_x, self.min_y, self.min_z = float(min_x), float(min_y), float(min_z)
        self.max_x, self.max_y, self.max_z = float(max_x), float(max_y), float(max_z)
        self.restitution = float(restitution)

    def name(self) -> str:
        return "box_collider"

    def execute(self, fields: FieldSet, dt: float) -> None:
        px, py, pz = fields.pos()
        vx, vy, vz = fields.vel()
        ctx = fields.context()
        check(_lib.load().fh_box_collider(
            ctx.handle, ptr(px), ptr(py), ptr(pz), ptr(vx), ptr(vy), ptr(vz),
            fields.particle_count, f3((self.min_x, self.min_y, self.min_z)),
            f3((self.max_x, self.max_y, self.max_z)), self.restitution))


class Pipeline:
    def __init__(self, fuse_epilogue: bool = True, resident: bool = True):
        self.modules: list[SimModule] = []
        self.fuse_epilogue = fuse_epilogue
        self.resident = resident  # run / capture: sorted state kept on the device between substeps
        self._plan: list[SimModule] | None = None
        self._captured_ctx: Context | None = None

    def add(self, module: SimModule) -> None:
        self.modules.append(module)
        self._plan = None

    def __len__(self) -> int:
        return len(self.modules)

    def _fused_plan(self) -> list[SimModule]:
        """Fold gravity / integrate / box that directly follow sph_fused into its force pass."""
        if self._plan is not None:
            return self._plan
        plan: list[SimModule] = []
        mods = self.modules
        i = 0
        while i < len(mods):
            m = mods[i]
            if self.fuse_epilogue and isinstance(m, SphFusedModule) and m.epilogue is None:
                epi = FhEpilogue()
                j = i + 1
                order = [GravityModule, IntegrateModule, BoxColliderModule]
                for kind in order:
                    if j < len(mods) and isinstance(mods[j], kind):
                        e = mods[j]
                        if kind is GravityModule:
                            epi.flags |= _lib.FH_EPI_GRAVITY
                            epi.gravity[:] = [e.gx, e.gy, e.gz]
                        elif kind is IntegrateModule:
                            epi.flags |= _lib.FH_EPI_INTEGRATE
                        else:
                            epi.flags |= _lib.FH_EPI_BOX
                            epi.box_min[:] = [e.min_x, e.min_y, e.min_z]
                            epi.box_max[:] = [e.max_x, e.max_y, e.max_z]
                            epi.restitution = e.restitution
                        j += 1
                if j > i + 1:
                    fused = SphFusedModule(m.smoothing_radius, m.cell_size, m.grid_dims,
                                           m.particle_mass, m.gas_constant, m.rest_density,
                                           m.viscosity_coefficient)
                    fused.epilogue = epi
                    fused.accel = m.accel
                    plan.append(fused)
                    i = j
                    continue
            plan.append(m)
            i += 1
        self._plan = plan
        return plan

    def step_async(self, fields: FieldSet, dt: float) -> None:
        """All modules in order, queued on the field set's stream (modules/mod.rs:90-95)."""
        ctx = fields.context(max((_cells(m.grid_dims) for m in self.modules
                                  if hasattr(m, "grid_dims")), default=1))
        if not getattr(ctx, "capturing", False):
            ctx.torch_stream().wait_stream(torch.cuda.current_stream())
        for m in self._fused_plan():
            m.execute(fields, dt)

    def step(self, fields: FieldSet, dt: float) -> None:
        """step_async, then wait for the stream (modules/mod.rs:98-104)."""
        self.step_async(fields, dt)
        fields.context().sync()

    def run_async(self, fields: FieldSet, dt: float, steps: int) -> None:
        """`steps` substeps queued on the field set's stream.  When the (fused) plan is a single
        sph_fused module and `resident` is set, they are one fh_sph_fused_steps call: the state
        stays in sorted order on the device and the fields are written after the last substep
        only (nothing else reads them in between)."""
        plan = self._fused_plan()
        steps = int(steps)
        if self.resident and steps > 1 and len(plan) == 1 and isinstance(plan[0], SphFusedModule):
            ctx = fields.context(_cells(plan[0].grid_dims))
            if not getattr(ctx, "capturing", False):
                ctx.torch_stream().wait_stream(torch.cuda.current_stream())
            plan[0].execute_steps(fields, dt, steps)
            return
        for _ in range(steps):
            self.step_async(fields, dt)

    def run(self, fields: FieldSet, dt: float, steps: int) -> None:
        """`steps` substeps, then wait for the stream (modules/mod.rs:106-112)."""
        self.run_async(fields, dt, steps)
        fields.context().sync()

    def capture(self, fields: FieldSet, dt: float, substeps: int) -> None:
        """Record `substeps` step_async calls into one HIP graph (manifest_runner.rs:57-69)."""
        ctx = fields.context(max((_cells(m.grid_dims) for m in self.modules
                                  if hasattr(m, "grid_dims")), default=1))
        for m in self._fused_plan():
            m.prepare(fields)
        ctx.torch_stream().wait_stream(torch.cuda.current_stream())
        ctx.sync()
        ctx.graph_begin()
        ctx.capturing = True
        try:
            self.run_async(fields, dt, substeps)
        finally:
            ctx.capturing = False
            ctx.graph_end()
        self._captured_ctx = ctx

    def replay(self, count: int = 1) -> None:
        """Launch the captured graph `count` times (manifest_runner.rs:74-77)."""
        if self._captured_ctx is None:
            raise _lib.ForgeError(_lib.FH_ESTATE, "no captured graph")
        self._captured_ctx.graph_launch(count)


def _grid_dims(spatial: dict | None) -> list[int]:
    """[spatial].grid_dims with each missing entry 32, or 32^3 (manifest_runner.rs:359-365)."""
    dims = list(spatial.get("grid_dims", [])) if spatial else []
    return [int(d) for d in (dims + [32, 32, 32][len(dims):])[:3]]


def build_pipeline(forces: list[dict], constraints: list[dict], n: int,
                   spatial: dict | None = None) -> Pipeline:
    """Pipeline construction of manifest_runner.rs:322-544 for the SPH path.

    forces: dicts with "type" in {"sph_density", "sph_pressure", "sph_viscosity", "gravity"}
    and the manifest's keys; constraints: {"type": "box", "min": [...], "max": [...],
    "restitution": e}.  Fusion, defaults (h 0.025, (k, rho0) = (2000, 1000), mu 0.01,
    cell_size 2h, dims 32^3, mass = rho0 / n * 0.001) and order (fused SPH, other forces,
    integrate, constraints) follow the reference."""
    from .workloads import particle_mass

    pipe = Pipeline()
    kinds = {f["type"] for f in forces}
    fuse = {"sph_density", "sph_pressure", "sph_viscosity"} <= kinds
    if fuse:
        h = next((float(f["smoothing_radius"]) for f in forces if f["type"] == "sph_density"), 0.025)
        k, rho0 = next(((float(f["gas_constant"]), float(f["rest_density"])) for f in forces
                        if f["type"] == "sph_pressure"), (2000.0, 1000.0))
        mu = next((float(f["coefficient"]) for f in forces if f["type"] == "sph_viscosity"), 0.01)
        cs = float(spatial["cell_size"]) if spatial else h * 2.0
        dims = list(spatial.get("grid_dims", [32, 32, 32])) if spatial else [32, 32, 32]
        dims = (dims + [32, 32, 32])[:3]
        pipe.add(SphFusedModule(h, cs, dims, particle_mass(rho0, n), k, rho0, mu))
    for f in forces:
        if f["type"] == "gravity":
            v = list(f.get("value", [0.0, -9.81, 0.0])) + [0.0, -9.81, 0.0][len(f.get("value", [])):]
            pipe.add(GravityModule(v[0], v[1], v[2]))
        elif f["type"] in ("sph_density", "sph_pressure", "sph_viscosity") and fuse:
            continue
        elif f["type"] == "sph_density":  # manifest_runner.rs:419-437
            h = float(f["smoothing_radius"])
            cs = float(spatial["cell_size"]) if spatial else h * 2.0
            pipe.add(SphDensityModule(h, cs, _grid_dims(spatial), particle_mass(1000.0, n)))
        elif f["type"] in ("sph_pressure", "sph_viscosity"):  # :438-488
            # cell size 0.05 and h 0.025 unless the manifest sets them (not 2h as for density)
            cs = float(spatial["cell_size"]) if spatial else 0.05
            h = next((float(g["smoothing_radius"]) for g in forces if g["type"] == "sph_density"),
                     0.025)
            if f["type"] == "sph_pressure":
                k, rho0 = float(f["gas_constant"]), float(f["rest_density"])
                pipe.add(SphPressureModule(k, rho0, h, cs, _grid_dims(spatial),
                                           particle_mass(rho0, n)))
            else:
                pipe.add(SphViscosityModule(float(f["coefficient"]), h, cs, _grid_dims(spatial),
                                            particle_mass(1000.0, n)))
        else:
            raise _lib.ForgeError(_lib.FH_EINVAL, f"force {f['type']} is outside the SPH path")
    pipe.add(IntegrateModule())
    for c in constraints:
        if c["type"] != "box":
            raise _lib.ForgeError(_lib.FH_EINVAL, f"constraint {c['type']} is outside the SPH path")
        # each missing element defaults on its own: min 0.0, max 1.0 (manifest_runner.rs:528-537);
        # restitution 0.5 when absent (schema.rs:151-159)
        mn = _elems(c.get("min", []), 3, 0.0)
        mx = _elems(c.get("max", []), 3, 1.0)
        pipe.add(BoxColliderModule(mn[0], mn[1], mn[2], mx[0], mx[1], mx[2],
                                   float(c.get("restitution", 0.5))))
    return pipe


# ---- fields from the manifest's field definitions (manifest_runner.rs:192-319) --------------

_BASE_NAMES = {"position": "pos", "pos": "pos", "velocity": "vel", "vel": "vel"}


def _elems(v, count: int, default: float) -> list[float]:
    """`v.first()/get(1)/get(2).unwrap_or(default)`: each missing element defaults alone."""
    v = list(v or [])
    return [float(v[a]) if a < len(v) else default for a in range(count)]


def _init_vec3(n: int, init: dict | None, seed: int, stream: int) -> list[np.ndarray]:
    """init_vec3 (manifest_runner.rs:255-300) in float32.  `random` draws from the seeded
    generator of workloads (the reference's thread_rng is unseeded, so no draw is reproducible
    there); every other kind is deterministic and equals the reference's values bit for bit."""
    from .workloads import uniform_f32

    f32 = np.float32
    kind = (init or {}).get("type", "zero")
    if kind == "random":
        mn = _elems(init.get("min", [-1.0, -1.0, -1.0]), 3, -1.0)  # schema.rs:83 defaults
        mx = _elems(init.get("max", [1.0, 1.0, 1.0]), 3, 1.0)
        out = []
        for a in range(3):
            u = uniform_f32(seed, 100 + 3 * stream + a, n)  # [0, 1)
            lo, hi = f32(mn[a]), f32(mx[a])
            v = (u * (hi - lo) + lo).astype(f32)
            out.append(np.minimum(v, np.nextafter(hi, lo)) if hi > lo else v)  # half-open range
        return out
    if kind == "constant":
        val = _elems(init.get("value", []), 3, 0.0)
        return [np.full(n, f32(val[a]), f32) for a in range(3)]
    if kind == "grid":
        # side = ceil(sqrt(n as f32)); particle i at (ox + ix sp, oy, oz + iz sp), ix = i % side
        sp = f32(init.get("spacing", 0.1))
        o = _elems(init.get("origin", [0.0, 0.0, 0.0]), 3, 0.0)
        side = int(np.ceil(np.sqrt(f32(n), dtype=f32)))
        i = np.arange(n, dtype=np.int64)
        ix, iz = (i % side).astype(f32), (i // side).astype(f32)
        return [(f32(o[0]) + ix * sp).astype(f32), np.full(n, f32(o[1]), f32),
                (f32(o[2]) + iz * sp).astype(f32)]
    return [np.zeros(n, f32) for _ in range(3)]  # zero, absent or unknown


def init_field_arrays(field_defs: list[dict], n: int, seed: int | None = None) -> dict:
    """Host arrays of init_fields: a vec3f field `name` becomes `<base>_x/_y/_z` (base "pos" for
    position / pos, "vel" for velocity / vel, else the name), an f32 field keeps its name
    (constant value[0] or zeros); vel_* and pos_* default to zeros when no field made them."""
    from .workloads import DEFAULT_SEED

    seed = DEFAULT_SEED if seed is None else int(seed)
    out: dict[str, np.ndarray] = {}
    for k, fd in enumerate(field_defs):
        name, kind = fd["name"], fd.get("type", "vec3f")
        if kind == "vec3f":
            base = _BASE_NAMES.get(name, name)
            for a, arr in zip("xyz", _init_vec3(n, fd.get("init"), seed, k)):
                out[f"{base}_{a}"] = arr
        elif kind == "f32":
            init = fd.get("init") or {}
            v = _elems(init.get("value", []), 1, 0.0)[0] if init.get("type") == "constant" else 0.0
            out[name] = np.full(n, np.float32(v), np.float32)
    for base in ("vel", "pos"):
        if f"{base}_x" not in out:
            for a in "xyz":
                out[f"{base}_{a}"] = np.zeros(n, np.float32)
    return out


def init_fields(fields: FieldSet, field_defs: list[dict], seed: int | None = None) -> None:
    """init_fields (manifest_runner.rs:192-233): the field definitions' arrays, uploaded."""
    for nm, arr in init_field_arrays(field_defs, fields.particle_count, seed).items():
        fields.add_f32(nm, arr)


# ---- frames (run_manifest_streaming, manifest_runner.rs:106-181; serve.rs:7-10,43-62) -------

def frame_bytes(n: int) -> int:
    """Size of one binary frame: u32 frame, u32 count, f32 x 3n."""
    return 8 + 12 * int(n)


def pack_frame(fields: FieldSet, frame: int, out: torch.Tensor | None = None,
               counter: torch.Tensor | None = None) -> torch.Tensor:
    """The binary frame of the current positions, packed on the device into `out` (uint8,
    frame_bytes(n)); with `counter` (a device int32 of one element) the frame number is taken
    from it and incremented there instead (for captured graphs)."""
    n = fields.particle_count
    ctx = fields.context()
    if out is None:
        out = torch.empty(frame_bytes(n), dtype=torch.uint8, device=f"cuda:{fields.device}")
    if out.numel() < frame_bytes(n) or out.dtype != torch.uint8:
        raise _lib.ForgeError(_lib.FH_EINVAL, f"frame buffer needs {frame_bytes(n)} uint8 bytes")
    px, py, pz = fields.pos()
    check(_lib.load().fh_pack_frame(ctx.handle, ptr(px), ptr(py), ptr(pz), n, int(frame),
                                    ptr(counter), ptr(out)))
    return out


def run_streaming(pipeline: Pipeline, fields: FieldSet, dt: float, total_steps: int,
                  substeps: int, frame_interval: int, on_frame) -> dict:
    """run_manifest_streaming's loop (manifest_runner.rs:145-181): each step runs `substeps`
    substeps; after step s with s % frame_interval == 0 (interval at least 1) the frame
    (u32 frame number, u32 count, interleaved f32 positions) is packed on the device, copied
    into pinned host memory and passed to on_frame(frame_number, frame) as a uint8 array of its
    own (the positions are frame[8:].view(float32)): the callback may keep it, as the Rust
    mirror's callback receives the frame by value.  Returns the final positions (interleaved),
    count, substeps run and elapsed seconds, as SimResult does."""
    import time

    n = fields.particle_count
    interval = max(int(frame_interval), 1)
    ctx = fields.context(max((_cells(m.grid_dims) for m in pipeline.modules
                              if hasattr(m, "grid_dims")), default=1))
    dev = torch.empty(frame_bytes(n), dtype=torch.uint8, device=f"cuda:{fields.device}")
    host = torch.empty(frame_bytes(n), dtype=torch.uint8, pin_memory=True)
    start = time.perf_counter()
    count = frame_num = 0
    for step in range(int(total_steps)):
        pipeline.run_async(fields, dt, int(substeps))
        count += int(substeps)
        if step % interval == 0:
            pack_frame(fields, frame_num, dev)
            with torch.cuda.stream(ctx.torch_stream()):
                host.copy_(dev, non_blocking=True)
            ctx.sync()
            # a copy: the pinned staging buffer is reused by the next frame
            on_frame(frame_num, host.numpy().copy())
            frame_num += 1
    ctx.sync()
    elapsed = time.perf_counter() - start
    pack_frame(fields, 0, dev)
    with torch.cuda.stream(ctx.torch_stream()):
        host.copy_(dev, non_blocking=True)
    ctx.sync()
    return dict(positions=host.numpy()[8:].view(np.float32).copy(), count=n, steps=count,
                elapsed_secs=elapsed)
