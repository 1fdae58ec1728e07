//! `FieldSet`, `SimModule`, the seven modules of the SPH path and `Pipeline`
//! (forge-manifest/src/modules/mod.rs:12-117, builtins/*.rs), each module one C ABI call on the
//! FieldSet's context.  Fields stay in particle order, keyed by the reference's names
//! (`pos_x/y/z`, `vel_x/y/z`, `density`; u32 `cell_start`, `sorted_indices` left by the density
//! module for the unfused pressure / viscosity modules).

use std::collections::HashMap;
use std::sync::Mutex;

use forge_hip_sys as sys;

use crate::array::{Array, Device, DevicePtr, Vec3f};
use crate::context::Ctx;
use crate::error::{check, ForgeError};

/// Named device arrays in particle order (modules/mod.rs:12-67), plus the context the SPH
/// modules run on (created on first use, sized for the largest grid a module asked for).
pub struct FieldSet {
    pub f32_fields: HashMap<String, Array<f32>>,
    pub vec3_fields: HashMap<String, Array<Vec3f>>,
    pub i32_fields: HashMap<String, Array<i32>>,
    pub u32_fields: HashMap<String, Array<u32>>,
    pub index_pairs: HashMap<String, Vec<[u32; 2]>>,
    pub particle_count: usize,
    pub device: Device,
    ctx: Mutex<Option<Ctx>>,
}

impl FieldSet {
    pub fn new(particle_count: usize, device: Device) -> Self {
        FieldSet {
            f32_fields: HashMap::new(),
            vec3_fields: HashMap::new(),
            i32_fields: HashMap::new(),
            u32_fields: HashMap::new(),
            index_pairs: HashMap::new(),
            particle_count,
            device,
            ctx: Mutex::new(None),
        }
    }

    pub fn add_f32(&mut self, name: &str, data: Vec<f32>) {
        self.f32_fields.insert(name.to_string(), Array::from_vec(data, self.device));
    }

    pub fn add_f32_zeros(&mut self, name: &str, len: usize) {
        self.f32_fields.insert(name.to_string(), Array::zeros(len, self.device));
    }

    pub fn add_vec3(&mut self, name: &str, data: Vec<Vec3f>) {
        self.vec3_fields.insert(name.to_string(), Array::from_vec(data, self.device));
    }

    pub fn get_f32(&self, name: &str) -> Option<&Array<f32>> {
        self.f32_fields.get(name)
    }

    pub fn get_f32_mut(&mut self, name: &str) -> Option<&mut Array<f32>> {
        self.f32_fields.get_mut(name)
    }

    /// The context for a module with `num_cells` cells: created on first use, recreated (outside
    /// graph capture) when a module needs a larger grid.
    pub fn hip_ctx(&self, num_cells: usize) -> Result<*mut sys::fh_ctx, ForgeError> {
        let mut g = self.ctx.lock().unwrap();
        let fits = matches!(&*g, Some(c) if c.max_cells() >= num_cells
                                          && c.max_n() >= self.particle_count);
        if !fits {
            *g = None;  // drop the old context first
            *g = Some(Ctx::new(self.device.ordinal()?, self.particle_count.max(1),
                               num_cells.max(1))?);
        }
        Ok(g.as_ref().unwrap().raw())
    }

    /// Waits for the context's stream (nothing queued: Ok).
    pub fn sync(&self) -> Result<(), ForgeError> {
        match &*self.ctx.lock().unwrap() {
            Some(c) => c.sync(),
            None => Ok(()),
        }
    }

    fn f32_ptr(&self, name: &str) -> Result<*mut f32, ForgeError> {
        // the C ABI takes mutable device pointers; the map only hands out shared references
        // while several fields are borrowed at once, and device memory is not aliased by Rust
        self.f32_fields
            .get(name)
            .map(|a| a.device_ptr() as *mut f32)
            .ok_or_else(|| ForgeError::LaunchFailed(format!("missing f32 field {}", name)))
    }

    fn u32_ptr(&self, name: &str) -> Result<*mut u32, ForgeError> {
        self.u32_fields
            .get(name)
            .map(|a| a.device_ptr() as *mut u32)
            .ok_or_else(|| ForgeError::LaunchFailed(format!("missing u32 field {}", name)))
    }

    fn ensure_f32(&mut self, name: &str) {
        if !self.f32_fields.contains_key(name) {
            let n = self.particle_count;
            self.add_f32_zeros(name, n);
        }
    }

    fn ensure_u32(&mut self, name: &str, len: usize) {
        let ok = matches!(self.u32_fields.get(name), Some(a) if a.len() == len);
        if !ok {
            self.u32_fields.insert(name.to_string(), Array::zeros(len, self.device));
        }
    }
}

/// What a module is, for the epilogue fusion of `build_pipeline` (manifest_runner.rs:371-393,
/// 508, 528-537).  The provided default keeps other modules' impls unchanged.
#[derive(Clone, Debug)]
pub enum ModuleKind {
    Other,
    SphFused(SphFusedModule),
    Gravity([f32; 3]),
    Integrate,
    BoxCollider { min: [f32; 3], max: [f32; 3], restitution: f32 },
}

/// modules/mod.rs:70-73.
pub trait SimModule: Send + Sync {
    fn name(&self) -> &str;
    fn execute(&self, fields: &mut FieldSet, dt: f32) -> Result<(), ForgeError>;
    fn kind(&self) -> ModuleKind {
        ModuleKind::Other
    }
}

fn cells(d: &[u32; 3]) -> usize {
    d[0] as usize * d[1] as usize * d[2] as usize
}

/// sph_fused.rs:14-22: rebuild, density, fused pressure + viscosity (v += a dt); with an
/// epilogue (set by `fuse_epilogue`) also gravity, integrate and box in the same pass.
#[derive(Clone, Debug)]
pub struct SphFusedModule {
    pub smoothing_radius: f32,
    pub cell_size: f32,
    pub grid_dims: [u32; 3],
    pub particle_mass: f32,
    pub gas_constant: f32,
    pub rest_density: f32,
    pub viscosity_coefficient: f32,
    pub epilogue: Option<sys::fh_epilogue>,
}

impl SphFusedModule {
    fn params(&self) -> sys::fh_sph_params {
        sys::fh_sph_params {
            smoothing_radius: self.smoothing_radius,
            cell_size: self.cell_size,
            grid_dims: self.grid_dims,
            particle_mass: self.particle_mass,
            gas_constant: self.gas_constant,
            rest_density: self.rest_density,
            viscosity_coefficient: self.viscosity_coefficient,
        }
    }

    fn epi_ptr(&self) -> *const sys::fh_epilogue {
        self.epilogue.as_ref().map_or(std::ptr::null(), |e| e as *const _)
    }

    /// `steps` substeps in one call (fh_sph_fused_steps): the state stays on the device in
    /// cell-sorted order between them; the fields are written after the last one.
    pub fn execute_steps(&self, f: &mut FieldSet, dt: f32, steps: u32) -> Result<(), ForgeError> {
        f.ensure_f32("density");
        let ctx = f.hip_ctx(cells(&self.grid_dims))?;
        let p = self.params();
        check(unsafe {
            sys::fh_sph_fused_steps(ctx, &p, self.epi_ptr(), f.f32_ptr("pos_x")?,
                                    f.f32_ptr("pos_y")?, f.f32_ptr("pos_z")?, f.f32_ptr("vel_x")?,
                                    f.f32_ptr("vel_y")?, f.f32_ptr("vel_z")?,
                                    f.f32_ptr("density")?, std::ptr::null_mut(),
                                    f.particle_count as u32, dt, steps)
        })
    }
}

impl SimModule for SphFusedModule {
    fn name(&self) -> &str {
        "sph_fused"
    }
    fn execute(&self, f: &mut FieldSet, dt: f32) -> Result<(), ForgeError> {
        f.ensure_f32("density");
        let ctx = f.hip_ctx(cells(&self.grid_dims))?;
        let p = self.params();
        check(unsafe {
            sys::fh_sph_fused(ctx, &p, self.epi_ptr(), f.f32_ptr("pos_x")?, f.f32_ptr("pos_y")?,
                              f.f32_ptr("pos_z")?, f.f32_ptr("vel_x")?, f.f32_ptr("vel_y")?,
                              f.f32_ptr("vel_z")?, f.f32_ptr("density")?, std::ptr::null_mut(),
                              f.particle_count as u32, dt)
        })
    }
    fn kind(&self) -> ModuleKind {
        ModuleKind::SphFused(self.clone())
    }
}

/// sph_density.rs:16-21: rebuild + density; leaves the grid in the u32 fields `cell_start`
/// (C + 1) and `sorted_indices` (n) for the unfused pressure / viscosity modules.
#[derive(Clone, Debug)]
pub struct SphDensityModule {
    pub smoothing_radius: f32,
    pub cell_size: f32,
    pub grid_dims: [u32; 3],
    pub particle_mass: f32,
}

impl SimModule for SphDensityModule {
    fn name(&self) -> &str {
        "sph_density"
    }
    fn execute(&self, f: &mut FieldSet, _dt: f32) -> Result<(), ForgeError> {
        let c = cells(&self.grid_dims);
        f.ensure_f32("density");
        f.ensure_u32("cell_start", c + 1);
        let n = f.particle_count;
        f.ensure_u32("sorted_indices", n);
        let ctx = f.hip_ctx(c)?;
        let p = sys::fh_sph_params {
            smoothing_radius: self.smoothing_radius,
            cell_size: self.cell_size,
            grid_dims: self.grid_dims,
            particle_mass: self.particle_mass,
            ..Default::default()
        };
        check(unsafe {
            sys::fh_sph_density(ctx, &p, f.f32_ptr("pos_x")?, f.f32_ptr("pos_y")?,
                                f.f32_ptr("pos_z")?, n as u32, f.f32_ptr("density")?,
                                f.u32_ptr("cell_start")?, f.u32_ptr("sorted_indices")?)
        })
    }
}

/// sph_pressure.rs:9-16 (over the grid the density module left in the field set).
#[derive(Clone, Debug)]
pub struct SphPressureModule {
    pub gas_constant: f32,
    pub rest_density: f32,
    pub smoothing_radius: f32,
    pub cell_size: f32,
    pub grid_dims: [u32; 3],
    pub particle_mass: f32,
}

impl SimModule for SphPressureModule {
    fn name(&self) -> &str {
        "sph_pressure"
    }
    fn execute(&self, f: &mut FieldSet, dt: f32) -> Result<(), ForgeError> {
        let ctx = f.hip_ctx(cells(&self.grid_dims))?;
        let p = sys::fh_sph_params {
            smoothing_radius: self.smoothing_radius,
            cell_size: self.cell_size,
            grid_dims: self.grid_dims,
            particle_mass: self.particle_mass,
            gas_constant: self.gas_constant,
            rest_density: self.rest_density,
            viscosity_coefficient: 0.0,
        };
        check(unsafe {
            sys::fh_sph_pressure(ctx, &p, f.f32_ptr("pos_x")?, f.f32_ptr("pos_y")?,
                                 f.f32_ptr("pos_z")?, f.f32_ptr("vel_x")?, f.f32_ptr("vel_y")?,
                                 f.f32_ptr("vel_z")?, f.f32_ptr("density")?,
                                 f.u32_ptr("cell_start")?, f.u32_ptr("sorted_indices")?,
                                 f.particle_count as u32, dt)
        })
    }
}

/// sph_viscosity.rs:9-15.
#[derive(Clone, Debug)]
pub struct SphViscosityModule {
    pub coefficient: f32,
    pub smoothing_radius: f32,
    pub cell_size: f32,
    pub grid_dims: [u32; 3],
    pub particle_mass: f32,
}

impl SimModule for SphViscosityModule {
    fn name(&self) -> &str {
        "sph_viscosity"
    }
    fn execute(&self, f: &mut FieldSet, dt: f32) -> Result<(), ForgeError> {
        let ctx = f.hip_ctx(cells(&self.grid_dims))?;
        let p = sys::fh_sph_params {
            smoothing_radius: self.smoothing_radius,
            cell_size: self.cell_size,
            grid_dims: self.grid_dims,
            particle_mass: self.particle_mass,
            viscosity_coefficient: self.coefficient,
            ..Default::default()
        };
        check(unsafe {
            sys::fh_sph_viscosity(ctx, &p, f.f32_ptr("pos_x")?, f.f32_ptr("pos_y")?,
                                  f.f32_ptr("pos_z")?, f.f32_ptr("vel_x")?, f.f32_ptr("vel_y")?,
                                  f.f32_ptr("vel_z")?, f.f32_ptr("density")?,
                                  f.u32_ptr("cell_start")?, f.u32_ptr("sorted_indices")?,
                                  f.particle_count as u32, dt)
        })
    }
}

/// gravity.rs:5-9.
#[derive(Clone, Debug)]
pub struct GravityModule {
    pub gx: f32,
    pub gy: f32,
    pub gz: f32,
}

impl GravityModule {
    pub fn new(gx: f32, gy: f32, gz: f32) -> Self {
        GravityModule { gx, gy, gz }
    }
}

impl SimModule for GravityModule {
    fn name(&self) -> &str {
        "gravity"
    }
    fn execute(&self, f: &mut FieldSet, dt: f32) -> Result<(), ForgeError> {
        let ctx = f.hip_ctx(1)?;
        check(unsafe {
            sys::fh_gravity(ctx, f.f32_ptr("vel_x")?, f.f32_ptr("vel_y")?, f.f32_ptr("vel_z")?,
                            f.particle_count as u32, self.gx, self.gy, self.gz, dt)
        })
    }
    fn kind(&self) -> ModuleKind {
        ModuleKind::Gravity([self.gx, self.gy, self.gz])
    }
}

/// integrate.rs:5.
#[derive(Clone, Debug)]
pub struct IntegrateModule;

impl SimModule for IntegrateModule {
    fn name(&self) -> &str {
        "integrate"
    }
    fn execute(&self, f: &mut FieldSet, dt: f32) -> Result<(), ForgeError> {
        let ctx = f.hip_ctx(1)?;
        check(unsafe {
            sys::fh_integrate(ctx, f.f32_ptr("pos_x")?, f.f32_ptr("pos_y")?, f.f32_ptr("pos_z")?,
                              f.f32_ptr("vel_x")?, f.f32_ptr("vel_y")?, f.f32_ptr("vel_z")?,
                              f.particle_count as u32, dt)
        })
    }
    fn kind(&self) -> ModuleKind {
        ModuleKind::Integrate
    }
}

/// box_collider.rs:6-14.
#[derive(Clone, Debug)]
pub struct BoxColliderModule {
    pub min_x: f32,
    pub min_y: f32,
    pub min_z: f32,
    pub max_x: f32,
    pub max_y: f32,
    pub max_z: f32,
    pub restitution: f32,
}

impl SimModule for BoxColliderModule {
    fn name(&self) -> &str {
        "box_collider"
    }
    fn execute(&self, f: &mut FieldSet, _dt: f32) -> Result<(), ForgeError> {
        let ctx = f.hip_ctx(1)?;
        let mn = [self.min_x, self.min_y, self.min_z];
        let mx = [self.max_x, self.max_y, self.max_z];
        check(unsafe {
            sys::fh_box_collider(ctx, f.f32_ptr("pos_x")?, f.f32_ptr("pos_y")?,
                                 f.f32_ptr("pos_z")?, f.f32_ptr("vel_x")?, f.f32_ptr("vel_y")?,
                                 f.f32_ptr("vel_z")?, f.particle_count as u32, mn.as_ptr(),
                                 mx.as_ptr(), self.restitution)
        })
    }
    fn kind(&self) -> ModuleKind {
        ModuleKind::BoxCollider { min: mn3(self), max: mx3(self), restitution: self.restitution }
    }
}

fn mn3(b: &BoxColliderModule) -> [f32; 3] {
    [b.min_x, b.min_y, b.min_z]
}

fn mx3(b: &BoxColliderModule) -> [f32; 3] {
    [b.max_x, b.max_y, b.max_z]
}

/// The module order build_pipeline produces (fused SPH, gravity, integrate, box:
/// manifest_runner.rs:334-393, 508, 528-537), collapsed: a `SphFusedModule` directly followed by
/// any of gravity / integrate / box (in that order) takes them as its epilogue and they are
/// dropped.  Same results as running them one after the other, one pass fewer.
pub fn fuse_epilogue(modules: Vec<Box<dyn SimModule>>) -> Vec<Box<dyn SimModule>> {
    let kinds: Vec<ModuleKind> = modules.iter().map(|m| m.kind()).collect();
    let mut out: Vec<Box<dyn SimModule>> = Vec::with_capacity(modules.len());
    let mut skip = 0usize;
    for (i, m) in modules.into_iter().enumerate() {
        if skip > 0 {
            skip -= 1;
            continue;
        }
        let sph = match &kinds[i] {
            ModuleKind::SphFused(s) if s.epilogue.is_none() => s.clone(),
            _ => {
                out.push(m);
                continue;
            }
        };
        let mut epi = sys::fh_epilogue::default();
        let mut j = i + 1;
        if let Some(ModuleKind::Gravity(g)) = kinds.get(j) {
            epi.flags |= sys::FH_EPI_GRAVITY;
            epi.gravity = *g;
            j += 1;
        }
        if let Some(ModuleKind::Integrate) = kinds.get(j) {
            epi.flags |= sys::FH_EPI_INTEGRATE;
            j += 1;
        }
        if let Some(ModuleKind::BoxCollider { min, max, restitution }) = kinds.get(j) {
            epi.flags |= sys::FH_EPI_BOX;
            epi.box_min = *min;
            epi.box_max = *max;
            epi.restitution = *restitution;
            j += 1;
        }
        if j == i + 1 {
            out.push(m);
        } else {
            let mut fused = sph;
            fused.epilogue = Some(epi);
            out.push(Box::new(fused));
            skip = j - i - 1;
        }
    }
    out
}

/// modules/mod.rs:76-117, with graph capture / replay (manifest_runner.rs:53-77).
pub struct Pipeline {
    modules: Vec<Box<dyn SimModule>>,
    /// run `steps` substeps of a pipeline that is one fused SPH module as one resident call
    pub resident: bool,
}

impl Default for Pipeline {
    fn default() -> Self {
        Pipeline::new()
    }
}

impl Pipeline {
    pub fn new() -> Self {
        Pipeline { modules: Vec::new(), resident: true }
    }

    pub fn add(&mut self, module: Box<dyn SimModule>) {
        self.modules.push(module);
    }

    pub fn len(&self) -> usize {
        self.modules.len()
    }

    pub fn is_empty(&self) -> bool {
        self.modules.is_empty()
    }

    /// Replace the modules by their fused form (`fuse_epilogue`); build_pipeline's output is
    /// already in the order this expects.
    pub fn fuse(&mut self) {
        let m = std::mem::take(&mut self.modules);
        self.modules = fuse_epilogue(m);
    }

    /// modules/mod.rs:90-95.
    pub fn step_async(&self, fields: &mut FieldSet, dt: f32) -> Result<(), ForgeError> {
        for m in &self.modules {
            m.execute(fields, dt)?;
        }
        Ok(())
    }

    /// modules/mod.rs:98-104.
    pub fn step(&self, fields: &mut FieldSet, dt: f32) -> Result<(), ForgeError> {
        self.step_async(fields, dt)?;
        fields.sync()
    }

    /// `steps` substeps queued: one resident fh_sph_fused_steps call when the pipeline is a
    /// single fused SPH module (nothing reads the fields in between), else step by step.
    pub fn run_async(&self, fields: &mut FieldSet, dt: f32, steps: usize)
                     -> Result<(), ForgeError> {
        if self.resident && steps > 1 && self.modules.len() == 1 {
            if let ModuleKind::SphFused(s) = self.modules[0].kind() {
                return s.execute_steps(fields, dt, steps as u32);
            }
        }
        for _ in 0..steps {
            self.step_async(fields, dt)?;
        }
        Ok(())
    }

    /// modules/mod.rs:106-112.
    pub fn run(&self, fields: &mut FieldSet, dt: f32, steps: usize) -> Result<(), ForgeError> {
        self.run_async(fields, dt, steps)?;
        fields.sync()
    }

    /// Record `substeps` substeps into the context's graph (manifest_runner.rs:57-69).  Every
    /// field the modules write must exist (run one `step` first).
    pub fn capture(&self, fields: &mut FieldSet, dt: f32, substeps: usize,
                   num_cells: usize) -> Result<(), ForgeError> {
        let ctx = fields.hip_ctx(num_cells)?;
        fields.sync()?;
        check(unsafe { sys::fh_graph_begin(ctx) })?;
        let r = self.run_async(fields, dt, substeps);
        let e = check(unsafe { sys::fh_graph_end(ctx) });
        r.and(e)
    }

    /// Replay the captured graph `count` times (manifest_runner.rs:74-77).
    pub fn replay(&self, fields: &FieldSet, count: u32, num_cells: usize)
                  -> Result<(), ForgeError> {
        let ctx = fields.hip_ctx(num_cells)?;
        check(unsafe { sys::fh_graph_launch(ctx, count) })
    }
}
