//! `HashGrid` with the reference's fields and methods (forge-runtime/src/hashgrid.rs:21-193).
//! `build` runs on the GPU (fh_hashgrid_build: hash, stable radix sort, CSR cell ranges) instead
//! of the reference's serial CPU counting sort; the outputs are bit-identical to it.

use forge_hip_sys as sys;

use crate::array::{Array, Device, DevicePtr, Vec3f};
use crate::context::Ctx;
use crate::error::{check, ForgeError};

pub struct HashGrid {
    /// Cell size (same in all dimensions).
    pub cell_size: f32,
    pub dim_x: u32,
    pub dim_y: u32,
    pub dim_z: u32,
    /// Lower corner of the grid.
    pub origin: Vec3f,
    /// CSR cell ranges, num_cells + 1 entries: particles of cell c are
    /// sorted_indices[cell_start[c] .. cell_start[c + 1]].
    pub cell_start: Array<u32>,
    /// Particle ids ordered by cell, ascending id within a cell.
    pub sorted_indices: Array<u32>,
    /// Cell of each particle.
    pub cell_indices: Array<u32>,
    pub num_particles: usize,
    device: Device,
    ctx: Ctx,
    /// Device copy of the positions of the last `build` (what the queries read).
    positions: Option<Array<Vec3f>>,
}

impl HashGrid {
    /// hashgrid.rs:50-72.  Panics like the reference when the device cannot be used.
    pub fn new(cell_size: f32, grid_dims: (u32, u32, u32), origin: Vec3f,
               max_particles: usize, device: Device) -> Self {
        Self::try_new(cell_size, grid_dims, origin, max_particles, device)
            .expect("HashGrid::new")
    }

    pub fn try_new(cell_size: f32, grid_dims: (u32, u32, u32), origin: Vec3f,
                   max_particles: usize, device: Device) -> Result<Self, ForgeError> {
        let (dim_x, dim_y, dim_z) = grid_dims;
        let num_cells = dim_x as usize * dim_y as usize * dim_z as usize;
        let ctx = Ctx::new(device.ordinal()?, max_particles.max(1), num_cells.max(1))?;
        Ok(HashGrid {
            cell_size,
            dim_x,
            dim_y,
            dim_z,
            origin,
            cell_start: Array::try_zeros(num_cells + 1, device)?,
            sorted_indices: Array::try_zeros(max_particles, device)?,
            cell_indices: Array::try_zeros(max_particles, device)?,
            num_particles: 0,
            device,
            ctx,
            positions: None,
        })
    }

    /// hashgrid.rs:75-77.
    pub fn num_cells(&self) -> usize {
        self.dim_x as usize * self.dim_y as usize * self.dim_z as usize
    }

    fn dims(&self) -> [u32; 3] {
        [self.dim_x, self.dim_y, self.dim_z]
    }

    fn origin3(&self) -> [f32; 3] {
        [self.origin.x, self.origin.y, self.origin.z]
    }

    /// hashgrid.rs:82-125: uploads `positions` once and builds the grid on the GPU.
    pub fn build(&mut self, positions: &[Vec3f]) -> Result<(), ForgeError> {
        let pos = Array::try_from_slice(positions, self.device)?;
        self.build_device(&pos, positions.len())?;
        self.positions = Some(pos);
        Ok(())
    }

    /// The same from positions already on the device (a 12-byte Vec3f array, stride 3 floats).
    pub fn build_device<P: DevicePtr<Vec3f>>(&mut self, pos: &P, n: usize)
                                             -> Result<(), ForgeError> {
        if n > self.sorted_indices.len() || n > pos.len() {
            return Err(ForgeError::LaunchFailed(format!(
                "HashGrid::build: {} particles, room for {}", n, self.sorted_indices.len())));
        }
        let p = pos.device_ptr() as *const f32;
        let (o, d) = (self.origin3(), self.dims());
        check(unsafe {
            sys::fh_hashgrid_build(self.ctx.raw(), p, p.add(1), p.add(2), 3, n as u32,
                                   self.cell_size, o.as_ptr(), d.as_ptr(),
                                   self.cell_start.device_ptr_mut(),
                                   self.sorted_indices.device_ptr_mut(),
                                   self.cell_indices.device_ptr_mut())
        })?;
        self.ctx.sync()?;
        self.num_particles = n;
        Ok(())
    }

    /// hashgrid.rs:128-139 on the host (Rust `as i32` saturates, NaN -> 0, as on the device).
    pub fn position_to_cell(&self, pos: Vec3f) -> u32 {
        let cx = ((pos.x - self.origin.x) / self.cell_size).floor() as i32;
        let cy = ((pos.y - self.origin.y) / self.cell_size).floor() as i32;
        let cz = ((pos.z - self.origin.z) / self.cell_size).floor() as i32;
        let cx = cx.max(0).min(self.dim_x as i32 - 1) as u32;
        let cy = cy.max(0).min(self.dim_y as i32 - 1) as u32;
        let cz = cz.max(0).min(self.dim_z as i32 - 1) as u32;
        cx.wrapping_add(cy.wrapping_mul(self.dim_x))
            .wrapping_add(cz.wrapping_mul(self.dim_x).wrapping_mul(self.dim_y))
    }

    /// hashgrid.rs:145-193: the particles within `radius` of `pos` (`<=`, self included), in the
    /// reference's visiting order.  The query runs on the GPU against the positions of the last
    /// `build`; `positions` must be those positions (it is only checked for length).
    pub fn query_neighbors(&self, pos: Vec3f, radius: f32, positions: &[Vec3f]) -> Vec<u32> {
        assert_eq!(positions.len(), self.num_particles,
                   "query_neighbors: positions differ from the last build");
        self.query_neighbors_batch(&[pos], radius)
            .expect("HashGrid::query_neighbors")
            .pop()
            .unwrap_or_default()
    }

    /// Neighbour lists of many query points in two GPU calls (counts, then ids).
    pub fn query_neighbors_batch(&self, queries: &[Vec3f], radius: f32)
                                 -> Result<Vec<Vec<u32>>, ForgeError> {
        let pts = self.positions.as_ref().ok_or_else(|| {
            ForgeError::LaunchFailed("query before a host-side build".into())
        })?;
        let nq = queries.len();
        if nq == 0 {
            return Ok(Vec::new());
        }
        let q = Array::try_from_slice(queries, self.device)?;
        let mut counts = Array::<u32>::try_zeros(nq, self.device)?;
        let p = pts.device_ptr() as *const f32;
        let qp = q.device_ptr() as *const f32;
        let (o, d) = (self.origin3(), self.dims());
        check(unsafe {
            sys::fh_query_neighbors(self.ctx.raw(), p, p.add(1), p.add(2), 3, self.cell_size,
                                    o.as_ptr(), d.as_ptr(), self.cell_start.device_ptr(),
                                    self.sorted_indices.device_ptr(), qp, qp.add(1), qp.add(2),
                                    3, nq as u32, radius, counts.device_ptr_mut(),
                                    std::ptr::null(), std::ptr::null_mut())
        })?;
        self.ctx.sync()?;
        let c = counts.try_to_vec()?;
        let mut offs = Vec::with_capacity(nq + 1);
        let mut total: u64 = 0;
        offs.push(0u32);
        for &k in &c {
            total += k as u64;
            if total > u32::MAX as u64 {
                return Err(ForgeError::LaunchFailed("more than 2^32 neighbours".into()));
            }
            offs.push(total as u32);
        }
        let offsets = Array::try_from_slice(&offs, self.device)?;
        let mut ids = Array::<u32>::try_zeros((total as usize).max(1), self.device)?;
        check(unsafe {
            sys::fh_query_neighbors(self.ctx.raw(), p, p.add(1), p.add(2), 3, self.cell_size,
                                    o.as_ptr(), d.as_ptr(), self.cell_start.device_ptr(),
                                    self.sorted_indices.device_ptr(), qp, qp.add(1), qp.add(2),
                                    3, nq as u32, radius, counts.device_ptr_mut(),
                                    offsets.device_ptr(), ids.device_ptr_mut())
        })?;
        self.ctx.sync()?;
        let flat = ids.try_to_vec()?;
        Ok((0..nq)
            .map(|i| flat[offs[i] as usize..offs[i + 1] as usize].to_vec())
            .collect())
    }

    /// Per-point neighbour counts and poly6 weight sums of every built point (configs[2]'s
    /// query): one GPU pass, results in point order.
    pub fn neighbor_counts(&self, radius: f32) -> Result<(Vec<u32>, Vec<f32>), ForgeError> {
        let pts = self.positions.as_ref().ok_or_else(|| {
            ForgeError::LaunchFailed("query before a host-side build".into())
        })?;
        let n = self.num_particles;
        let mut counts = Array::<u32>::try_zeros(n, self.device)?;
        let mut wsum = Array::<f32>::try_zeros(n, self.device)?;
        let p = pts.device_ptr() as *const f32;
        let (o, d) = (self.origin3(), self.dims());
        check(unsafe {
            sys::fh_neighbor_query(self.ctx.raw(), p, p.add(1), p.add(2), 3, n as u32,
                                   self.cell_size, o.as_ptr(), d.as_ptr(),
                                   self.cell_start.device_ptr(), self.sorted_indices.device_ptr(),
                                   radius, counts.device_ptr_mut(), wsum.device_ptr_mut())
        })?;
        self.ctx.sync()?;
        Ok((counts.try_to_vec()?, wsum.try_to_vec()?))
    }
}
