//! Raw declarations of the C ABI of `libforge_hip.so` (`include/forge_hip.h`), the MI355X
//! (gfx950) SPH / hash-grid hot path that replaces forge-gpu's NVRTC-compiled kernels.
//!
//! Conventions (see the header for each entry point):
//! * return value: 0 = ok, < 0 = argument / state error (`FH_E*`), > 0 = a `hipError_t`;
//!   `fh_last_error()` is a thread-local message, never NULL; nothing unwinds across the ABI;
//! * every buffer is a device pointer owned by the caller; the context owns its scratch, its
//!   stream and its captured graph;
//! * compute calls are asynchronous on `fh_stream(ctx)`; `fh_sync` waits (and reports the
//!   device-side error flag);
//! * `fh_create` allocates every scratch buffer, so any later call may be captured into a graph.
//!
//! The wrappers with forge-gpu's names (`HashGrid`, `RadixSorter`, `SimModule`, ...) are in the
//! `forge-hip` crate next to this one.
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

pub const FH_ABI_VERSION: c_int = 3;

pub const FH_OK: c_int = 0;
pub const FH_EINVAL: c_int = -1;
pub const FH_ERANGE: c_int = -2;
pub const FH_ESTATE: c_int = -3;
pub const FH_ENODEV: c_int = -4;

pub const FH_EPI_GRAVITY: u32 = 1;
pub const FH_EPI_INTEGRATE: u32 = 2;
pub const FH_EPI_BOX: u32 = 4;

pub const FH_OPT_SPH_EXACT: c_int = 1;
pub const FH_OPT_HEAVY_WORK: c_int = 2;
pub const FH_OPT_DIRECT_ITEMS: c_int = 3;
pub const FH_OPT_HEAVY_PARTS: c_int = 4;
pub const FH_OPT_EPOCH_PERIOD: c_int = 5;
pub const FH_OPT_SPIN_LIMIT: c_int = 6;
pub const FH_OPT_HEAVY_SLOTS: c_int = 7;
pub const FH_OPT_SUBCELL: c_int = 8;

pub const FH_NOALLOC_MAX_N: u32 = 1_048_576;
pub const FH_NOALLOC_SCRATCH_BYTES: u32 = 19_939_328;

/// Opaque context (stream, scratch, graph).
#[repr(C)]
pub struct fh_ctx {
    _private: [u8; 0],
}

/// `SphFusedModule`'s parameters (forge-manifest/src/modules/builtins/sph_fused.rs:14-22).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq)]
pub struct fh_sph_params {
    pub smoothing_radius: f32,
    pub cell_size: f32,
    pub grid_dims: [u32; 3],
    pub particle_mass: f32,
    pub gas_constant: f32,
    pub rest_density: f32,
    pub viscosity_coefficient: f32,
}

/// Gravity / integrate / box steps fused after the SPH velocity update.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq)]
pub struct fh_epilogue {
    pub flags: u32,
    pub gravity: [f32; 3],
    pub box_min: [f32; 3],
    pub box_max: [f32; 3],
    pub restitution: f32,
}

extern "C" {
    // ---- context ----
    pub fn fh_create(device: c_int, max_n: u32, max_cells: u32, stream: *mut c_void,
                     out: *mut *mut fh_ctx) -> c_int;
    pub fn fh_destroy(ctx: *mut fh_ctx) -> c_int;
    pub fn fh_stream(ctx: *mut fh_ctx) -> *mut c_void;
    pub fn fh_sync(ctx: *mut fh_ctx) -> c_int;
    pub fn fh_last_error() -> *const c_char;
    pub fn fh_abi_version() -> c_int;
    pub fn fh_scratch_bytes(ctx: *const fh_ctx) -> usize;

    // ---- hashing and sorting ----
    pub fn fh_hash_cells(ctx: *mut fh_ctx, x: *const f32, y: *const f32, z: *const f32,
                         stride: u32, n: u32, cell_size: f32, origin: *const f32,
                         dims: *const u32, keys: *mut u32, vals: *mut u32) -> c_int;
    pub fn fh_sort_pairs(ctx: *mut fh_ctx, keys: *mut u32, vals: *mut u32, n: u32,
                         num_bits: u32) -> c_int;
    pub fn fh_sort_plan(ctx: *mut fh_ctx, plan: *mut u32) -> c_int;
    pub fn fh_sort_pairs_noalloc(stream: *mut c_void, keys: *mut u32, vals: *mut u32, n: u32,
                                 num_bits: u32) -> c_int;
    pub fn fh_noalloc_status(stream: *mut c_void) -> c_int;
    pub fn fh_find_cell_boundaries(ctx: *mut fh_ctx, sorted_keys: *const u32, n: u32,
                                   num_cells: u32, cell_start: *mut u32,
                                   cell_end: *mut u32) -> c_int;
    pub fn fh_cell_start_csr(ctx: *mut fh_ctx, sorted_keys: *const u32, n: u32, num_cells: u32,
                             cell_start: *mut u32) -> c_int;

    // ---- hash grid ----
    pub fn fh_hashgrid_build(ctx: *mut fh_ctx, x: *const f32, y: *const f32, z: *const f32,
                             stride: u32, n: u32, cell_size: f32, origin: *const f32,
                             dims: *const u32, cell_start: *mut u32, sorted_indices: *mut u32,
                             cell_indices: *mut u32) -> c_int;
    pub fn fh_neighbor_query(ctx: *mut fh_ctx, x: *const f32, y: *const f32, z: *const f32,
                             stride: u32, n: u32, cell_size: f32, origin: *const f32,
                             dims: *const u32, cell_start: *const u32,
                             sorted_indices: *const u32, radius: f32, counts: *mut u32,
                             wsum: *mut f32) -> c_int;
    pub fn fh_query_neighbors(ctx: *mut fh_ctx, x: *const f32, y: *const f32, z: *const f32,
                              stride: u32, cell_size: f32, origin: *const f32, dims: *const u32,
                              cell_start: *const u32, sorted_indices: *const u32,
                              qx: *const f32, qy: *const f32, qz: *const f32, qstride: u32,
                              nq: u32, radius: f32, counts: *mut u32, offsets: *const u32,
                              indices: *mut u32) -> c_int;

    // ---- SPH modules ----
    pub fn fh_sph_density(ctx: *mut fh_ctx, prm: *const fh_sph_params, px: *const f32,
                          py: *const f32, pz: *const f32, n: u32, density: *mut f32,
                          cell_start: *mut u32, sorted_indices: *mut u32) -> c_int;
    pub fn fh_sph_pressure(ctx: *mut fh_ctx, prm: *const fh_sph_params, px: *const f32,
                           py: *const f32, pz: *const f32, vx: *mut f32, vy: *mut f32,
                           vz: *mut f32, density: *const f32, cell_start: *const u32,
                           sorted_indices: *const u32, n: u32, dt: f32) -> c_int;
    pub fn fh_sph_viscosity(ctx: *mut fh_ctx, prm: *const fh_sph_params, px: *const f32,
                            py: *const f32, pz: *const f32, vx: *mut f32, vy: *mut f32,
                            vz: *mut f32, density: *const f32, cell_start: *const u32,
                            sorted_indices: *const u32, n: u32, dt: f32) -> c_int;
    pub fn fh_sph_fused(ctx: *mut fh_ctx, prm: *const fh_sph_params, epi: *const fh_epilogue,
                        px: *mut f32, py: *mut f32, pz: *mut f32, vx: *mut f32, vy: *mut f32,
                        vz: *mut f32, density: *mut f32, accel: *mut f32, n: u32,
                        dt: f32) -> c_int;
    pub fn fh_sph_force(ctx: *mut fh_ctx, prm: *const fh_sph_params, px: *const f32,
                        py: *const f32, pz: *const f32, vx: *mut f32, vy: *mut f32, vz: *mut f32,
                        density: *const f32, cell_start: *const u32, sorted_indices: *const u32,
                        accel: *mut f32, n: u32, dt: f32) -> c_int;
    pub fn fh_sph_fused_steps(ctx: *mut fh_ctx, prm: *const fh_sph_params,
                              epi: *const fh_epilogue, px: *mut f32, py: *mut f32, pz: *mut f32,
                              vx: *mut f32, vy: *mut f32, vz: *mut f32, density: *mut f32,
                              accel: *mut f32, n: u32, dt: f32, steps: u32) -> c_int;
    pub fn fh_set_option(ctx: *mut fh_ctx, option: c_int, value: c_int) -> c_int;
    pub fn fh_gravity(ctx: *mut fh_ctx, vx: *mut f32, vy: *mut f32, vz: *mut f32, n: u32,
                      gx: f32, gy: f32, gz: f32, dt: f32) -> c_int;
    pub fn fh_integrate(ctx: *mut fh_ctx, px: *mut f32, py: *mut f32, pz: *mut f32,
                        vx: *mut f32, vy: *mut f32, vz: *mut f32, n: u32, dt: f32) -> c_int;
    pub fn fh_box_collider(ctx: *mut fh_ctx, px: *mut f32, py: *mut f32, pz: *mut f32,
                           vx: *mut f32, vy: *mut f32, vz: *mut f32, n: u32,
                           box_min: *const f32, box_max: *const f32, restitution: f32) -> c_int;

    // ---- frames ----
    pub fn fh_pack_frame(ctx: *mut fh_ctx, px: *const f32, py: *const f32, pz: *const f32,
                         n: u32, frame: u32, frame_counter: *mut u32, out: *mut c_void) -> c_int;

    // ---- graphs ----
    pub fn fh_graph_begin(ctx: *mut fh_ctx) -> c_int;
    pub fn fh_graph_end(ctx: *mut fh_ctx) -> c_int;
    pub fn fh_graph_launch(ctx: *mut fh_ctx, count: u32) -> c_int;

    // ---- timing ----
    pub fn fh_event_record(ctx: *mut fh_ctx, slot: u32) -> c_int;
    pub fn fh_event_elapsed_ms(ctx: *mut fh_ctx, slot_start: u32, slot_end: u32,
                               ms: *mut f32) -> c_int;
    pub fn fh_time_kernel(ctx: *mut fh_ctx, name: *const c_char, max_launches: u32) -> c_int;
    pub fn fh_kernel_times(ctx: *mut fh_ctx, name: *const c_char, ms: *mut f32, cap: u32,
                           count: *mut u32) -> c_int;
}

/// The few HIP runtime calls the safe wrappers need for their own device buffers
/// (`forge_hip::Array`): allocation, fill, host transfers.  A forge-runtime that keeps its own
/// `Array<T>` does not need them.
pub mod hip {
    use std::os::raw::{c_int, c_void};

    pub const HIP_MEMCPY_HOST_TO_DEVICE: c_int = 1;
    pub const HIP_MEMCPY_DEVICE_TO_HOST: c_int = 2;

    extern "C" {
        pub fn hipSetDevice(device: c_int) -> c_int;
        pub fn hipMalloc(ptr: *mut *mut c_void, size: usize) -> c_int;
        pub fn hipFree(ptr: *mut c_void) -> c_int;
        pub fn hipMemset(dst: *mut c_void, value: c_int, size: usize) -> c_int;
        pub fn hipMemcpy(dst: *mut c_void, src: *const c_void, size: usize, kind: c_int) -> c_int;
    }
}
