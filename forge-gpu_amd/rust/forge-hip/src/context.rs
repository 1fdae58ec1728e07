//! `Ctx`: an owned `fh_ctx` (stream, scratch, captured graph), the counterpart of the
//! reference's per-ordinal stream (forge-runtime/src/cuda.rs:13-63) plus the scratch that
//! `SphFusedModule` creates lazily in the FieldSet (sph_fused.rs:43-74) and that `RadixSorter::new`
//! allocates (radix_sort.rs:55-70).

use std::os::raw::{c_int, c_void};

use forge_hip_sys as sys;

use crate::error::{check, check_sync, ForgeError};

pub struct Ctx {
    raw: *mut sys::fh_ctx,
    max_n: usize,
    max_cells: usize,
    ordinal: usize,
}

// A context is used by one thread at a time (the C ABI's rule); moving it between threads is fine.
unsafe impl Send for Ctx {}

impl Ctx {
    /// A context on device `ordinal` for up to `max_n` particles / pairs and `max_cells` cells,
    /// with a private stream.  Every scratch buffer is allocated here.
    pub fn new(ordinal: usize, max_n: usize, max_cells: usize) -> Result<Self, ForgeError> {
        Self::with_stream(ordinal, max_n, max_cells, std::ptr::null_mut())
    }

    /// The same on the caller's `hipStream_t`.
    pub fn with_stream(ordinal: usize, max_n: usize, max_cells: usize,
                       stream: *mut c_void) -> Result<Self, ForgeError> {
        if max_n > u32::MAX as usize || max_cells > u32::MAX as usize {
            return Err(ForgeError::LaunchFailed("max_n / max_cells exceed u32".into()));
        }
        let mut raw: *mut sys::fh_ctx = std::ptr::null_mut();
        check(unsafe {
            sys::fh_create(ordinal as c_int, max_n as u32, max_cells as u32, stream, &mut raw)
        })?;
        Ok(Ctx { raw, max_n, max_cells, ordinal })
    }

    pub fn raw(&self) -> *mut sys::fh_ctx {
        self.raw
    }
    pub fn max_n(&self) -> usize {
        self.max_n
    }
    pub fn max_cells(&self) -> usize {
        self.max_cells
    }
    pub fn ordinal(&self) -> usize {
        self.ordinal
    }
    /// The `hipStream_t` every call is queued on.
    pub fn stream(&self) -> *mut c_void {
        unsafe { sys::fh_stream(self.raw) }
    }
    /// Wait for the stream; reports device-side failures (Pipeline::step's sync,
    /// modules/mod.rs:98-104).
    pub fn sync(&self) -> Result<(), ForgeError> {
        check_sync(unsafe { sys::fh_sync(self.raw) })
    }
    pub fn set_option(&self, option: c_int, value: c_int) -> Result<(), ForgeError> {
        check(unsafe { sys::fh_set_option(self.raw, option, value) })
    }
    pub fn scratch_bytes(&self) -> usize {
        unsafe { sys::fh_scratch_bytes(self.raw) }
    }
    pub fn graph_begin(&self) -> Result<(), ForgeError> {
        check(unsafe { sys::fh_graph_begin(self.raw) })
    }
    pub fn graph_end(&self) -> Result<(), ForgeError> {
        check(unsafe { sys::fh_graph_end(self.raw) })
    }
    pub fn graph_launch(&self, count: u32) -> Result<(), ForgeError> {
        check(unsafe { sys::fh_graph_launch(self.raw, count) })
    }
}

impl Drop for Ctx {
    fn drop(&mut self) {
        if !self.raw.is_null() {
            unsafe {
                let _ = sys::fh_destroy(self.raw);
            }
        }
    }
}
