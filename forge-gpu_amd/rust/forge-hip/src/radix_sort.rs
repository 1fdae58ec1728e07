//! `RadixSorter` and `find_cell_boundaries` with the reference's signatures
//! (forge-runtime/src/radix_sort.rs:55-220, 229-317).  The sort is stable and in place (no
//! buffer swap); any 1..32 bits is accepted (the reference required a multiple of 4) and
//! n > max_n is an error instead of a panic.

use forge_hip_sys as sys;

use crate::array::DevicePtr;
use crate::context::Ctx;
use crate::error::{check, ForgeError};

pub struct RadixSorter {
    max_n: usize,
    ctx: Ctx,
}

impl RadixSorter {
    /// radix_sort.rs:55-70: all scratch allocated here (graph-capture safe afterwards).
    pub fn new(max_n: usize, ordinal: usize) -> Self {
        Self::try_new(max_n, ordinal).expect("RadixSorter::new")
    }

    pub fn try_new(max_n: usize, ordinal: usize) -> Result<Self, ForgeError> {
        Ok(RadixSorter { max_n, ctx: Ctx::new(ordinal, max_n.max(1), 1)? })
    }

    pub fn max_n(&self) -> usize {
        self.max_n
    }

    /// radix_sort.rs:79-220: sort (keys, values) in place by the low `num_bits` bits of the
    /// keys, equal keys in input order; waits for the result.
    pub fn sort<K: DevicePtr<u32>, V: DevicePtr<u32>>(&mut self, keys: &mut K, values: &mut V,
                                                       n: usize, num_bits: u32)
                                                       -> Result<(), ForgeError> {
        self.sort_async(keys, values, n, num_bits)?;
        self.ctx.sync()
    }

    /// The same without waiting (the call is queued on the sorter's stream).
    pub fn sort_async<K: DevicePtr<u32>, V: DevicePtr<u32>>(&mut self, keys: &mut K,
                                                             values: &mut V, n: usize,
                                                             num_bits: u32)
                                                             -> Result<(), ForgeError> {
        if n > keys.len() || n > values.len() {
            return Err(ForgeError::LaunchFailed("sort: n exceeds the buffers".into()));
        }
        if n > u32::MAX as usize {
            return Err(ForgeError::LaunchFailed("sort: n exceeds u32".into()));
        }
        check(unsafe {
            sys::fh_sort_pairs(self.ctx.raw(), keys.device_ptr_mut(), values.device_ptr_mut(),
                               n as u32, num_bits)
        })
    }

    pub fn context(&self) -> &Ctx {
        &self.ctx
    }
}

/// radix_sort.rs:229-317: from keys sorted ascending, cell_start[c] = first index with key c,
/// cell_end[c] = last index + 1; empty cells keep 0xFFFFFFFF / 0.  Keys >= num_cells are
/// ignored (the reference kernel wrote out of bounds).  Like the reference (which compiled its
/// kernels and set the outputs with memset launches on every call) this is a one-off helper: it
/// makes a context for the call; loops should keep a `Ctx` and call `fh_find_cell_boundaries`.
pub fn find_cell_boundaries<S, A, B>(sorted_cell_ids: &S, cell_start: &mut A, cell_end: &mut B,
                                     n: usize, num_cells: usize, ordinal: usize)
                                     -> Result<(), ForgeError>
where
    S: DevicePtr<u32>,
    A: DevicePtr<u32>,
    B: DevicePtr<u32>,
{
    if n > sorted_cell_ids.len() || num_cells > cell_start.len() || num_cells > cell_end.len() {
        return Err(ForgeError::LaunchFailed("find_cell_boundaries: buffers too small".into()));
    }
    let ctx = Ctx::new(ordinal, n.max(1), num_cells.max(1))?;
    check(unsafe {
        sys::fh_find_cell_boundaries(ctx.raw(), sorted_cell_ids.device_ptr(), n as u32,
                                     num_cells as u32, cell_start.device_ptr_mut(),
                                     cell_end.device_ptr_mut())
    })?;
    ctx.sync()
}
