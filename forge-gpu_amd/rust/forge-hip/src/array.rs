//! Device buffers.  `Array<T>` is an owned HIP allocation with the reference's constructors
//! (`zeros`, `from_vec`, `to_vec`; forge-runtime/src/array.rs:193-214,286-308,366-406).  The
//! wrappers only need [`DevicePtr`]: a forge-runtime that keeps its own `Array<T>` implements it
//! and passes its buffers unchanged.

use std::marker::PhantomData;
use std::os::raw::{c_int, c_void};

use forge_hip_sys::hip;

use crate::error::{check_hip, ForgeError};

/// Where an array lives (forge-runtime/src/device.rs).  The GPU path takes `Gpu(ordinal)`.
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Device {
    Cpu,
    Gpu(usize),
}

impl Device {
    pub fn ordinal(&self) -> Result<usize, ForgeError> {
        match self {
            Device::Gpu(o) => Ok(*o),
            Device::Cpu => Err(ForgeError::WrongDevice("a device buffer is required".into())),
        }
    }
}

/// forge-core's `Vec3f`: `#[repr(C)]` 3 x f32, 12 bytes (forge-core/src/vec.rs:137-139).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default, PartialEq)]
pub struct Vec3f {
    pub x: f32,
    pub y: f32,
    pub z: f32,
}

impl Vec3f {
    pub fn new(x: f32, y: f32, z: f32) -> Self {
        Vec3f { x, y, z }
    }
    pub fn zero() -> Self {
        Vec3f::default()
    }
}

/// A buffer in device memory: what every wrapper passes to the C ABI.
pub trait DevicePtr<T> {
    fn device_ptr(&self) -> *const T;
    fn device_ptr_mut(&mut self) -> *mut T;
    fn len(&self) -> usize;
    fn is_empty(&self) -> bool {
        self.len() == 0
    }
}

/// Owned device buffer of `len` elements of `T` (RAII `hipMalloc` / `hipFree`); host transfers
/// are synchronous, as the reference's `from_vec` / `to_vec`.
pub struct Array<T: Copy> {
    ptr: *mut T,
    len: usize,
    device: Device,
    _t: PhantomData<T>,
}

// The buffer is plain device memory; the reference's Array is Send + Sync as well.
unsafe impl<T: Copy + Send> Send for Array<T> {}
unsafe impl<T: Copy + Sync> Sync for Array<T> {}

impl<T: Copy> Array<T> {
    fn alloc(len: usize, device: Device) -> Result<Self, ForgeError> {
        let ordinal = device.ordinal()?;
        let mut p: *mut c_void = std::ptr::null_mut();
        if len > 0 {
            check_hip(unsafe { hip::hipSetDevice(ordinal as c_int) }, "hipSetDevice")?;
            check_hip(unsafe { hip::hipMalloc(&mut p, len * std::mem::size_of::<T>()) },
                      "hipMalloc")?;
        }
        Ok(Array { ptr: p as *mut T, len, device, _t: PhantomData })
    }

    /// `len` zero-filled elements (array.rs:193-214).
    pub fn zeros(len: usize, device: Device) -> Self {
        Self::try_zeros(len, device).expect("Array::zeros")
    }

    pub fn try_zeros(len: usize, device: Device) -> Result<Self, ForgeError> {
        let a = Self::alloc(len, device)?;
        if len > 0 {
            check_hip(unsafe {
                hip::hipMemset(a.ptr as *mut c_void, 0, len * std::mem::size_of::<T>())
            }, "hipMemset")?;
        }
        Ok(a)
    }

    /// Upload `data` (array.rs:286-308).
    pub fn from_vec(data: Vec<T>, device: Device) -> Self {
        Self::from_slice(&data, device)
    }

    pub fn from_slice(data: &[T], device: Device) -> Self {
        Self::try_from_slice(data, device).expect("Array::from_slice")
    }

    pub fn try_from_slice(data: &[T], device: Device) -> Result<Self, ForgeError> {
        let a = Self::alloc(data.len(), device)?;
        if !data.is_empty() {
            check_hip(unsafe {
                hip::hipMemcpy(a.ptr as *mut c_void, data.as_ptr() as *const c_void,
                               data.len() * std::mem::size_of::<T>(),
                               hip::HIP_MEMCPY_HOST_TO_DEVICE)
            }, "hipMemcpy")?;
        }
        Ok(a)
    }

    /// Download (array.rs:366-406).  Waits for the device (hipMemcpy is synchronous).
    pub fn to_vec(&self) -> Vec<T> {
        self.try_to_vec().expect("Array::to_vec")
    }

    pub fn try_to_vec(&self) -> Result<Vec<T>, ForgeError> {
        let mut v: Vec<T> = Vec::with_capacity(self.len);
        if self.len > 0 {
            check_hip(unsafe {
                hip::hipMemcpy(v.as_mut_ptr() as *mut c_void, self.ptr as *const c_void,
                               self.len * std::mem::size_of::<T>(),
                               hip::HIP_MEMCPY_DEVICE_TO_HOST)
            }, "hipMemcpy")?;
            // the copy above initialised all `len` elements
            unsafe { v.set_len(self.len) };
        }
        Ok(v)
    }

    pub fn len(&self) -> usize {
        self.len
    }

    pub fn is_empty(&self) -> bool {
        self.len == 0
    }

    pub fn device(&self) -> Device {
        self.device
    }
}

impl<T: Copy> Drop for Array<T> {
    fn drop(&mut self) {
        if !self.ptr.is_null() {
            unsafe {
                let _ = hip::hipFree(self.ptr as *mut c_void);
            }
        }
    }
}

impl<T: Copy> DevicePtr<T> for Array<T> {
    fn device_ptr(&self) -> *const T {
        self.ptr
    }
    fn device_ptr_mut(&mut self) -> *mut T {
        self.ptr
    }
    fn len(&self) -> usize {
        self.len
    }
}
