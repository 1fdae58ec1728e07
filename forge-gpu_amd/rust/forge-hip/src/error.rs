//! `ForgeError` with the reference's variants (`forge-runtime/src/error.rs:7-22`), and the
//! mapping of the C ABI's return codes onto them.

use std::ffi::CStr;
use std::fmt;
use std::os::raw::c_int;

use forge_hip_sys as sys;

#[derive(Debug, Clone)]
pub enum ForgeError {
    /// Kernel compilation failed (unused: the kernels are compiled ahead of time for gfx950).
    CompilationFailed(String),
    /// The code object could not be loaded onto the device.
    ModuleLoadFailed(String),
    /// A kernel was not found in the code object.
    FunctionLoadFailed(String),
    /// A call was rejected (bad argument, n > max_n, ...) or a launch failed.
    LaunchFailed(String),
    /// Waiting on the stream failed, or the device reported an error (e.g. a sort look-back
    /// that gave up).
    SyncFailed(String),
    /// A buffer is not on the context's device.
    WrongDevice(String),
    /// No HIP device, or not a gfx950 one.
    DeviceNotFound(String),
}

impl fmt::Display for ForgeError {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        match self {
            ForgeError::CompilationFailed(m) => write!(f, "compilation failed: {}", m),
            ForgeError::ModuleLoadFailed(m) => write!(f, "module load failed: {}", m),
            ForgeError::FunctionLoadFailed(m) => write!(f, "function load failed: {}", m),
            ForgeError::LaunchFailed(m) => write!(f, "kernel launch failed: {}", m),
            ForgeError::SyncFailed(m) => write!(f, "sync failed: {}", m),
            ForgeError::WrongDevice(m) => write!(f, "wrong device: {}", m),
            ForgeError::DeviceNotFound(m) => write!(f, "device not found: {}", m),
        }
    }
}

impl std::error::Error for ForgeError {}

/// The calling thread's last message from the library.
pub(crate) fn last_error() -> String {
    // fh_last_error never returns NULL
    unsafe { CStr::from_ptr(sys::fh_last_error()) }.to_string_lossy().into_owned()
}

/// Return code of a queued call -> Result.
pub(crate) fn check(rc: c_int) -> Result<(), ForgeError> {
    match rc {
        sys::FH_OK => Ok(()),
        sys::FH_ENODEV => Err(ForgeError::DeviceNotFound(last_error())),
        _ => Err(ForgeError::LaunchFailed(format!("[{}] {}", rc, last_error()))),
    }
}

/// Return code of fh_sync -> Result.
pub(crate) fn check_sync(rc: c_int) -> Result<(), ForgeError> {
    match rc {
        sys::FH_OK => Ok(()),
        _ => Err(ForgeError::SyncFailed(format!("[{}] {}", rc, last_error()))),
    }
}

/// Return code of a HIP runtime call -> Result.
pub(crate) fn check_hip(rc: c_int, what: &str) -> Result<(), ForgeError> {
    if rc == 0 {
        Ok(())
    } else {
        Err(ForgeError::LaunchFailed(format!("{}: hipError_t {}", what, rc)))
    }
}
