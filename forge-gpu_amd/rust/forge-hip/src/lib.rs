//! forge-gpu's hot-path API over `libforge_hip.so` (MI355X, gfx950).
//!
//! The types keep the reference's names, fields and signatures so that forge-runtime /
//! forge-manifest code written against them keeps compiling:
//!
//! | here | reference |
//! |---|---|
//! | [`HashGrid`] | `forge-runtime/src/hashgrid.rs:21-193` |
//! | [`RadixSorter`], [`find_cell_boundaries`] | `forge-runtime/src/radix_sort.rs:26-317` |
//! | [`ForgeError`] | `forge-runtime/src/error.rs:7-22` |
//! | [`Array`], [`Device`] | `forge-runtime/src/array.rs:81-107`, `device.rs` |
//! | [`FieldSet`], [`SimModule`], [`Pipeline`] | `forge-manifest/src/modules/mod.rs:12-117` |
//! | [`SphFusedModule`] ... [`BoxColliderModule`] | `forge-manifest/src/modules/builtins/*.rs` |
//! | [`fuse_epilogue`] | the module order of `build_pipeline`, `manifest_runner.rs:322-544` |
//!
//! Every GPU call goes through the C ABI (`forge-hip-sys`); nothing here launches kernels itself.
//! A forge-runtime that keeps its own `Array<T>` implements [`DevicePtr`] for it (a raw device
//! pointer and a length) and uses the wrappers unchanged.

mod array;
mod context;
mod error;
mod hashgrid;
mod modules;
mod radix_sort;

pub use array::{Array, Device, DevicePtr, Vec3f};
pub use context::Ctx;
pub use error::ForgeError;
pub use hashgrid::HashGrid;
pub use modules::{
    fuse_epilogue, BoxColliderModule, FieldSet, GravityModule, IntegrateModule, ModuleKind,
    Pipeline, SimModule, SphDensityModule, SphFusedModule, SphPressureModule, SphViscosityModule,
};
pub use radix_sort::{find_cell_boundaries, RadixSorter};

pub use forge_hip_sys as sys;
