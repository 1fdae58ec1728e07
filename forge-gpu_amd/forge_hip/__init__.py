"""forge_hip -- MI355X (gfx950) SPH / hash-grid hot path of forge-gpu behind its own API.

The compute path is libforge_hip.so (hand-written HIP kernels behind the C ABI of
include/forge_hip.h); this package is the host-side mirror of the reference's interfaces for
the path (HashGrid, RadixSorter, find_cell_boundaries, FieldSet, SimModule, Pipeline and the
SPH / gravity / integrate / box modules).  Importing it never loads a CPU fallback: there is
none.
"""
from ._lib import (FH_EINVAL, FH_ENODEV, FH_EPI_BOX, FH_EPI_GRAVITY, FH_EPI_INTEGRATE,
                   FH_ERANGE, FH_ESTATE, FH_OK, FH_OPT_DIRECT_ITEMS, FH_OPT_EPOCH_PERIOD,
                   FH_OPT_HEAVY_PARTS, FH_OPT_HEAVY_SLOTS, FH_OPT_HEAVY_WORK, FH_OPT_SPH_EXACT,
                   FH_OPT_SUBCELL,
                   FH_OPT_SPIN_LIMIT,
                   ForgeError, LibraryNotBuilt, load)
from .hashgrid import HashGrid, RadixSorter, cell_start_csr, find_cell_boundaries
from .modules import (BoxColliderModule, FieldSet, GravityModule, IntegrateModule, Pipeline,
                      SimModule, SphDensityModule, SphFusedModule, SphPressureModule,
                      SphViscosityModule, build_pipeline, frame_bytes, init_field_arrays,
                      init_fields, pack_frame, run_streaming)
from .runtime import Context, default_context, from_u32, to_u32, u32_empty

__all__ = [
    "FH_OK", "FH_EINVAL", "FH_ERANGE", "FH_ESTATE", "FH_ENODEV", "FH_EPI_GRAVITY",
    "FH_EPI_INTEGRATE", "FH_EPI_BOX", "FH_OPT_SPH_EXACT", "FH_OPT_HEAVY_WORK",
    "FH_OPT_DIRECT_ITEMS", "FH_OPT_HEAVY_PARTS", "FH_OPT_EPOCH_PERIOD", "FH_OPT_SPIN_LIMIT",
    "FH_OPT_HEAVY_SLOTS", "FH_OPT_SUBCELL",
    "ForgeError", "LibraryNotBuilt", "load", "HashGrid",
    "RadixSorter", "find_cell_boundaries", "cell_start_csr", "FieldSet", "SimModule", "Pipeline",
    "SphDensityModule", "SphFusedModule", "SphPressureModule", "SphViscosityModule",
    "GravityModule", "IntegrateModule",
    "BoxColliderModule", "build_pipeline", "init_fields", "init_field_arrays", "pack_frame",
    "frame_bytes", "run_streaming", "Context", "default_context", "to_u32", "from_u32",
    "u32_empty",
]
