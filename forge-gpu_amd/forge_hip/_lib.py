"""ctypes binding of libforge_hip.so (the C ABI declared in include/forge_hip.h).

The library is the product: there is no CPU fallback.  If the shared library is missing the
import of the compute API fails loudly (``LibraryNotBuilt``); if no gfx950 device is present,
context creation fails with ``ForgeError(FH_ENODEV)``.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent          # forge-gpu_amd/
LIB_PATH = PKG_ROOT / "lib" / "libforge_hip.so"
HEADER_PATH = PKG_ROOT.parent / "include" / "forge_hip.h"

FH_OK = 0
FH_EINVAL = -1
FH_ERANGE = -2
FH_ESTATE = -3
FH_ENODEV = -4

FH_EPI_GRAVITY = 1
FH_EPI_INTEGRATE = 2
FH_EPI_BOX = 4

FH_OPT_SPH_EXACT = 1
FH_OPT_HEAVY_WORK = 2
FH_OPT_DIRECT_ITEMS = 3
FH_OPT_HEAVY_PARTS = 4
FH_OPT_EPOCH_PERIOD = 5
FH_OPT_SPIN_LIMIT = 6
FH_OPT_HEAVY_SLOTS = 7
FH_OPT_SUBCELL = 8


class LibraryNotBuilt(RuntimeError):
    """libforge_hip.so has not been built (run ``python -c 'import __graft_entry__ as g; g.build()'``)."""


class ForgeError(RuntimeError):
    """A nonzero status from the C ABI.

    Mirrors forge-runtime/src/error.rs:7-22 (ForgeError): the reference's variants are
    launch/sync failures of the CUDA driver; here ``code`` is the C ABI status (negative:
    argument error detected on the host, positive: the hipError_t)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class FhSphParams(ctypes.Structure):
    _fields_ = [
        ("smoothing_radius", ctypes.c_float),
        ("cell_size", ctypes.c_float),
        ("grid_dims", ctypes.c_uint32 * 3),
        ("particle_mass", ctypes.c_float),
        ("gas_constant", ctypes.c_float),
        ("rest_density", ctypes.c_float),
        ("viscosity_coefficient", ctypes.c_float),
    ]


class FhEpilogue(ctypes.Structure):
    _fields_ = [
        ("flags", ctypes.c_uint32),
        ("gravity", ctypes.c_float * 3),
        ("box_min", ctypes.c_float * 3),
        ("box_max", ctypes.c_float * 3),
        ("restitution", ctypes.c_float),
    ]


_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_F32 = ctypes.c_float
_I = ctypes.c_int
_F3 = ctypes.POINTER(ctypes.c_float)
_U3 = ctypes.POINTER(ctypes.c_uint32)

# name -> (restype, argtypes); every symbol declared in include/forge_hip.h.
SIGNATURES = {
    "fh_abi_version": (_I, []),
    "fh_last_error": (ctypes.c_char_p, []),
    "fh_create": (_I, [_I, _U32, _U32, _P, ctypes.POINTER(_P)]),
    "fh_destroy": (_I, [_P]),
    "fh_stream": (_P, [_P]),
    "fh_sync": (_I, [_P]),
    "fh_scratch_bytes": (ctypes.c_size_t, [_P]),
    "fh_hash_cells": (_I, [_P, _P, _P, _P, _U32, _U32, _F32, _F3, _U3, _P, _P]),
    "fh_sort_pairs": (_I, [_P, _P, _P, _U32, _U32]),
    "fh_sort_plan": (_I, [_P, ctypes.POINTER(_U32)]),
    "fh_sort_pairs_noalloc": (_I, [_P, _P, _P, _U32, _U32]),
    "fh_noalloc_status": (_I, [_P]),
    "fh_find_cell_boundaries": (_I, [_P, _P, _U32, _U32, _P, _P]),
    "fh_cell_start_csr": (_I, [_P, _P, _U32, _U32, _P]),
    "fh_hashgrid_build": (_I, [_P, _P, _P, _P, _U32, _U32, _F32, _F3, _U3, _P, _P, _P]),
    "fh_neighbor_query": (_I, [_P, _P, _P, _P, _U32, _U32, _F32, _F3, _U3, _P, _P, _F32, _P, _P]),
    "fh_query_neighbors": (_I, [_P, _P, _P, _P, _U32, _F32, _F3, _U3, _P, _P,
                                _P, _P, _P, _U32, _U32, _F32, _P, _P, _P]),
    "fh_sph_density": (_I, [_P, ctypes.POINTER(FhSphParams), _P, _P, _P, _U32, _P, _P, _P]),
    "fh_sph_pressure": (_I, [_P, ctypes.POINTER(FhSphParams), _P, _P, _P, _P, _P, _P, _P, _P,
                             _P, _U32, _F32]),
    "fh_sph_viscosity": (_I, [_P, ctypes.POINTER(FhSphParams), _P, _P, _P, _P, _P, _P, _P, _P,
                              _P, _U32, _F32]),
    "fh_sph_force": (_I, [_P, ctypes.POINTER(FhSphParams), _P, _P, _P, _P, _P, _P, _P, _P,
                          _P, _P, _U32, _F32]),
    "fh_sph_fused": (_I, [_P, ctypes.POINTER(FhSphParams), ctypes.POINTER(FhEpilogue),
                          _P, _P, _P, _P, _P, _P, _P, _P, _U32, _F32]),
    "fh_sph_fused_steps": (_I, [_P, ctypes.POINTER(FhSphParams), ctypes.POINTER(FhEpilogue),
                                _P, _P, _P, _P, _P, _P, _P, _P, _U32, _F32, _U32]),
    "fh_set_option": (_I, [_P, _I, _I]),
    "fh_gravity": (_I, [_P, _P, _P, _P, _U32, _F32, _F32, _F32, _F32]),
    "fh_integrate": (_I, [_P, _P, _P, _P, _P, _P, _P, _U32, _F32]),
    "fh_box_collider": (_I, [_P, _P, _P, _P, _P, _P, _P, _U32, _F3, _F3, _F32]),
    "fh_pack_frame": (_I, [_P, _P, _P, _P, _U32, _U32, _P, _P]),
    "fh_graph_begin": (_I, [_P]),
    "fh_graph_end": (_I, [_P]),
    "fh_graph_launch": (_I, [_P, _U32]),
    "fh_event_record": (_I, [_P, _U32]),
    "fh_event_elapsed_ms": (_I, [_P, _U32, _U32, ctypes.POINTER(ctypes.c_float)]),
    "fh_time_kernel": (_I, [_P, ctypes.c_char_p, _U32]),
    "fh_kernel_times": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float), _U32,
                             ctypes.POINTER(ctypes.c_uint32)]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libforge_hip.so from the package tree (never from a system path)."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("FORGE_HIP_LIB", LIB_PATH))
    if not path.exists():
        raise LibraryNotBuilt(f"{path} not found; build it first (__graft_entry__.build())")
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != FH_OK:
        msg = load().fh_last_error().decode("utf-8", "replace")
        raise ForgeError(rc, msg)


def f3(v) -> ctypes.Array:
    return (ctypes.c_float * 3)(*[float(x) for x in v])


def u3(v) -> ctypes.Array:
    return (ctypes.c_uint32 * 3)(*[int(x) for x in v])
