"""ctypes front end of oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

The CPU restatement of the reference path is the checker of the HIP product.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.  Each function
takes and returns numpy arrays; see oracle.h for the reference file:line each one restates.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "liboracle.so"

_P = ctypes.c_void_p
_U = ctypes.c_uint32
_F = ctypes.c_float


class SphParams(ctypes.Structure):
    _fields_ = [("h", _F), ("cell_size", _F), ("dims", _U * 3), ("mass", _F),
                ("gas_constant", _F), ("rest_density", _F), ("visc", _F)]


_SIG = {
    "or_f32_as_i32": (ctypes.c_int32, [_F]),
    "or_position_to_cell": (_U, [_F, _F, _F, _F, _P, _P]),
    "or_hash_cells": (None, [_P, _P, _P, _U, _U, _F, _P, _P, _P, _P]),
    "or_stable_sort_pairs": (ctypes.c_int, [_P, _P, _U, _U]),
    "or_find_cell_boundaries": (None, [_P, _U, _U, _P, _P]),
    "or_cell_start_csr": (None, [_P, _U, _U, _P]),
    "or_hashgrid_build": (ctypes.c_int, [_P, _P, _P, _U, _U, _F, _P, _P, _P, _P, _P]),
    "or_query_neighbors": (_U, [_F, _F, _F, _F, _P, _P, _P, _U, _F, _P, _P, _P, _P, _P, _U]),
    "or_neighbor_counts": (None, [_P, _P, _P, _U, _U, _F, _P, _P, _P, _P, _F, _P, _P]),
    "or_sph_density": (None, [ctypes.POINTER(SphParams), _P, _P, _P, _U, _P, _P, _P]),
    "or_sph_density_at": (None, [ctypes.POINTER(SphParams), _P, _P, _P, _P, _P, _P, _U, _P]),
    "or_sph_force_f64_at": (None, [ctypes.POINTER(SphParams), _P, _P, _P, _P, _P, _P, _P, _P,
                                   _P, _P, _U, _P, _P, _P]),
    "or_sph_force": (None, [ctypes.POINTER(SphParams), _P, _P, _P, _P, _P, _P, _P, _U, _P, _P,
                            _F, _P, _P]),
    "or_sph_force_f64": (None, [ctypes.POINTER(SphParams), _P, _P, _P, _P, _P, _P, _P, _U, _P,
                                _P, _P, _P, _P]),
    "or_sph_pressure": (None, [ctypes.POINTER(SphParams), _P, _P, _P, _P, _P, _P, _P, _U, _P,
                               _P, _F, _P]),
    "or_sph_viscosity": (None, [ctypes.POINTER(SphParams), _P, _P, _P, _P, _P, _P, _P, _U, _P,
                                _P, _F, _P]),
    "or_gravity": (None, [_P, _P, _P, _U, _F, _F, _F, _F]),
    "or_integrate": (None, [_P, _P, _P, _P, _P, _P, _U, _F]),
    "or_box_collider": (None, [_P, _P, _P, _P, _P, _P, _U, _P, _P, _F]),
    "or_sph_step": (ctypes.c_int, [ctypes.POINTER(SphParams), _U, _P, _P, _P, _F, _P, _P, _P,
                                   _P, _P, _P, _U, _F, _P, _P]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(str(LIB_PATH))
        for k, (r, a) in _SIG.items():
            f = getattr(L, k)
            f.restype = r
            f.argtypes = a
        _lib = L
    return _lib


def _p(a):
    """Data pointer of a numpy array.  The caller must keep `a` referenced for the whole call:
    never pass a temporary (its buffer may be freed before the C function runs)."""
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def _vec3(v, dt=np.float32):
    return np.ascontiguousarray(np.asarray(v, dtype=dt).reshape(3))


def f32_as_i32(f: float) -> int:
    return int(lib().or_f32_as_i32(float(f)))


def position_to_cell(p, cell_size, origin, dims) -> int:
    o, d = _vec3(origin), _vec3(dims, np.uint32)
    return int(lib().or_position_to_cell(float(p[0]), float(p[1]), float(p[2]), float(cell_size),
                                         _p(o), _p(d)))


def hash_cells(x, y, z, cell_size, origin, dims):
    x, y, z = _f32(x), _f32(y), _f32(z)
    n = x.size
    keys = np.empty(n, np.uint32)
    vals = np.empty(n, np.uint32)
    o, d = _vec3(origin), _vec3(dims, np.uint32)
    lib().or_hash_cells(_p(x), _p(y), _p(z), 1, n, float(cell_size), _p(o), _p(d), _p(keys), _p(vals))
    return keys, vals


def stable_sort_pairs(keys, vals, num_bits=32):
    k, v = _u32(keys).copy(), _u32(vals).copy()
    if lib().or_stable_sort_pairs(_p(k), _p(v), k.size, int(num_bits)) != 0:
        raise ValueError("or_stable_sort_pairs failed")
    return k, v


def find_cell_boundaries(sorted_keys, num_cells):
    k = _u32(sorted_keys)
    s = np.empty(num_cells, np.uint32)
    e = np.empty(num_cells, np.uint32)
    lib().or_find_cell_boundaries(_p(k), k.size, int(num_cells), _p(s), _p(e))
    return s, e


def cell_start_csr(sorted_keys, num_cells):
    k = _u32(sorted_keys)
    s = np.empty(num_cells + 1, np.uint32)
    lib().or_cell_start_csr(_p(k), k.size, int(num_cells), _p(s))
    return s


def hashgrid_build(x, y, z, cell_size, origin, dims):
    x, y, z = _f32(x), _f32(y), _f32(z)
    n = x.size
    C = int(dims[0]) * int(dims[1]) * int(dims[2])
    cs = np.empty(C + 1, np.uint32)
    si = np.empty(max(n, 1), np.uint32)
    ci = np.empty(max(n, 1), np.uint32)
    o, d = _vec3(origin), _vec3(dims, np.uint32)
    if lib().or_hashgrid_build(_p(x), _p(y), _p(z), 1, n, float(cell_size), _p(o), _p(d),
                               _p(cs), _p(si), _p(ci)) != 0:
        raise MemoryError("or_hashgrid_build")
    return cs, si[:n], ci[:n]


def query_neighbors(q, radius, x, y, z, cell_size, origin, dims, cell_start, sorted_indices):
    x, y, z = _f32(x), _f32(y), _f32(z)
    o, d = _vec3(origin), _vec3(dims, np.uint32)
    cs, si = _u32(cell_start), _u32(sorted_indices)
    cap = x.size
    out = np.empty(max(cap, 1), np.uint32)
    cnt = lib().or_query_neighbors(float(q[0]), float(q[1]), float(q[2]), float(radius), _p(x), _p(y),
                                   _p(z), 1, float(cell_size), _p(o), _p(d), _p(cs), _p(si), _p(out), cap)
    return out[:min(cnt, cap)].copy()


def neighbor_counts(x, y, z, cell_size, origin, dims, cell_start, sorted_indices, radius):
    x, y, z = _f32(x), _f32(y), _f32(z)
    n = x.size
    o, d = _vec3(origin), _vec3(dims, np.uint32)
    cs, si = _u32(cell_start), _u32(sorted_indices)
    cnt = np.empty(n, np.uint32)
    w = np.empty(n, np.float32)
    lib().or_neighbor_counts(_p(x), _p(y), _p(z), 1, n, float(cell_size), _p(o), _p(d), _p(cs),
                             _p(si), float(radius), _p(cnt), _p(w))
    return cnt, w


def sph_params(h, cell_size, dims, mass, gas_constant=2000.0, rest_density=1000.0, visc=0.01):
    p = SphParams()
    p.h, p.cell_size, p.mass = float(h), float(cell_size), float(mass)
    for q in range(3):
        p.dims[q] = int(dims[q])
    p.gas_constant, p.rest_density, p.visc = float(gas_constant), float(rest_density), float(visc)
    return p


def sph_density(p: SphParams, x, y, z, cell_start, sorted_indices):
    x, y, z = _f32(x), _f32(y), _f32(z)
    cs, si = _u32(cell_start), _u32(sorted_indices)
    rho = np.empty(x.size, np.float32)
    lib().or_sph_density(ctypes.byref(p), _p(x), _p(y), _p(z), x.size, _p(cs), _p(si), _p(rho))
    return rho


def sph_density_at(p: SphParams, x, y, z, cell_start, sorted_indices, which):
    """Densities of the particles `which` only (same sums as sph_density)."""
    x, y, z = _f32(x), _f32(y), _f32(z)
    cs, si, w = _u32(cell_start), _u32(sorted_indices), _u32(which)
    rho = np.empty(w.size, np.float32)
    lib().or_sph_density_at(ctypes.byref(p), _p(x), _p(y), _p(z), _p(cs), _p(si), _p(w), w.size,
                            _p(rho))
    return rho


def sph_force_f64_at(p: SphParams, x, y, z, vx, vy, vz, density, cell_start, sorted_indices,
                     which):
    """sph_force_f64 of the particles `which` only: (3, m) accelerations, error scales and
    distance-rounding sensitivities."""
    arrs = [_f32(a) for a in (x, y, z, vx, vy, vz, density)]
    cs, si, w = _u32(cell_start), _u32(sorted_indices), _u32(which)
    m = w.size
    a64 = np.empty(3 * m, np.float64)
    s64 = np.empty(3 * m, np.float64)
    e64 = np.empty(3 * m, np.float64)
    lib().or_sph_force_f64_at(ctypes.byref(p), *[_p(a) for a in arrs], _p(cs), _p(si), _p(w), m,
                              _p(a64), _p(s64), _p(e64))
    return a64.reshape(3, m), s64.reshape(3, m), e64.reshape(3, m)


def sph_force(p: SphParams, x, y, z, vx, vy, vz, density, cell_start, sorted_indices, dt):
    arrs = [_f32(a) for a in (x, y, z, vx, vy, vz, density)]
    n = arrs[0].size
    cs, si = _u32(cell_start), _u32(sorted_indices)
    vout = np.empty(3 * n, np.float32)
    acc = np.empty(3 * n, np.float32)
    lib().or_sph_force(ctypes.byref(p), *[_p(a) for a in arrs], n, _p(cs), _p(si), float(dt),
                       _p(vout), _p(acc))
    return vout.reshape(3, n), acc.reshape(3, n)


def sph_force_f64(p: SphParams, x, y, z, vx, vy, vz, density, cell_start, sorted_indices):
    arrs = [_f32(a) for a in (x, y, z, vx, vy, vz, density)]
    n = arrs[0].size
    cs, si = _u32(cell_start), _u32(sorted_indices)
    a64 = np.empty(3 * n, np.float64)
    s64 = np.empty(3 * n, np.float64)
    e64 = np.empty(3 * n, np.float64)
    lib().or_sph_force_f64(ctypes.byref(p), *[_p(a) for a in arrs], n, _p(cs), _p(si),
                           _p(a64), _p(s64), _p(e64))
    return a64.reshape(3, n), s64.reshape(3, n), e64.reshape(3, n)


def _unfused(fn, p: SphParams, x, y, z, vx, vy, vz, density, cell_start, sorted_indices, dt):
    arrs = [_f32(a) for a in (x, y, z, vx, vy, vz, density)]
    n = arrs[0].size
    cs, si = _u32(cell_start), _u32(sorted_indices)
    vout = np.empty(3 * n, np.float32)
    fn(ctypes.byref(p), *[_p(a) for a in arrs], n, _p(cs), _p(si), float(dt), _p(vout))
    return vout.reshape(3, n)


def sph_pressure(p: SphParams, x, y, z, vx, vy, vz, density, cell_start, sorted_indices, dt):
    """Unfused SphPressureModule pass; returns the new velocities (3, n)."""
    return _unfused(lib().or_sph_pressure, p, x, y, z, vx, vy, vz, density, cell_start,
                    sorted_indices, dt)


def sph_viscosity(p: SphParams, x, y, z, vx, vy, vz, density, cell_start, sorted_indices, dt):
    """Unfused SphViscosityModule pass; returns the new velocities (3, n)."""
    return _unfused(lib().or_sph_viscosity, p, x, y, z, vx, vy, vz, density, cell_start,
                    sorted_indices, dt)


def gravity(vx, vy, vz, g, dt):
    v = [_f32(a).copy() for a in (vx, vy, vz)]
    lib().or_gravity(*[_p(a) for a in v], v[0].size, float(g[0]), float(g[1]), float(g[2]), float(dt))
    return v


def integrate(x, y, z, vx, vy, vz, dt):
    s = [_f32(a).copy() for a in (x, y, z, vx, vy, vz)]
    lib().or_integrate(*[_p(a) for a in s], s[0].size, float(dt))
    return s


def box_collider(x, y, z, vx, vy, vz, mn, mx, e):
    s = [_f32(a).copy() for a in (x, y, z, vx, vy, vz)]
    lo, hi = _vec3(mn), _vec3(mx)
    lib().or_box_collider(*[_p(a) for a in s], s[0].size, _p(lo), _p(hi), float(e))
    return s


def sph_step(p: SphParams, flags, g, mn, mx, e, x, y, z, vx, vy, vz, dt):
    """One Pipeline::step; returns (x, y, z, vx, vy, vz, density, accel(3, n))."""
    s = [_f32(a).copy() for a in (x, y, z, vx, vy, vz)]
    n = s[0].size
    rho = np.empty(n, np.float32)
    acc = np.empty(3 * n, np.float32)
    gv, lo, hi = _vec3(g), _vec3(mn), _vec3(mx)
    rc = lib().or_sph_step(ctypes.byref(p), int(flags), _p(gv), _p(lo), _p(hi), float(e),
                           *[_p(a) for a in s], n, float(dt), _p(rho), _p(acc))
    if rc != 0:
        raise MemoryError("or_sph_step")
    return (*s, rho, acc.reshape(3, n))
