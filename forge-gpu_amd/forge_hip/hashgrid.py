"""HashGrid and RadixSorter: host-side mirror of forge-runtime/src/hashgrid.rs and
forge-runtime/src/radix_sort.rs over the C ABI.

Same names, argument meaning and outputs as the reference:
  HashGrid(cell_size, grid_dims, origin, max_particles)      hashgrid.rs:50-72
  HashGrid.num_cells()                                        hashgrid.rs:75-77
  HashGrid.build(positions)                                   hashgrid.rs:82-125 (on the GPU here)
  HashGrid.position_to_cell(pos)                              hashgrid.rs:128-139
  HashGrid.query_neighbors(pos, radius, positions)            hashgrid.rs:145-193
  RadixSorter(max_n).sort(keys, values, n, num_bits)          radix_sort.rs:55-220
  find_cell_boundaries(sorted, start, end, n, num_cells)      radix_sort.rs:229-317
  cell_start_csr(sorted, n, num_cells)                        hashgrid.rs:102-106 (CSR from
                                                              already-sorted keys)
Differences: errors raise ForgeError instead of panicking (n > max_n, bad num_bits), and
num_bits may be any of 1..32 (the reference required a multiple of 4).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import check, f3, u3
from .runtime import Context, U32, default_context, ptr, to_u32, u32_empty


def _xyz(positions):
    """(x, y, z, stride, n) device views of positions given as an (N, 3) float32 tensor
    (Vec3f array-of-structures, 12 bytes per particle) or a tuple of three (N,) tensors."""
    if isinstance(positions, (tuple, list)):
        x, y, z = positions
        for t, nm in ((x, "x"), (y, "y"), (z, "z")):
            ptr(t, torch.float32, nm)
        n = x.numel()
        if y.numel() != n or z.numel() != n:
            raise ValueError("x, y, z lengths differ")
        return x, y, z, 1, n
    p = positions
    if p.dim() != 2 or p.shape[1] != 3:
        raise ValueError("positions must be (N, 3)")
    ptr(p, torch.float32, "positions")
    return p[:, 0], p[:, 1], p[:, 2], 3, p.shape[0]


def _fptr(t) -> ctypes.c_void_p:
    """Pointer to the first element of a possibly strided float view."""
    return ctypes.c_void_p(t.data_ptr())


def _pre(ctx: Context) -> None:
    """Order the context stream after the work torch has queued on its current stream."""
    if not getattr(ctx, "capturing", False):
        ctx.torch_stream().wait_stream(torch.cuda.current_stream())


class HashGrid:
    def __init__(self, cell_size: float, grid_dims, origin=(0.0, 0.0, 0.0),
                 max_particles: int = 0, device: int = 0, ctx: Context | None = None):
        self.cell_size = float(np.float32(cell_size))
        self.dim_x, self.dim_y, self.dim_z = (int(d) for d in grid_dims)
        self.origin = tuple(float(np.float32(o)) for o in origin)
        self.num_particles = 0
        C = self.num_cells()
        self.ctx = ctx or default_context(max(int(max_particles), 1), C, device)
        dev = f"cuda:{self.ctx.device}"
        self.cell_start = torch.zeros(C + 1, dtype=U32, device=dev)
        self.sorted_indices = torch.zeros(max(int(max_particles), 0), dtype=U32, device=dev)
        self.cell_indices = torch.zeros(max(int(max_particles), 0), dtype=U32, device=dev)
        self._positions = None

    def num_cells(self) -> int:
        return self.dim_x * self.dim_y * self.dim_z

    @property
    def dims(self):
        return (self.dim_x, self.dim_y, self.dim_z)

    def build(self, positions) -> None:
        x, y, z, stride, n = _xyz(positions)
        if n > self.sorted_indices.numel():
            self.sorted_indices = u32_empty(n, x.device)
            self.cell_indices = u32_empty(n, x.device)
        _pre(self.ctx)
        check(_lib.load().fh_hashgrid_build(
            self.ctx.handle, _fptr(x), _fptr(y), _fptr(z), stride, n, self.cell_size,
            f3(self.origin), u3(self.dims), ptr(self.cell_start), ptr(self.sorted_indices),
            ptr(self.cell_indices)))
        self.ctx.sync()
        self.num_particles = n
        self._positions = positions

    def position_to_cell(self, pos) -> int:
        p = torch.tensor([list(map(float, pos))], dtype=torch.float32,
                         device=self.cell_start.device)
        keys = u32_empty(1, p.device)
        _pre(self.ctx)
        check(_lib.load().fh_hash_cells(self.ctx.handle, _fptr(p[:, 0]), _fptr(p[:, 1]),
                                        _fptr(p[:, 2]), 3, 1, self.cell_size, f3(self.origin),
                                        u3(self.dims), ptr(keys), None))
        self.ctx.sync()
        return int(to_u32(keys)[0])

    def query_neighbors_batch(self, queries, radius: float, positions):
        """All neighbours of every query point: (counts, offsets, indices) u32 device tensors."""
        x, y, z, stride, _ = _xyz(positions)
        qx, qy, qz, qstride, nq = _xyz(queries)
        lib = _lib.load()
        counts = u32_empty(nq, x.device)
        args = (self.ctx.handle, _fptr(x), _fptr(y), _fptr(z), stride, self.cell_size,
                f3(self.origin), u3(self.dims), ptr(self.cell_start), ptr(self.sorted_indices),
                _fptr(qx), _fptr(qy), _fptr(qz), qstride, nq, float(radius))
        _pre(self.ctx)
        check(lib.fh_query_neighbors(*args, ptr(counts), None, None))
        self.ctx.sync()
        offsets = torch.zeros(nq + 1, dtype=torch.int64, device=x.device)
        offsets[1:] = torch.cumsum(counts.to(torch.int64), 0)
        total = int(offsets[-1].item())
        offsets32 = offsets.to(U32)
        indices = u32_empty(max(total, 1), x.device)
        _pre(self.ctx)
        check(lib.fh_query_neighbors(*args, ptr(counts), ptr(offsets32), ptr(indices)))
        self.ctx.sync()
        return counts, offsets32, indices[:total]

    def query_neighbors(self, pos, radius: float, positions) -> list:
        q = torch.tensor([list(map(float, pos))], dtype=torch.float32,
                         device=self.cell_start.device)
        _, _, idx = self.query_neighbors_batch(q, radius, positions)
        return [int(v) for v in to_u32(idx)]

    def neighbor_counts(self, radius: float, positions, with_weights: bool = True):
        """Every point of the grid as a query of its own grid: (counts u32, poly6 weight sums)."""
        x, y, z, stride, n = _xyz(positions)
        counts = u32_empty(n, x.device)
        wsum = torch.empty(n, dtype=torch.float32, device=x.device) if with_weights else None
        _pre(self.ctx)
        check(_lib.load().fh_neighbor_query(
            self.ctx.handle, _fptr(x), _fptr(y), _fptr(z), stride, n, self.cell_size,
            f3(self.origin), u3(self.dims), ptr(self.cell_start), ptr(self.sorted_indices),
            float(radius), ptr(counts), ptr(wsum)))
        self.ctx.sync()
        return counts, wsum


class RadixSorter:
    # Keys of 17..20 bits below this many pairs are sorted in two 10-bit passes, all others in
    # 8-bit passes (the library's digits_for).
    WIDE_BELOW_N = 1 << 23

    @staticmethod
    def digit_layout(num_bits: int, n: int) -> tuple[int, int]:
        """(digit bits, passes) of a num_bits sort of n pairs."""
        db = 10 if 16 < num_bits <= 20 and n < RadixSorter.WIDE_BELOW_N else 8
        return db, (num_bits + db - 1) // db

    def __init__(self, max_n: int, device: int = 0, ctx: Context | None = None):
        self.max_n = int(max_n)
        self.ctx = ctx or default_context(self.max_n, 1, device)

    def sort(self, keys: torch.Tensor, values: torch.Tensor, n: int, num_bits: int,
             sync: bool = True) -> None:
        if n > self.max_n:
            raise _lib.ForgeError(_lib.FH_ERANGE, f"n={n} exceeds max_n={self.max_n}")
        _pre(self.ctx)
        check(_lib.load().fh_sort_pairs(self.ctx.handle, ptr(keys, U32, "keys"),
                                        ptr(values, U32, "values"), int(n), int(num_bits)))
        if sync:
            self.ctx.sync()


def find_cell_boundaries(sorted_cell_ids: torch.Tensor, cell_start: torch.Tensor,
                         cell_end: torch.Tensor, n: int, num_cells: int,
                         ctx: Context | None = None) -> None:
    ctx = ctx or default_context(max(int(n), 1), int(num_cells))
    _pre(ctx)
    check(_lib.load().fh_find_cell_boundaries(ctx.handle, ptr(sorted_cell_ids, U32),
                                              int(n), int(num_cells), ptr(cell_start, U32),
                                              ptr(cell_end, U32)))
    ctx.sync()


def cell_start_csr(sorted_cell_ids: torch.Tensor, n: int, num_cells: int,
                   cell_start: torch.Tensor | None = None, ctx: Context | None = None):
    """CSR cell_start[0..num_cells] of keys sorted ascending: cell_start[c] = number of keys < c
    (the prefix sum of per-cell counts of hashgrid.rs:102-106).  Returns cell_start."""
    ctx = ctx or default_context(max(int(n), 1), int(num_cells))
    if cell_start is None:
        cell_start = u32_empty(int(num_cells) + 1, sorted_cell_ids.device)
    _pre(ctx)
    check(_lib.load().fh_cell_start_csr(ctx.handle, ptr(sorted_cell_ids, U32), int(n),
                                        int(num_cells), ptr(cell_start, U32)))
    ctx.sync()
    return cell_start
