"""Context, stream and device-buffer plumbing over the C ABI.

Device buffers are torch tensors on the HIP device (torch is used for allocation and copies
only); u32 buffers are stored as torch.int32 and reinterpreted as unsigned on the host.
Mirrors the runtime pieces the reference path uses: the simulation stream
(forge-runtime/src/cuda.rs:55-63) and synchronous Array<T> transfers (array.rs:193-214,366-406).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import check

U32 = torch.int32  # storage dtype of u32 device buffers


def ptr(t, dtype=None, what: str = "tensor") -> ctypes.c_void_p | None:
    """Device pointer of a contiguous HIP tensor (None passes through as NULL)."""
    if t is None:
        return None
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{what}: expected a torch tensor, got {type(t).__name__}")
    if not t.is_cuda:
        raise ValueError(f"{what}: tensor must live on the HIP device")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{what}: expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def to_u32(t: torch.Tensor) -> np.ndarray:
    """Copy a u32 device buffer to host as numpy uint32 (synchronous, like Array::to_vec)."""
    return t.detach().cpu().numpy().view(np.uint32)


def from_u32(a, device="cuda") -> torch.Tensor:
    a = np.ascontiguousarray(np.asarray(a, dtype=np.uint32))
    return torch.from_numpy(a.view(np.int32).copy()).to(device)


def u32_empty(n: int, device="cuda") -> torch.Tensor:
    return torch.empty(max(int(n), 0), dtype=U32, device=device)


class Context:
    """Owns an fh_ctx: the stream, all scratch (sized for max_n particles and max_cells cells)
    and the captured graph.  One host thread at a time."""

    def __init__(self, max_n: int, max_cells: int, device: int = 0):
        lib = _lib.load()
        h = ctypes.c_void_p()
        check(lib.fh_create(int(device), int(max_n), int(max_cells), None, ctypes.byref(h)))
        self._h = h
        self.max_n = int(max_n)
        self.max_cells = int(max_cells)
        self.device = int(device)

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise RuntimeError("context is closed")
        return self._h

    @property
    def stream_ptr(self) -> int:
        return int(_lib.load().fh_stream(self.handle) or 0)

    def torch_stream(self) -> torch.cuda.ExternalStream:
        return torch.cuda.ExternalStream(self.stream_ptr, device=f"cuda:{self.device}")

    @property
    def scratch_bytes(self) -> int:
        return int(_lib.load().fh_scratch_bytes(self.handle))

    def sync(self) -> None:
        check(_lib.load().fh_sync(self.handle))

    def graph_begin(self) -> None:
        check(_lib.load().fh_graph_begin(self.handle))

    def graph_end(self) -> None:
        check(_lib.load().fh_graph_end(self.handle))

    def graph_launch(self, count: int = 1) -> None:
        check(_lib.load().fh_graph_launch(self.handle, int(count)))

    def event_record(self, slot: int) -> None:
        check(_lib.load().fh_event_record(self.handle, int(slot)))

    def event_elapsed_ms(self, a: int, b: int) -> float:
        ms = ctypes.c_float()
        check(_lib.load().fh_event_elapsed_ms(self.handle, int(a), int(b), ctypes.byref(ms)))
        return float(ms.value)

    def sort_plan(self) -> int:
        """Bit p set: digit pass p of the last sort moved data (fh_sort_plan; synchronises)."""
        v = ctypes.c_uint32()
        check(_lib.load().fh_sort_plan(self.handle, ctypes.byref(v)))
        return int(v.value)

    def set_option(self, option: int, value: int) -> None:
        """fh_set_option, e.g. set_option(FH_OPT_SPH_EXACT, 1) for the bit-exact SPH passes."""
        check(_lib.load().fh_set_option(self.handle, int(option), int(value)))

    def time_kernel(self, name: str, max_launches: int) -> None:
        """Bracket the next `max_launches` launches of kernel `name` with HIP events (captured
        launches re-record them on every graph replay)."""
        check(_lib.load().fh_time_kernel(self.handle, name.encode(), int(max_launches)))

    def kernel_times_ms(self, name: str, cap: int = 4096) -> list:
        buf = (ctypes.c_float * cap)()
        cnt = ctypes.c_uint32()
        check(_lib.load().fh_kernel_times(self.handle, name.encode(), buf, cap, ctypes.byref(cnt)))
        return [float(buf[q]) for q in range(cnt.value)]

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            _lib.load().fh_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_default: dict = {}


def default_context(max_n: int, max_cells: int, device: int = 0) -> Context:
    """A process-wide context per device that grows on demand (outside graph capture), like the
    reference's one global simulation stream per ordinal (cuda.rs:13,55-63)."""
    ctx = _default.get(device)
    if ctx is None or ctx.max_n < max_n or ctx.max_cells < max_cells:
        if ctx is not None:
            ctx.sync()
            ctx.close()
        old_n = ctx.max_n if ctx is not None else 0
        old_c = ctx.max_cells if ctx is not None else 0
        ctx = Context(max(max_n, old_n, 1), max(max_cells, old_c, 1), device)
        _default[device] = ctx
    return ctx
