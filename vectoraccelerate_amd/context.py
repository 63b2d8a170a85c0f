"""GPUContext — the Python face of ``va_context`` (replaces Metal4Context / GPUContext).

Reference: ``Sources/VectorAccelerate/Core/Metal4Context.swift:183-269`` (device + queue),
``:342-410`` (executeAndWait), ``:471-488`` (getBuffer); ``VectorAccelerate.swift:254``
(``typealias GPUContext = Metal4Context``).

Device memory is held in torch CUDA tensors (plumbing only); every computation runs in
libva_hip.so.  The context owns a HIP stream; the high-level ``execute``/``compute`` tiers
order torch's stream before the call and wait for the context stream after it.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib


class VectorError(Exception):
    """Mirrors VectorCore's ``VectorError`` / the index's ``IndexError`` cases.

    ``kind`` is one of: invalidInput, dimensionMismatch, bufferAllocationFailed,
    computeFailed, unsupported.
    """

    _KINDS = {
        _lib.VA_ERR_INVALID_ARG: "invalidInput",
        _lib.VA_ERR_DIMENSION_MISMATCH: "dimensionMismatch",
        _lib.VA_ERR_OOM: "bufferAllocationFailed",
        _lib.VA_ERR_HIP: "computeFailed",
        _lib.VA_ERR_UNSUPPORTED: "unsupported",
    }

    def __init__(self, kind: str, message: str = "", status: int | None = None):
        super().__init__(f"{kind}: {message}" if message else kind)
        self.kind = kind
        self.message = message
        self.status = status

    @classmethod
    def from_status(cls, status: int, message: str) -> "VectorError":
        return cls(cls._KINDS.get(status, "computeFailed"), message, status)

    @classmethod
    def invalidInput(cls, message: str) -> "VectorError":
        return cls("invalidInput", message)

    @classmethod
    def dimensionMismatch(cls, expected: int, got: int) -> "VectorError":
        return cls("dimensionMismatch", f"expected {expected}, got {got}")


def _torch():
    import torch  # imported lazily: the CPU-only symbol tests never need it

    return torch


class GPUContext:
    """One HIP device + one stream + the library's scratch arena."""

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        h = C.c_void_p()
        st = self.lib.va_context_create(int(device), C.byref(h))
        if st != _lib.VA_OK:
            raise VectorError.from_status(st, f"va_context_create(device={device}) failed")
        self._h = h
        self.device = int(device)
        self._ext_stream = None

    # -- lifecycle -------------------------------------------------------------------
    @property
    def handle(self) -> C.c_void_p:
        if self._h is None:
            raise VectorError("computeFailed", "context destroyed")
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            self.lib.va_context_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- stream / errors ---------------------------------------------------------------
    @property
    def stream_ptr(self) -> int:
        return int(self.lib.va_context_stream(self.handle) or 0)

    def torch_stream(self):
        """The context stream as a torch ExternalStream (for events / ordering)."""
        if self._ext_stream is None:
            torch = _torch()
            self._ext_stream = torch.cuda.ExternalStream(self.stream_ptr, device=f"cuda:{self.device}")
        return self._ext_stream

    def check(self, status: int, what: str) -> None:
        if status != _lib.VA_OK:
            msg = self.lib.va_last_error_message(self.handle) or b""
            raise VectorError.from_status(status, f"{what}: {msg.decode(errors='replace')}")

    def synchronize(self) -> None:
        """executeAndWait's wait: block until the context's queued work is done."""
        self.check(self.lib.va_context_synchronize(self.handle), "va_context_synchronize")

    def order_after_torch(self) -> None:
        """Make work queued on torch's current stream visible to the context stream."""
        _torch().cuda.current_stream(self.device).synchronize()

    def set_profiling(self, enable) -> None:
        """Metal4Configuration.enableProfiling: time every scan phase with hipEvents.  True (or 1):
        every phase and the counts; 2: the scan phase alone (two events per scan, nothing else)."""
        level = 2 if (not isinstance(enable, bool) and enable == 2) else int(bool(enable))
        self.check(self.lib.va_context_set_profiling(self.handle, level), "va_context_set_profiling")

    def last_scan_timings(self) -> dict:
        """Phase timings of the last profiled scan (waits for its events)."""
        t = _lib.ScanTimings()
        self.check(self.lib.va_context_last_scan(self.handle, C.byref(t)), "va_context_last_scan")
        return t.as_dict()

    def reset_scan_totals(self) -> None:
        self.check(self.lib.va_context_reset_scan_totals(self.handle), "va_context_reset_scan_totals")

    def scan_totals(self) -> tuple[dict, int]:
        """(phase times and counts summed over the profiled scans since the reset, number of scans)."""
        t = _lib.ScanTimings()
        n = C.c_uint32(0)
        self.check(self.lib.va_context_scan_totals(self.handle, C.byref(t), C.byref(n)), "va_context_scan_totals")
        return t.as_dict(), int(n.value)

    def set_option(self, option: int, value: int) -> None:
        self.check(self.lib.va_context_set_option(self.handle, int(option), int(value)), "va_context_set_option")

    # -- buffers (getBuffer) -------------------------------------------------------------
    def buffer(self, data, dtype=None):
        """Copy host data (list / numpy) into a new device tensor (getBuffer(for:))."""
        torch = _torch()
        arr = np.ascontiguousarray(np.asarray(data, dtype=dtype))
        return torch.from_numpy(arr).to(f"cuda:{self.device}")

    def empty(self, shape, dtype):
        torch = _torch()
        return torch.empty(shape, dtype=dtype, device=f"cuda:{self.device}")


# The reference's names for the same type.
Metal4Context = GPUContext


class DeviceRows:
    """A row-major fp32 [rows x dim] array in device memory the library owns (an index's
    storage), accepted wherever this package's bindings take a contiguous device tensor."""

    is_cuda = True

    def __init__(self, ptr: int, rows: int, dim: int):
        self.ptr = int(ptr)
        self.shape = (int(rows), int(dim))

    def is_contiguous(self) -> bool:
        return True

    def contiguous(self) -> "DeviceRows":
        return self

    def data_ptr(self) -> int:
        return self.ptr

    def rows(self, start: int, stop: int) -> "DeviceRows":
        """Rows [start, stop) as a view."""
        n, d = self.shape
        start, stop = max(0, start), min(n, stop)
        return DeviceRows(self.ptr + start * d * 4, max(0, stop - start), d)


def dptr(t) -> int:
    """Device pointer of a contiguous CUDA tensor (0 for None)."""
    if t is None:
        return 0
    if not t.is_cuda:
        raise VectorError.invalidInput("expected a device (CUDA) tensor")
    if not t.is_contiguous():
        raise VectorError.invalidInput("expected a contiguous tensor")
    return int(t.data_ptr())
