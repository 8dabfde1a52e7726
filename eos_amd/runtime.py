"""Runtime handle and device buffers over libeoship (one device, one stream).

The Python counterpart of the reference's device runtime
(runtime/backends/cuda/native_linux.go:150-283): a Runtime owns the HIP stream
that every call of this package is ordered on.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib


class DeviceBuffer:
    """Device allocation owned through a Runtime."""

    def __init__(self, rt: "Runtime", nbytes: int):
        self.rt = rt
        self.nbytes = int(nbytes)
        self.ptr = C.c_void_p()
        _lib.call("eoship_malloc", rt.handle, C.c_size_t(self.nbytes), C.byref(self.ptr))

    @classmethod
    def from_array(cls, rt: "Runtime", arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(rt, arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes > self.nbytes:
            raise ValueError("array larger than device buffer")
        _lib.call("eoship_h2d", self.rt.handle, self.ptr, arr.ctypes.data_as(C.c_void_p),
                  C.c_size_t(arr.nbytes))

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ValueError("requested more bytes than the buffer holds")
        _lib.call("eoship_d2h", self.rt.handle, out.ctypes.data_as(C.c_void_p), self.ptr,
                  C.c_size_t(out.nbytes))
        return out

    def view(self, offset: int, nbytes: int) -> "DeviceBuffer":
        """A non-owning window [offset, offset + nbytes) of this allocation."""
        if offset < 0 or nbytes < 0 or offset + nbytes > self.nbytes:
            raise ValueError("view outside the buffer")
        v = DeviceBuffer.__new__(DeviceBuffer)
        v.rt, v.nbytes, v._owner = self.rt, int(nbytes), self
        v.ptr = C.c_void_p(self.ptr.value + int(offset))
        return v

    def free(self) -> None:
        if getattr(self, "_owner", None) is not None:
            return  # a view owns nothing
        if self.ptr:
            _lib.call("eoship_free", self.rt.handle, self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            if self.ptr and self.rt.handle:
                self.free()
        except Exception:
            pass


class Runtime:
    """One gfx950 device and its stream."""

    def __init__(self, device: int = 0):
        self.handle = C.c_void_p()
        _lib.call("eoship_runtime_create", int(device), C.byref(self.handle))

    def close(self) -> None:
        if self.handle:
            _lib.call("eoship_runtime_destroy", self.handle)
            self.handle = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self) -> dict:
        name = C.create_string_buffer(256)
        arch = C.create_string_buffer(64)
        cus = C.c_int()
        _lib.call("eoship_device_info", self.handle, name, C.c_size_t(256), C.byref(cus), arch,
                  C.c_size_t(64))
        return {"name": name.value.decode(), "arch": arch.value.decode(), "compute_units": cus.value}

    def wait_for(self, other: "Runtime") -> None:
        """Work enqueued here after this call starts after everything enqueued
        on ``other`` so far (no host wait)."""
        _lib.call("eoship_runtime_wait", self.handle, other.handle)

    def sync(self) -> None:
        _lib.call("eoship_sync", self.handle)

    def profile(self, enabled: bool) -> None:
        _lib.call("eoship_profile_enable", self.handle, int(bool(enabled)))

    def profile_select(self, prefix: str | None) -> None:
        """Record only launches whose label starts with ``prefix`` (None = all)."""
        _lib.call("eoship_profile_select", self.handle, prefix.encode() if prefix else None)

    def profile_reset(self) -> None:
        _lib.call("eoship_profile_reset", self.handle)

    def profile_read(self, prefix: str) -> tuple[int, float]:
        n = C.c_int64()
        ms = C.c_double()
        _lib.call("eoship_profile_read", self.handle, prefix.encode(), C.byref(n), C.byref(ms))
        return n.value, ms.value

    def accounting(self, reset: bool = False) -> dict:
        """Execution accounting since creation or the last reset (the keys of
        the reference's StepDispatchResult.Metadata / ExecutionAccounting)."""
        a = _lib.EosHipAccounting()
        _lib.call("eoship_accounting_read", self.handle, C.byref(a), C.c_int32(int(reset)))
        return {"device_execution": bool(a.device_execution), "execution_mode": "hip_device",
                "kernel_launches": a.kernel_launches, "uploaded_bytes": a.uploaded_bytes,
                "downloaded_bytes": a.downloaded_bytes, "sync_count": a.sync_count,
                "graph_captures": a.graph_captures, "graph_replays": a.graph_replays}

    def profile_samples(self, prefix: str) -> np.ndarray:
        """Per-launch durations (ms) of the recorded launches matching prefix."""
        n = C.c_int64()
        _lib.call("eoship_profile_samples", self.handle, prefix.encode(), None, C.c_int64(0),
                  C.byref(n))
        out = np.zeros(max(n.value, 1), np.float32)
        _lib.call("eoship_profile_samples", self.handle, prefix.encode(),
                  out.ctypes.data_as(C.c_void_p), C.c_int64(n.value), C.byref(n))
        return out[:n.value]

    def mark(self, slot: int) -> None:
        _lib.call("eoship_timer_mark", self.handle, int(slot))

    def elapsed_ms(self, begin: int, end: int) -> float:
        ms = C.c_double()
        _lib.call("eoship_timer_elapsed", self.handle, int(begin), int(end), C.byref(ms))
        return ms.value
