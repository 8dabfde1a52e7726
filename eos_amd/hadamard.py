"""Host side of the Hadamard TurboQuant codec (libeoship): the
turboquant_encode / turboquant_decode steps on NCHW tensors
(runtime/backend/image_ops.go:212-300; CUDA runtime/backends/cuda/
native_linux.go:1812-2004). The spec tables (permutation, signs, centroids,
boundaries of one rotation round) come from the caller, as the quantizer
module's Spec() gives them to the reference's CUDA backend."""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .runtime import DeviceBuffer, Runtime


class HadamardTQ:
    def __init__(self, rt: Runtime, perm, signs1, signs2, centroids, boundaries, bits: int):
        self.rt = rt
        self.perm = np.ascontiguousarray(perm, np.int32)
        self.channels = int(self.perm.shape[0])
        self.bits = int(bits)
        keep = [self.perm, np.ascontiguousarray(signs1, np.float32),
                np.ascontiguousarray(signs2, np.float32),
                np.ascontiguousarray(centroids, np.float32),
                np.ascontiguousarray(boundaries, np.float32)]
        if keep[3].shape != (1 << self.bits,) or keep[4].shape != ((1 << self.bits) - 1,):
            raise ValueError("centroids [2^bits] and boundaries [2^bits - 1] required")
        spec = _lib.EosHipHadamardSpec(self.channels, self.bits,
                                       *[k.ctypes.data_as(C.c_void_p).value for k in keep])
        self.handle = C.c_void_p()
        _lib.call("eoship_hadamard_tq_bind", rt.handle, C.byref(spec), C.byref(self.handle))

    def release(self) -> None:
        if self.handle and self.rt.handle:
            _lib.call("eoship_hadamard_tq_release", self.rt.handle, self.handle)
        self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass

    def encode(self, x: np.ndarray):
        """f32 [n, C, H, W] -> (coords u8 [n, C, H, W], norm codes u8 [n, H, W])."""
        x = np.ascontiguousarray(x, np.float32)
        n, c, h, w = x.shape
        if c != self.channels:
            raise ValueError("channel count differs from the spec")
        dx = DeviceBuffer.from_array(self.rt, x)
        dc = DeviceBuffer(self.rt, max(1, x.size))
        dn = DeviceBuffer(self.rt, max(1, n * h * w))
        try:
            _lib.call("eoship_hadamard_tq_encode_device", self.rt.handle, self.handle, dx.ptr,
                      C.c_int32(n), C.c_int32(h), C.c_int32(w), dc.ptr, dn.ptr)
            return dc.download(np.uint8, x.shape), dn.download(np.uint8, (n, h, w))
        finally:
            for b in (dx, dc, dn):
                b.free()

    def decode(self, coords: np.ndarray, norms: np.ndarray) -> np.ndarray:
        coords = np.ascontiguousarray(coords, np.uint8)
        norms = np.ascontiguousarray(norms, np.uint8)
        n, c, h, w = coords.shape
        dc = DeviceBuffer.from_array(self.rt, coords)
        dn = DeviceBuffer.from_array(self.rt, norms)
        do = DeviceBuffer(self.rt, max(4, coords.size * 4))
        try:
            _lib.call("eoship_hadamard_tq_decode_device", self.rt.handle, self.handle, dc.ptr,
                      dn.ptr, C.c_int32(n), C.c_int32(h), C.c_int32(w), do.ptr)
            return do.download(np.float32, coords.shape)
        finally:
            for b in (dc, dn, do):
                b.free()
