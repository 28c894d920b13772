"""Device memory and stream plumbing over the C ABI (no torch involved).

``Context`` wraps a ``tf_ctx`` (one stream + the device pool); ``DeviceArray``
is a typed, shaped pool allocation that frees itself back to the pool.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import call, lib

_NP_TO_TF = {
    np.dtype(np.float32): _lib.TF_F32,
    np.dtype(np.float16): _lib.TF_F16,
    np.dtype(np.int32): _lib.TF_I32,
    np.dtype(np.int64): _lib.TF_I64,
    np.dtype(np.bool_): _lib.TF_BOOL,
}
BF16 = "bfloat16"   # stored as uint16 bit patterns on the host


def tf_dtype(dtype) -> int:
    if dtype == BF16:
        return _lib.TF_BF16
    return _NP_TO_TF[np.dtype(dtype)]


def _itemsize(dtype) -> int:
    return 2 if dtype == BF16 else np.dtype(dtype).itemsize


class DeviceArray:
    """A contiguous device buffer with a shape and dtype."""

    def __init__(self, ctx: "Context", shape, dtype=np.float32):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        self.size = int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1
        self.nbytes = self.size * _itemsize(dtype)
        p = C.c_void_p()
        call("tf_hip_alloc", ctx.handle, self.nbytes, C.byref(p))
        self.ptr = p.value

    @property
    def tf_dtype(self) -> int:
        return tf_dtype(self.dtype)

    def upload(self, host: np.ndarray) -> "DeviceArray":
        host = np.ascontiguousarray(host)
        if host.nbytes != self.nbytes:
            raise ValueError(f"upload: {host.nbytes} bytes into a {self.nbytes}-byte buffer")
        call("tf_hip_memcpy", self.ctx.handle, self.ptr, host.ctypes.data, self.nbytes, _lib.TF_COPY_H2D)
        return self

    def numpy(self) -> np.ndarray:
        np_dtype = np.uint16 if self.dtype == BF16 else self.dtype
        out = np.empty(self.shape, dtype=np_dtype)
        call("tf_hip_memcpy", self.ctx.handle, out.ctypes.data, self.ptr, self.nbytes, _lib.TF_COPY_D2H)
        return out

    def free(self) -> None:
        if self.ptr is not None and self.ctx.handle is not None:
            call("tf_hip_free", self.ctx.handle, self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self, ctx: "Context"):
        self.ctx = ctx
        e = C.c_void_p()
        call("tf_hip_event_create", ctx.handle, C.byref(e))
        self.handle = e.value

    def record(self) -> None:
        call("tf_hip_event_record", self.ctx.handle, self.handle)

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        call("tf_hip_event_elapsed", self.handle, end.handle, C.byref(ms))
        return ms.value

    def __del__(self):
        try:
            lib.tf_hip_event_destroy(self.handle)
        except Exception:
            pass


class Context:
    """One tf_ctx: a device, its stream and its memory pool."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        call("tf_hip_init", device, C.byref(h))
        self.handle = h.value
        self.device = device

    def empty(self, shape, dtype=np.float32) -> DeviceArray:
        return DeviceArray(self, shape, dtype)

    def array(self, host: np.ndarray, dtype=None) -> DeviceArray:
        host = np.ascontiguousarray(host)
        d = self.empty(host.shape, dtype if dtype is not None else host.dtype)
        return d.upload(host)

    def zeros(self, shape, dtype=np.float32) -> DeviceArray:
        d = self.empty(shape, dtype)
        call("tf_hip_zero", self.handle, d.ptr, d.nbytes)
        return d

    def sync(self) -> None:
        call("tf_hip_sync", self.handle)

    def event(self) -> Event:
        return Event(self)

    def stream(self) -> int:
        s = C.c_void_p()
        call("tf_hip_stream", self.handle, C.byref(s))
        return s.value or 0

    def pool_stats(self) -> tuple[int, int]:
        r, u = C.c_uint64(), C.c_uint64()
        call("tf_hip_pool_stats", self.handle, C.byref(r), C.byref(u))
        return r.value, u.value

    def close(self) -> None:
        if self.handle is not None:
            lib.tf_hip_shutdown(self.handle)
            self.handle = None


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
