"""Context, device memory, streams and events over the C ABI.

The host-side mirror of the reference's MetalContext / PinnedBuffer /
TokenCommandBuffer plumbing (crates/hawking-core/src/metal/mod.rs): a
Context owns one hk_ctx bound to one gfx950 device; DeviceArray is a typed
device allocation with numpy upload/download; every compute call enqueues on
a stream and only `synchronize` waits.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import HawkingError


class Context:
    def __init__(self, device: int = 0):
        L = _lib.lib()
        h = C.c_void_p()
        rc = L.hk_ctx_create(device, C.byref(h))
        if rc != _lib.HK_OK:
            raise HawkingError("hk_ctx_create", rc, f"no usable gfx950 device {device}")
        self.h = h
        self.L = L
        self.stream = None  # null stream unless the caller sets one

    def close(self):
        if self.h:
            self.L.hk_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- error plumbing ---------------------------------------------------------
    def last_error(self) -> str:
        buf = C.create_string_buffer(1024)
        self.L.hk_last_error(self.h, buf, len(buf))
        return buf.value.decode(errors="replace")

    def check(self, fn: str, rc: int) -> None:
        if rc != _lib.HK_OK:
            raise HawkingError(fn, rc, self.last_error())

    def call(self, fn: str, *args) -> None:
        self.check(fn, getattr(self.L, fn)(self.h, *args))

    # -- info / sync ----------------------------------------------------------------
    def device_info(self) -> dict:
        name = C.create_string_buffer(256)
        cus = C.c_int()
        hbm = C.c_size_t()
        self.call("hk_device_info", name, len(name), C.byref(cus), C.byref(hbm))
        return {"name": name.value.decode(), "cu_count": cus.value, "hbm_bytes": hbm.value}

    def synchronize(self, stream=None) -> None:
        self.call("hk_stream_synchronize", stream if stream is not None else self.stream)

    def device_synchronize(self) -> None:
        self.call("hk_device_synchronize")

    def device_status(self, stream=None) -> int:
        bits = C.c_uint32()
        self.call("hk_check_device_status", stream if stream is not None else self.stream, C.byref(bits))
        return bits.value

    # -- memory ---------------------------------------------------------------------
    def empty(self, shape, dtype=np.float32) -> "DeviceArray":
        return DeviceArray(self, shape, dtype)

    def to_device(self, arr: np.ndarray) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        d = DeviceArray(self, arr.shape, arr.dtype)
        d.upload(arr)
        return d

    def new_stream(self):
        s = C.c_void_p()
        self.call("hk_stream_create", C.byref(s))
        return s

    def event(self) -> "Event":
        return Event(self)


class DeviceArray:
    """A typed device allocation (library-owned, freed on collection)."""

    def __init__(self, ctx: Context, shape, dtype=np.float32):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        ctx.call("hk_malloc", max(self.nbytes, 1), C.byref(p))
        self.ptr = p

    @property
    def addr(self) -> int:
        return self.ptr.value

    def offset(self, elements: int) -> C.c_void_p:
        return C.c_void_p(self.ptr.value + elements * self.dtype.itemsize)

    def upload(self, arr: np.ndarray, stream=None) -> "DeviceArray":
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        if arr.nbytes != self.nbytes:
            raise ValueError(f"upload of {arr.nbytes} bytes into a {self.nbytes}-byte array")
        s = stream if stream is not None else self.ctx.stream
        self.ctx.call("hk_memcpy_htod", self.ptr, arr.ctypes.data, arr.nbytes, s)
        self.ctx.synchronize(s)
        return self

    def download(self, stream=None) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        s = stream if stream is not None else self.ctx.stream
        self.ctx.call("hk_memcpy_dtoh", out.ctypes.data, self.ptr, self.nbytes, s)
        self.ctx.synchronize(s)
        return out

    def zero(self, stream=None) -> "DeviceArray":
        self.ctx.call("hk_memset", self.ptr, 0, self.nbytes, stream if stream is not None else self.ctx.stream)
        return self

    def free(self):
        if self.ptr and self.ptr.value and self.ctx.h:
            self.ctx.L.hk_free(self.ctx.h, self.ptr)
        self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self, ctx: Context):
        self.ctx = ctx
        e = C.c_void_p()
        ctx.call("hk_event_create", C.byref(e))
        self.h = e

    def record(self, stream=None) -> "Event":
        self.ctx.call("hk_event_record", self.h, stream if stream is not None else self.ctx.stream)
        return self

    def elapsed_ms(self, later: "Event") -> float:
        ms = C.c_float()
        self.ctx.call("hk_event_elapsed_ms", self.h, later.h, C.byref(ms))
        return float(ms.value)

    def __del__(self):
        try:
            if self.h and self.ctx.h:
                self.ctx.L.hk_event_destroy(self.ctx.h, self.h)
        except Exception:
            pass
