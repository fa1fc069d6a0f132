"""Device context and buffers over the C ABI (numpy on the host side)."""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np

from . import _lib
from ._lib import check


class Context:
    """One HIP stream + event set on one device (emu_ctx)."""

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        h = C.c_void_p()
        check(self.lib.emu_ctx_create(device, C.byref(h)), "emu_ctx_create")
        self.h = h
        self._live = True

    @property
    def live(self) -> bool:
        return self._live

    def close(self) -> None:
        """Destroy the context; buffers, models and sessions made from it become inert."""
        if self._live:
            self._live = False
            self.lib.emu_ctx_destroy(self.h)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):  # pragma: no cover - never call into HIP during interpreter teardown
        if not sys.is_finalizing():
            try:
                self.close()
            except Exception:
                pass

    def check(self, status: int, what: str) -> None:
        check(status, what, self.h)

    def sync(self) -> None:
        self.check(self.lib.emu_ctx_sync(self.h), "emu_ctx_sync")

    def device_info(self) -> tuple[int, str]:
        cus = C.c_int()
        buf = C.create_string_buffer(64)
        self.check(self.lib.emu_device_info(self.h, C.byref(cus), buf, 64), "emu_device_info")
        return cus.value, buf.value.decode()

    # -- buffers --------------------------------------------------------
    def alloc(self, nbytes: int) -> "DeviceBuffer":
        return DeviceBuffer(self, nbytes)

    def upload(self, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = DeviceBuffer(self, arr.nbytes)
        buf.write(arr)
        buf.dtype = arr.dtype
        buf.shape = arr.shape
        return buf

    def event_record(self, slot: int) -> None:
        self.check(self.lib.emu_event_record(self.h, slot), "emu_event_record")

    def hbm_read_rate(self, nbytes: int = 2 << 30, passes: int = 4) -> float:
        """GB/s that HBM delivers to a read-only stream of an nbytes buffer
        (emu_hbm_read_rate), the storage rate of the scan metrics."""
        buf = self.alloc(nbytes)
        try:
            gbs = C.c_float()
            self.check(self.lib.emu_hbm_read_rate(self.h, buf.ptr, nbytes, passes, C.byref(gbs)),
                       "emu_hbm_read_rate")
            return float(gbs.value)
        finally:
            buf.free()

    def host_read_rate(self, nbytes: int = 1 << 30, passes: int = 2) -> float:
        """GB/s that kernels get reading pinned host memory (over PCIe)."""
        h, d = C.c_void_p(), C.c_void_p()
        self.check(self.lib.emu_host_alloc(self.h, nbytes, C.byref(h)), "emu_host_alloc")
        try:
            C.memset(h, 0, nbytes)
            self.check(self.lib.emu_host_device_pointer(self.h, h, C.byref(d)), "emu_host_device_pointer")
            gbs = C.c_float()
            self.check(self.lib.emu_hbm_read_rate(self.h, d, nbytes, passes, C.byref(gbs)), "emu_hbm_read_rate")
            return float(gbs.value)
        finally:
            self.lib.emu_host_free(self.h, h)

    def event_elapsed(self, a: int, b: int) -> float:
        ms = C.c_float()
        self.check(self.lib.emu_event_elapsed(self.h, a, b, C.byref(ms)), "emu_event_elapsed")
        return ms.value


class DeviceBuffer:
    """Device allocation owned by the library (emu_malloc / emu_free)."""

    def __init__(self, ctx: Context, nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        ctx.check(ctx.lib.emu_malloc(ctx.h, max(self.nbytes, 1), C.byref(p)), "emu_malloc")
        self.ptr = p
        self.dtype = np.dtype(np.uint8)
        self.shape = (self.nbytes,)

    @property
    def addr(self) -> int:
        return self.ptr.value

    def free(self) -> None:
        if self.ptr is not None and self.ptr.value and self.ctx.live:
            self.ctx.lib.emu_free(self.ctx.h, self.ptr)
        self.ptr = None

    def __del__(self):  # pragma: no cover
        if not sys.is_finalizing():
            try:
                self.free()
            except Exception:
                pass

    def write(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise ValueError("write past the end of the device buffer")
        self.ctx.check(
            self.ctx.lib.emu_memcpy_htod(self.ctx.h, C.c_void_p(self.addr + offset),
                                         arr.ctypes.data_as(C.c_void_p), arr.nbytes),
            "emu_memcpy_htod")

    def read(self, dtype=None, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype or self.dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("read past the end of the device buffer")
        self.ctx.check(
            self.ctx.lib.emu_memcpy_dtoh(self.ctx.h, out.ctypes.data_as(C.c_void_p),
                                         C.c_void_p(self.addr + offset), out.nbytes),
            "emu_memcpy_dtoh")
        return out

    def zero(self) -> None:
        self.ctx.check(self.ctx.lib.emu_memset(self.ctx.h, self.ptr, 0, self.nbytes), "emu_memset")
