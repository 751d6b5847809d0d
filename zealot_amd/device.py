"""Device context and buffers over the C ABI (no torch: memory comes from zl_alloc)."""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _ffi


class ZealotError(RuntimeError):
    """A non-zero zl_status, with the library's error string."""

    def __init__(self, status: int, msg: str):
        super().__init__(f"zealot_hip status {status}: {msg}")
        self.status = status


class DeviceBuffer:
    """A device allocation owned by a Context (freed on close / garbage collection)."""

    def __init__(self, ctx: "Context", ptr: int, nbytes: int, shape=None, dtype=np.float32):
        self.ctx = ctx
        self.ptr = ptr
        self.nbytes = nbytes
        self.shape = tuple(shape) if shape is not None else (nbytes // np.dtype(dtype).itemsize,)
        self.dtype = np.dtype(dtype)

    @property
    def p(self) -> C.c_void_p:
        return C.c_void_p(self.ptr)

    def offset(self, elems: int) -> C.c_void_p:
        """Pointer `elems` elements past the start."""
        return C.c_void_p(self.ptr + elems * self.dtype.itemsize)

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        self.ctx.check(
            self.ctx.lib.zl_download(self.ctx.h, out.ctypes.data_as(C.c_void_p), self.p, out.nbytes),
            "zl_download",
        )
        return out

    def upload(self, arr) -> "DeviceBuffer":
        a = np.ascontiguousarray(arr, dtype=self.dtype)
        if a.nbytes != self.nbytes:
            raise ValueError(f"upload of {a.nbytes} bytes into a {self.nbytes}-byte buffer")
        self.ctx.check(
            self.ctx.lib.zl_upload(self.ctx.h, self.p, a.ctypes.data_as(C.c_void_p), a.nbytes),
            "zl_upload",
        )
        return self

    def free(self):
        if self.ptr and self.ctx.h:
            self.ctx.lib.zl_free(self.ctx.h, C.c_void_p(self.ptr))
        self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """One zl_ctx: a HIP stream on `device` with the gfx950 code object loaded.

    zl_init runs the numeric self-test; a failure raises ZealotError (the
    caller's signal to use another path, as CutileGemm::init returning None).
    """

    def __init__(self, device: int = 0):
        self.lib = _ffi.load_library()
        h = C.c_void_p()
        st = self.lib.zl_init(device, C.byref(h))
        if st != _ffi.ZL_OK:
            raise ZealotError(st, self.lib.zl_global_error().decode(errors="replace"))
        self.h = h
        self.self_test_error = float(self.lib.zl_self_test_error(h))

    def check(self, status: int, what: str = ""):
        if status != _ffi.ZL_OK:
            raise ZealotError(status, f"{what}: {self.lib.zl_last_error(self.h).decode(errors='replace')}")

    def alloc(self, shape, dtype=np.float32) -> DeviceBuffer:
        shape = (shape,) if isinstance(shape, int) else tuple(shape)
        nbytes = int(np.prod(shape, dtype=np.int64)) * np.dtype(dtype).itemsize
        p = C.c_void_p()
        self.check(self.lib.zl_alloc(self.h, max(nbytes, 4), C.byref(p)), "zl_alloc")
        return DeviceBuffer(self, p.value, nbytes, shape, dtype)

    def to_device(self, arr, dtype=None) -> DeviceBuffer:
        a = np.ascontiguousarray(arr, dtype=dtype if dtype is not None else np.asarray(arr).dtype)
        buf = self.alloc(a.shape, a.dtype)
        return buf.upload(a)

    def synchronize(self):
        self.check(self.lib.zl_synchronize(self.h), "zl_synchronize")

    def close(self):
        if self.h:
            self.lib.zl_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
