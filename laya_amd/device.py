"""Device context and device arrays over the library's own allocator and stream."""
from __future__ import annotations

import ctypes
import weakref
from typing import Optional, Sequence

import numpy as np

from ._native import check, lib


class Context:
    """One device, one HIP stream (laya_ctx). Calls on it are stream-ordered; sync() waits."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        check(lib().laya_ctx_create(device, ctypes.byref(h)))
        self.handle = h.value
        self.device = device
        self.matmul_precision = "fp32"
        self._dependents = weakref.WeakSet()

    def register(self, obj) -> None:
        """Objects holding library handles tied to this context; closed before the context is."""
        self._dependents.add(obj)

    def close(self) -> None:
        if getattr(self, "handle", None):
            for obj in list(self._dependents):
                obj.close()
            lib().laya_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sync(self) -> None:
        check(lib().laya_sync(self.handle))

    def set_memory_cap(self, nbytes: int) -> None:
        check(lib().laya_ctx_set_memory_cap(self.handle, nbytes))

    # Products that take bf16 operands under each policy: forward (y = x·Wᵀ), input gradient (dx = dy·W),
    # weight gradient (dW += dyᵀ·x).
    MATMUL_POLICIES = {"fp32": 0, "fp32-mfma": 8, "fp32-split3": 240, "fp32-split3-forward": 16,
                       "fp32-split3-backward": 96, "fp32-split3-attention": 128, "bf16": 7, "bf16-forward": 1,
                       "bf16-backward": 6, "bf16-weight-grad": 4}

    def set_matmul_precision(self, precision: str) -> None:
        """The operand precision of the matrix products launched afterwards: 'fp32' (default: fp32-accurate
        products from exact three-piece bf16 splits on the bf16 matrix cores), 'fp32-mfma' (the fp32 matrix
        cores), 'bf16' (every product), or one class in bf16 ('bf16-forward', 'bf16-backward',
        'bf16-weight-grad', the other classes fp32). bf16 operands are rounded to nearest even;
        accumulation and outputs stay fp32."""
        if precision not in self.MATMUL_POLICIES:
            raise ValueError(f"matmul precision '{precision}': expected one of {sorted(self.MATMUL_POLICIES)}")
        check(lib().laya_ctx_set_matmul_precision(self.handle, self.MATMUL_POLICIES[precision]))
        self.matmul_precision = precision

    def memory_in_use(self) -> int:
        v = ctypes.c_size_t()
        check(lib().laya_ctx_memory_in_use(self.handle, ctypes.byref(v)))
        return v.value

    def profile_begin(self) -> None:
        check(lib().laya_profile_begin(self.handle))

    def profile_end(self) -> dict:
        """Ends a live profile; returns {kernel: {launches, ms, flops, bytes}}."""
        L = lib()
        check(L.laya_profile_end(self.handle))
        n = ctypes.c_int()
        check(L.laya_profile_count(self.handle, ctypes.byref(n)))
        out = {}
        for i in range(n.value):
            name = ctypes.c_char_p()
            launches = ctypes.c_int()
            ms, flops, nbytes = ctypes.c_double(), ctypes.c_double(), ctypes.c_double()
            check(L.laya_profile_get(self.handle, i, ctypes.byref(name), ctypes.byref(launches), ctypes.byref(ms),
                                     ctypes.byref(flops), ctypes.byref(nbytes)))
            out[name.value.decode()] = {"launches": launches.value, "ms": ms.value, "flops": flops.value,
                                        "bytes": nbytes.value}
        return out


class DeviceArray:
    """A device allocation with a shape and dtype (fp32 or int32)."""

    def __init__(self, ctx: Context, shape: Sequence[int], dtype=np.float32, zero: bool = True):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.size = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = self.size * self.dtype.itemsize
        p = ctypes.c_void_p()
        check(lib().laya_alloc(ctx.handle, max(self.nbytes, 16), ctypes.byref(p)))
        self.ptr = p.value
        if zero and self.nbytes:
            check(lib().laya_fill(ctx.handle, self.ptr, 0.0, (self.nbytes + 3) // 4))

    @classmethod
    def from_numpy(cls, ctx: Context, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        if a.dtype not in (np.float32, np.int32):
            a = a.astype(np.float32 if np.issubdtype(a.dtype, np.floating) else np.int32)
        d = cls(ctx, a.shape, a.dtype, zero=False)
        d.upload(a)
        return d

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.size == self.size, f"size {a.size} vs {self.size}"
        check(lib().laya_upload(self.ctx.handle, self.ptr, a.ctypes.data, self.nbytes))

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(lib().laya_download(self.ctx.handle, out.ctypes.data, self.ptr, self.nbytes))
        return out

    def fill(self, value: float) -> None:
        assert self.dtype == np.float32
        check(lib().laya_fill(self.ctx.handle, self.ptr, float(value), self.size))

    def free(self) -> None:
        if getattr(self, "ptr", None) and getattr(self.ctx, "handle", None):
            lib().laya_free(self.ctx.handle, self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def device_array(ctx: Context, a: Optional[np.ndarray]) -> Optional[DeviceArray]:
    return None if a is None else DeviceArray.from_numpy(ctx, a)
