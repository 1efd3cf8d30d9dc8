"""Device-buffer helpers of the GPU parity tests (everything goes through the C ABI)."""
from __future__ import annotations

import sys

import numpy as np

from sharplight_amd import native


def log(msg: str) -> None:
    """Names the case on stdout before each GPU step, so a failing run says what it was doing."""
    print(msg, flush=True)
    sys.stdout.flush()


class Dev:
    """Owns the device buffers of one test; element offsets let a test misalign a tensor on purpose."""

    def __init__(self):
        self.bufs = []

    def put(self, arr: np.ndarray, pad_bytes: int = 0):
        """Uploads ``arr`` at byte offset ``pad_bytes`` into a fresh buffer; returns the device address."""
        arr = np.ascontiguousarray(arr)
        b = native.DeviceBuffer(max(arr.nbytes + pad_bytes, 16))
        if arr.nbytes:
            b.upload(arr, offset=pad_bytes)
        self.bufs.append(b)
        return b.ptr + pad_bytes

    def empty(self, nbytes: int, pad_bytes: int = 0, fill: int | None = 0xAB):
        b = native.DeviceBuffer(max(nbytes + pad_bytes, 16))
        if fill is not None:
            native.call("slhip_memset", b.ptr, fill, b.nbytes, None)
        self.bufs.append(b)
        return b.ptr + pad_bytes

    @staticmethod
    def get(addr: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        if out.nbytes:
            native.call("slhip_memcpy_d2h", out.ctypes.data, addr, out.nbytes, None)
        native.synchronize()
        return out

    def free(self):
        for b in self.bufs:
            b.free()
        self.bufs = []

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        native.synchronize()
        self.free()
