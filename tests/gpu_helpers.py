"""Shared helpers for the GPU parity tests: run the HIP path through the C ABI
and compare with the oracle under the parity metric."""
import ctypes
import hashlib

import numpy as np

from pixelina_amd import _lib
from pixelina_amd.session import Session

TOL = 1e-4  # max |y - r| / max |r| per output row (cpu_quant_matmul's fp32 outputs)


def row_rel_error(y, r):
    """Per-row max|y-r| / max|r| (rows of [columns][rows] outputs are tokens)."""
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    den = np.maximum(np.abs(r).max(axis=-1), 1e-30)
    return (np.abs(y - r).max(axis=-1) / den)


def gpu_matmul(sess, wbytes, wtype, x, rows, key=None, **kw):
    x = np.ascontiguousarray(x, np.float32)
    cols, k = x.shape
    wbytes = np.ascontiguousarray(wbytes, np.uint8)
    digest = hashlib.blake2b(wbytes.tobytes(), digest_size=16).hexdigest()
    w = sess.weight(key or f"test:{digest}:{wtype}:{rows}:{k}", wbytes, wtype, k, rows)
    xb = sess.to_device(x)
    yb = sess.alloc(cols * rows * 4)
    _lib.check(sess.matmul(w, xb.ptr, cols, yb.ptr), "pixhip_matmul")
    y = yb.download(np.float32, cols * rows).reshape(cols, rows)
    xb.free()
    yb.free()
    return y


def new_session():
    return Session(0)


class Pinned:
    """Pinned host memory from hipHostMalloc (what HipAllocator hands over)."""

    def __init__(self, sess, array):
        lib = sess.lib
        lib.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
        lib.hipHostFree.argtypes = [ctypes.c_void_p]
        self.lib, self.nbytes, self.p = lib, array.nbytes, ctypes.c_void_p()
        assert lib.hipHostMalloc(ctypes.byref(self.p), self.nbytes, 0) == 0
        ctypes.memmove(self.p, array.ctypes.data, self.nbytes)

    def read(self, dtype, shape):
        out = np.empty(shape, dtype)
        ctypes.memmove(out.ctypes.data, self.p, out.nbytes)
        return out

    def free(self):
        self.lib.hipHostFree(self.p)
