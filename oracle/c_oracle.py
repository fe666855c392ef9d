"""ctypes access to the C oracle (TEST INFRASTRUCTURE ONLY)."""

from __future__ import annotations

import ctypes

import numpy as np

from oracle.build_oracle import OUT, build_oracle

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not OUT.exists():
            build_oracle()
        l = ctypes.CDLL(str(OUT))
        l.philox_many.argtypes = [ctypes.c_uint32] * 6 + [ctypes.c_int, ctypes.c_void_p]
        l.philox_many.restype = None
        l.leaf_normals.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int64,
                                   ctypes.c_int64, ctypes.c_void_p]
        l.leaf_normals.restype = None
        _lib = l
    return _lib


def philox(counter, key, n: int) -> np.ndarray:
    out = np.zeros((n, 4), dtype=np.uint32)
    lib().philox_many(*[c & 0xFFFFFFFF for c in counter], *[k & 0xFFFFFFFF for k in key], n,
                      out.ctypes.data)
    return out


def leaf_normals(seed: int, leaf: int, rows: int, cols: int) -> np.ndarray:
    out = np.zeros((rows, cols), dtype=np.float64)
    lib().leaf_normals(seed & ((1 << 64) - 1), leaf & 0xFFFFFFFF, rows, cols, out.ctypes.data)
    return out
