"""ctypes loader for oracle.c (TEST INFRASTRUCTURE ONLY).

The shared object is built by oracle/build.py into oracle/_build/.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"
_LIB = None


def available() -> bool:
    return LIB_PATH.exists()


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle library not built at {LIB_PATH}; run python oracle/build.py")
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        I = ctypes.c_int
        L.oracle_matmul_i8.argtypes = [P, P, P, I, I, I, I]
        L.oracle_matmul_i8.restype = None
        L.oracle_dense_int4_nn.argtypes = [P, P, P, P, P, I, I, I, I, I, I, I, I]
        L.oracle_dense_int4_nn.restype = None
        L.oracle_max_threads.restype = I
        _LIB = L
    return _LIB


def default_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def matmul_i8(a: np.ndarray, b: np.ndarray, threads: int | None = None) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    m, k = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError("inner dimensions differ")
    c = np.empty((m, n), dtype=np.int32)
    lib().oracle_matmul_i8(_ptr(a), _ptr(b), _ptr(c), m, n, k, threads or default_threads())
    return c


def dense_int4_nn(a_packed, b_packed, a_scale_bits, b_scale_bits, *, m: int, n: int, k: int,
                  subchannel: int = 0, epilogue: int = 0, row0: int = 0, rows: int | None = None,
                  threads: int | None = None) -> np.ndarray:
    """bf16 bits of the whole dense int4 NN path for rows [row0, row0+rows)."""
    a = np.ascontiguousarray(a_packed, dtype=np.uint8)
    b = np.ascontiguousarray(b_packed, dtype=np.uint8)
    sa = np.ascontiguousarray(a_scale_bits, dtype=np.uint16)
    sb = np.ascontiguousarray(b_scale_bits, dtype=np.uint16)
    rows = m - row0 if rows is None else rows
    out = np.zeros((m, n), dtype=np.uint16)
    lib().oracle_dense_int4_nn(_ptr(a), _ptr(b), _ptr(sa), _ptr(sb), _ptr(out), m, n, k, subchannel, epilogue,
                               row0, rows, threads or default_threads())
    return out
