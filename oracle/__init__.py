"""CPU oracle for palladium_amd's hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker. `liboracle.so` is the C
restatement in oracle.c (built by oracle/Makefile); `ref64` holds float64
NumPy references used to pin it.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
_lib = None

_F = ctypes.POINTER(ctypes.c_float)
_U = ctypes.POINTER(ctypes.c_uint32)


def build() -> Path:
    subprocess.run(["make", "-C", str(HERE), "-s"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.oracle_lv_rk4.argtypes = [ctypes.c_long, _F, _F, _F, _F, _F, _F, ctypes.c_double, ctypes.c_long, _F, _F, _F]
        L.oracle_lv_rk4.restype = None
        L.oracle_threefry2x32.argtypes = [ctypes.c_uint32] * 4 + [_U, _U]
        L.oracle_random_bits.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_long, _U]
        L.oracle_fold_in.argtypes = [ctypes.c_uint32] * 3 + [_U, _U]
        L.oracle_bits_to_uniform.argtypes = [ctypes.c_uint32, ctypes.c_float, ctypes.c_float]
        L.oracle_bits_to_uniform.restype = ctypes.c_float
        _lib = L
    return _lib


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_F)


def lv_rk4(x0, y0, a, b, c, d, dt: float, steps: int, track_max: bool = False):
    """SAFE-order fp32 RK4 LV; returns (x, y) or (x, y, max|y|)."""
    arrs = [np.ascontiguousarray(v, dtype=np.float32) for v in (x0, y0, a, b, c, d)]
    n = arrs[0].size
    xo = np.empty(n, np.float32)
    yo = np.empty(n, np.float32)
    m = np.empty(n, np.float32) if track_max else None
    lib().oracle_lv_rk4(n, *[_fp(v) for v in arrs], float(dt), int(steps), _fp(xo), _fp(yo),
                        _fp(m) if m is not None else None)
    return (xo, yo, m) if track_max else (xo, yo)


def threefry2x32(k0: int, k1: int, c0: int, c1: int) -> tuple[int, int]:
    a, b = ctypes.c_uint32(), ctypes.c_uint32()
    lib().oracle_threefry2x32(k0 & 0xFFFFFFFF, k1 & 0xFFFFFFFF, c0 & 0xFFFFFFFF, c1 & 0xFFFFFFFF,
                              ctypes.byref(a), ctypes.byref(b))
    return a.value, b.value


def random_bits(key, n: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().oracle_random_bits(int(key[0]), int(key[1]), n, out.ctypes.data_as(_U))
    return out


def fold_in(key, data: int) -> np.ndarray:
    a, b = ctypes.c_uint32(), ctypes.c_uint32()
    lib().oracle_fold_in(int(key[0]), int(key[1]), data & 0xFFFFFFFF, ctypes.byref(a), ctypes.byref(b))
    return np.array([a.value, b.value], np.uint32)


def bits_to_uniform(bits: int, lo: float = 0.0, hi: float = 1.0) -> np.float32:
    return np.float32(lib().oracle_bits_to_uniform(int(bits), lo, hi))
