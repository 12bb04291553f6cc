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
        L.oracle_set_threads.argtypes = [ctypes.c_int]
        L.oracle_set_threads.restype = None
        L.oracle_max_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def set_threads(n: int) -> None:
    """OpenMP threads for the oracle's parallel loops."""
    lib().oracle_set_threads(int(n))


def max_threads() -> int:
    return int(lib().oracle_max_threads())


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


_I = ctypes.POINTER(ctypes.c_int32)


def _declare_more(L):
    f, l, u = ctypes.c_float, ctypes.c_long, ctypes.c_uint32
    L.oracle_gbm.argtypes = [l, l, l, u, u, f, f, f, f, f, _F]
    L.oracle_pow.argtypes = [f, f]
    L.oracle_pow.restype = f
    L.oracle_pow_many.argtypes = [l, _F, _F, _F]
    L.oracle_pow_many.restype = None
    L.oracle_pow_log_many.argtypes = [l, _F, ctypes.POINTER(ctypes.c_double)]
    L.oracle_pow_log_many.restype = None
    L.oracle_bs3_vdp.argtypes = [l, _F, _F, _F, f, f, f, f, l, _F, _F, _F, _I, _I]
    L.oracle_bs3_vdp_r.argtypes = [l, _F, _F, _F, f, f, f, f, l, _F, _F, _F, _I, _I]
    L.oracle_rpow.argtypes = [f, f]
    L.oracle_rpow.restype = f
    L.oracle_rpow_many.argtypes = [l, _F, _F, _F]
    L.oracle_rpow_many.restype = None
    L.oracle_rpow_log.argtypes = [f]
    L.oracle_rpow_log.restype = ctypes.c_double
    L.oracle_rpow_log_many.argtypes = [l, _F, ctypes.POINTER(ctypes.c_double)]
    L.oracle_rpow_log_many.restype = None
    L.oracle_rdiv.argtypes = [f, f]
    L.oracle_rdiv.restype = f
    L.oracle_dlog2f_many.argtypes = [l, _F, _F]
    L.oracle_dexp2f_many.argtypes = [l, _F, _F]
    for fn in ("dexpf", "dlogf", "dsinf", "dcosf", "dtanhf"):
        getattr(L, f"oracle_{fn}_many").argtypes = [l, _F, _F]
    L.oracle_gbm_r.argtypes = [l, l, l, u, u, f, f, f, f, f, _F]
    L.oracle_lv_rk4_r.argtypes = [l, _F, _F, _F, _F, _F, _F, ctypes.c_double, l, _F, _F, _F]
    L.oracle_gray_scott_step.argtypes = [l, _F, _F, f, f, f, f, f, _F, _F]
    L.oracle_gray_scott.argtypes = [l, l, _F, _F, _F, _F, f, f, f, f, f]
    L.oracle_df32_add.argtypes = [l] + [_F] * 6
    L.oracle_df32_mul.argtypes = [l] + [_F] * 6
    L.oracle_lv_rk4_df32.argtypes = [l] + [_F] * 6 + [f, l] + [_F] * 4


def _lib2():
    L = lib()
    if not getattr(L, "_more", False):
        _declare_more(L)
        L._more = True
    return L


def gbm(cfg, n_paths: int, first_path: int = 0, mode: str = "ieee") -> np.ndarray:
    """Per-path undiscounted call payoff for paths [first, first+n): IEEE
    float ops with libm's transcendentals ("ieee"), or the REPRODUCIBLE
    kernel's program bit for bit ("reproducible")."""
    if mode not in ("ieee", "reproducible"):
        raise ValueError(f"mode must be 'ieee' or 'reproducible', got {mode!r}")
    out = np.empty(n_paths, np.float32)
    key = (0, cfg.seed)
    two_pi = float(np.float32(2.0 * np.pi))
    fn = _lib2().oracle_gbm if mode == "ieee" else _lib2().oracle_gbm_r
    fn(n_paths, first_path, cfg.n_steps, key[0], key[1], float(np.float32(cfg.s0)),
                       float(np.float32(cfg.strike)), float(np.float32(cfg.drift_dt)),
                       float(np.float32(cfg.vol_sqdt)), two_pi, _fp(out))
    return out


def pow32(x: float, y: float) -> np.float32:
    return np.float32(_lib2().oracle_pow(float(x), float(y)))


def pow_many(x, y) -> np.ndarray:
    """The SAFE deterministic pow, elementwise over float32 arrays."""
    x, y = np.broadcast_arrays(np.asarray(x, np.float32), np.asarray(y, np.float32))
    x = np.ascontiguousarray(x.ravel())
    y = np.ascontiguousarray(y.ravel())
    out = np.empty(x.size, np.float32)
    _lib2().oracle_pow_many(x.size, _fp(x), _fp(y), _fp(out))
    return out


def pow_log(x: np.ndarray) -> np.ndarray:
    """The double log2 the deterministic pow takes of each float base."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size, np.float64)
    _lib2().oracle_pow_log_many(x.size, _fp(x), out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    return out


def bs3_vdp(x0, v0, mu, cfg, mode: str = "safe"):
    """(t, x, v, accepted, rejected) of the adaptive loop: SAFE order
    (`mode="safe"`), or the REPRODUCIBLE mode's fused and reciprocal form
    (`mode="reproducible"`)."""
    n = x0.size
    outs = [np.empty(n, np.float32) for _ in range(3)] + [np.empty(n, np.int32) for _ in range(2)]
    a = [np.ascontiguousarray(v, np.float32) for v in (x0, v0, mu)]
    f32 = lambda v: float(np.float32(v))  # noqa: E731
    fn = {"safe": _lib2().oracle_bs3_vdp, "reproducible": _lib2().oracle_bs3_vdp_r}[mode]
    fn(n, *[_fp(v) for v in a], f32(cfg.t1), f32(cfg.dt0), f32(cfg.rtol), f32(cfg.atol),
       int(cfg.max_attempts), _fp(outs[0]), _fp(outs[1]), _fp(outs[2]),
       outs[3].ctypes.data_as(_I), outs[4].ctypes.data_as(_I))
    return tuple(outs)


def rpow(x, y) -> np.ndarray:
    """The REPRODUCIBLE mode's power, elementwise over float32 arrays."""
    x, y = np.broadcast_arrays(np.asarray(x, np.float32), np.asarray(y, np.float32))
    x = np.ascontiguousarray(x.ravel())
    y = np.ascontiguousarray(y.ravel())
    out = np.empty(x.size, np.float32)
    _lib2().oracle_rpow_many(x.size, _fp(x), _fp(y), _fp(out))
    return out


def lv_rk4_r(x0, y0, a, b, c, d, dt: float, steps: int):
    """The REPRODUCIBLE mode's RK4 LV (FAST's algebra, fused multiply-adds at
    the contraction's sites): (x, y, max|y|)."""
    arrs = [np.ascontiguousarray(v, dtype=np.float32) for v in (x0, y0, a, b, c, d)]
    n = arrs[0].size
    outs = [np.empty(n, np.float32) for _ in range(3)]
    _lib2().oracle_lv_rk4_r(n, *[_fp(v) for v in arrs], float(dt), int(steps), *[_fp(o) for o in outs])
    return tuple(outs)


def dlog2f(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(x.size, np.float32)
    _lib2().oracle_dlog2f_many(x.size, _fp(x), _fp(out))
    return out


def dexp2f(x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(x.size, np.float32)
    _lib2().oracle_dexp2f_many(x.size, _fp(x), _fp(out))
    return out


def _many(name: str, x) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.empty(x.size, np.float32)
    getattr(_lib2(), f"oracle_{name}_many")(x.size, _fp(x), _fp(out))
    return out


def dexpf(x) -> np.ndarray:
    return _many("dexpf", x)


def dlogf(x) -> np.ndarray:
    return _many("dlogf", x)


def dsinf(x) -> np.ndarray:
    return _many("dsinf", x)


def dcosf(x) -> np.ndarray:
    return _many("dcosf", x)


def dtanhf(x) -> np.ndarray:
    return _many("dtanhf", x)


def rdiv(a: float, b: float) -> np.float32:
    """The REPRODUCIBLE mode's division, a * RN(1/b)."""
    return np.float32(_lib2().oracle_rdiv(float(a), float(b)))


def rpow_log(x: float) -> float:
    return float(_lib2().oracle_rpow_log(float(x)))


def rpow_log_many(x: np.ndarray) -> np.ndarray:
    """oracle_rpow_log elementwise (the REPRODUCIBLE pow's double log2)."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size, np.float64)
    _lib2().oracle_rpow_log_many(x.size, _fp(x), out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    return out


def _gs_consts(cfg):
    f32 = lambda v: float(np.float32(v))  # noqa: E731
    return f32(cfg.du), f32(cfg.dv), f32(cfg.f), f32(cfg.f + cfg.k), f32(cfg.dt)


def gray_scott(u0, v0, cfg, steps: int):
    n = u0.shape[0]
    u = np.ascontiguousarray(u0, np.float32).copy()
    v = np.ascontiguousarray(v0, np.float32).copy()
    tu, tv = np.empty_like(u), np.empty_like(v)
    _lib2().oracle_gray_scott(n, steps, _fp(u), _fp(v), _fp(tu), _fp(tv), *_gs_consts(cfg))
    return u, v


def df32_add(ah, al, bh, bl):
    n = ah.size
    oh, ol = np.empty(n, np.float32), np.empty(n, np.float32)
    _lib2().oracle_df32_add(n, *[_fp(np.ascontiguousarray(x, np.float32)) for x in (ah, al, bh, bl)], _fp(oh), _fp(ol))
    return oh, ol


def df32_mul(ah, al, bh, bl):
    n = ah.size
    oh, ol = np.empty(n, np.float32), np.empty(n, np.float32)
    _lib2().oracle_df32_mul(n, *[_fp(np.ascontiguousarray(x, np.float32)) for x in (ah, al, bh, bl)], _fp(oh), _fp(ol))
    return oh, ol


def lv_rk4_df32(x0, y0, a, b, c, d, dt: float, steps: int):
    n = x0.size
    arrs = [np.ascontiguousarray(v, np.float32) for v in (x0, y0, a, b, c, d)]
    outs = [np.empty(n, np.float32) for _ in range(4)]
    _lib2().oracle_lv_rk4_df32(n, *[_fp(v) for v in arrs], float(np.float32(dt)), int(steps), *[_fp(o) for o in outs])
    return tuple(outs)
