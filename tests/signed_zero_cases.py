"""A kernel exercising float min/max, clamp and max/min reductions on
zeros of both signs (shared by the CPU and GPU tests)."""

import numpy as np

import palladium_amd as pa
from palladium_amd import dtypes
from palladium_amd.frontend import jnp, lax, pl

N = 16
# every ordered pair of (+0, -0), then zeros against nonzeros and NaN
A = np.array([0.0, -0.0, 0.0, -0.0, 0.0, -0.0, 1.0, -1.0, np.nan, -0.0, 0.0, -0.0, 0.0, -0.0, 2.0, -2.0], np.float32)
B = np.array([-0.0, 0.0, 0.0, -0.0, 1.0, -1.0, -0.0, 0.0, -0.0, np.nan, -0.0, 0.0, -0.0, 0.0, 0.0, -0.0], np.float32)


def call(dtype=np.float32):
    def kernel(a_ref, b_ref, mn_ref, mx_ref, cl_ref, rmax_ref, rmin_ref):
        a, b = a_ref[...], b_ref[...]
        mn_ref[...] = jnp.minimum(a, b)
        mx_ref[...] = jnp.maximum(a, b)
        cl_ref[...] = lax.clamp(b, a, b)  # min(max(a, b), b)
        z = a * 0.0  # zeros of both signs (and a NaN)
        rmax_ref[...] = jnp.max(z, keepdims=True)
        rmin_ref[...] = jnp.min(z, keepdims=True)

    shp = pl.ShapeDtypeStruct((N,), dtype)
    one = pl.ShapeDtypeStruct((1,), dtype)
    return pa.hip_call(kernel, out_shape=(shp, shp, shp, one, one), math_mode="safe")


def inputs(dtype=np.float32):
    if dtypes.is_bf16(dtype):
        return dtypes.from_float(A), dtypes.from_float(B)
    return A.copy(), B.copy()


def expected():
    """min/max with -0 < +0 (NaN-suppressing), written out per pair."""
    def mn(x, y):
        if np.isnan(x):
            return y
        if np.isnan(y):
            return x
        if x == 0 and y == 0:
            return -0.0 if (np.signbit(x) or np.signbit(y)) else 0.0
        return min(x, y)

    def mx(x, y):
        if np.isnan(x):
            return y
        if np.isnan(y):
            return x
        if x == 0 and y == 0:
            return -0.0 if (np.signbit(x) and np.signbit(y)) else 0.0
        return max(x, y)

    lo = np.array([mn(x, y) for x, y in zip(A, B)], np.float32)
    hi = np.array([mx(x, y) for x, y in zip(A, B)], np.float32)
    cl = np.array([mn(mx(x, y), y) for x, y in zip(A, B)], np.float32)
    return lo, hi, cl, np.array([0.0], np.float32), np.array([-0.0], np.float32)


# zeros, halves, the largest float below 0.5, odd integers past 2^23,
# infinities and NaN
R = np.array([-0.0, 0.0, -0.3, 0.3, -2.5, 2.5, 0.49999997, -0.49999997, 8388609.0, -8388609.0, 1.5, -1.5,
              np.inf, -np.inf, np.nan, 1e-40], np.float32)


def rounding_inputs(dtype=np.float32):
    return dtypes.from_float(R) if dtypes.is_bf16(dtype) else R.copy()


def rounding_call(dtype=np.float32):
    def kernel(x_ref, r_ref, e_ref, s_ref, f_ref, c_ref):
        x = x_ref[...]
        r_ref[...] = lax.round(x)  # away from zero
        e_ref[...] = jnp.round(x)  # ties to even
        s_ref[...] = jnp.sign(x)
        f_ref[...] = jnp.floor(x)
        c_ref[...] = jnp.ceil(x)

    shp = pl.ShapeDtypeStruct((N,), dtype)
    return pa.hip_call(kernel, out_shape=(shp,) * 5, math_mode="safe")


def rounding_expected():
    """C roundf (halves away from zero, signed zeros kept), rintf (ties to
    even), sign keeping
    zeros and NaN, floorf/ceilf: written out with Python's exact math."""
    import math

    def rnd(v):
        if not math.isfinite(v) or v == 0:
            return v
        t = math.trunc(v)
        r = t + (math.copysign(1.0, v) if abs(v - t) >= 0.5 else 0.0)
        return math.copysign(r, v) if r == 0 else r

    def even(v):
        if not math.isfinite(v) or v == 0:
            return v
        t = math.floor(v)
        d = v - t
        r = t + 1 if (d > 0.5 or (d == 0.5 and t % 2 == 1)) else t
        return math.copysign(float(r), v) if r == 0 else float(r)

    def sgn(v):
        return v if (v == 0 or math.isnan(v)) else math.copysign(1.0, v)

    def fl(v, f):
        if not math.isfinite(v):
            return v
        r = float(f(v))
        return math.copysign(r, v) if r == 0 else r

    xs = [float(v) for v in R]
    return (np.array([rnd(v) for v in xs], np.float32), np.array([even(v) for v in xs], np.float32),
            np.array([sgn(v) for v in xs], np.float32),
            np.array([fl(v, math.floor) for v in xs], np.float32), np.array([fl(v, math.ceil) for v in xs], np.float32))
