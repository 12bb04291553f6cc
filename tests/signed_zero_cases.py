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
