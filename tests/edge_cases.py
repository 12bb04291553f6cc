"""Every element-wise primitive on a grid of special values (signed zeros,
infinities, NaN, subnormals, halves, integer extremes, out-of-range
conversions and shift amounts), for the device/interpreter differential
test. Integer division, remainder, float->int conversion and shifts are
defined for every input (XLA's definitions), so the comparison is exact;
NaN results are compared as NaN (their sign and payload are not specified
by IEEE 754 and differ between x86 and gfx950)."""

import numpy as np

import palladium_amd as pa
from palladium_amd.frontend import jnp, lax, pl

FLOATS = np.array([0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 1.5, 2.5, -2.5, 3.0, 1e-40, -1e-40, 1.17549435e-38,
                   3.4028235e38, -3.4028235e38, np.inf, -np.inf, np.nan, 2147483648.0, -2147483904.0,
                   4294967296.0, 0.49999997, 8388609.0, 1e10, -7.0], np.float32)
INTS = np.array([0, 1, -1, 2, -2, 7, -7, 31, 32, 33, -32, -2**31, 2**31 - 1, -2**31 + 1, 65536, 1103515245],
                np.int64).astype(np.int32)


def float_pairs():
    x, y = np.meshgrid(FLOATS, FLOATS, indexing="ij")
    return x.reshape(-1).copy(), y.reshape(-1).copy()


def int_pairs():
    a, b = np.meshgrid(INTS, INTS, indexing="ij")
    return a.reshape(-1).copy(), b.reshape(-1).copy()


FLOAT_OPS = {
    "add": lambda x, y: x + y,
    "sub": lambda x, y: x - y,
    "mul": lambda x, y: x * y,
    "div": lambda x, y: x / y,
    "rem": lambda x, y: lax.rem(x, y),
    "min": jnp.minimum,
    "max": jnp.maximum,
    "neg": lambda x, y: -x,
    "abs": lambda x, y: jnp.abs(x),
    "sign": lambda x, y: jnp.sign(x),
    "floor": lambda x, y: jnp.floor(x),
    "ceil": lambda x, y: jnp.ceil(x),
    "round_away": lambda x, y: lax.round(x),
    "round_even": lambda x, y: jnp.round(x),
    "sqrt": lambda x, y: jnp.sqrt(x),
    "select": lambda x, y: jnp.where(x < y, x, y),
    "clamp": lambda x, y: lax.clamp(-2.0, x, y),
    "to_f16_and_back": lambda x, y: x.astype(jnp.float16).astype(jnp.float32),
}
FLOAT_TO_INT = {
    "to_i32": lambda x: x.astype(jnp.int32),
    "to_u32": lambda x: x.astype(jnp.uint32),
    "bits": lambda x: lax.bitcast_convert_type(x, jnp.int32),
}
CMP = {"lt": jnp.less, "le": jnp.less_equal, "gt": jnp.greater, "ge": jnp.greater_equal, "eq": jnp.equal,
       "ne": jnp.not_equal}
INT_OPS = {
    "add": lambda a, b: a + b,
    "sub": lambda a, b: a - b,
    "mul": lambda a, b: a * b,
    "div": lambda a, b: lax.div(a, b),
    "rem": lambda a, b: lax.rem(a, b),
    "floordiv": lambda a, b: a // b,
    "neg": lambda a, b: -a,
    "abs": lambda a, b: jnp.abs(a),
    "and": lambda a, b: a & b,
    "or": lambda a, b: a | b,
    "xor": lambda a, b: a ^ b,
    "not": lambda a, b: ~a,
    "shl": lambda a, b: lax.shift_left(a, b),
    "shr_logical": lambda a, b: lax.shift_right_logical(a, b),
    "shr_arith": lambda a, b: lax.shift_right_arithmetic(a, b),
    "max": jnp.maximum,
    "min": jnp.minimum,
    "to_f32": lambda a, b: a.astype(jnp.float32),
    "u32_div": lambda a, b: lax.div(a.astype(jnp.uint32), b.astype(jnp.uint32)),
    "u32_rem": lambda a, b: lax.rem(a.astype(jnp.uint32), b.astype(jnp.uint32)),
    "u32_to_f32": lambda a, b: a.astype(jnp.uint32).astype(jnp.float32),
}


def _gridless(kernel, n, out_dtypes):
    return pa.hip_call(kernel, grid=(n // 64,), in_specs=[pl.BlockSpec((64,), lambda i: (i,))] * 2,
                       out_specs=tuple(pl.BlockSpec((64,), lambda i: (i,)) for _ in out_dtypes),
                       out_shape=tuple(pl.ShapeDtypeStruct((n,), d) for d in out_dtypes), math_mode="safe")


def float_call(n):
    names = list(FLOAT_OPS) + list(FLOAT_TO_INT) + list(CMP)
    dts = [np.float32] * len(FLOAT_OPS) + [np.int32, np.uint32, np.int32] + [np.bool_] * len(CMP)

    def kernel(x_ref, y_ref, *outs):
        x, y = x_ref[...], y_ref[...]
        vals = [f(x, y) for f in FLOAT_OPS.values()] + [f(x) for f in FLOAT_TO_INT.values()] + \
               [f(x, y) for f in CMP.values()]
        for o, v in zip(outs, vals):
            o[...] = v

    return names, _gridless(kernel, n, dts)


def int_call(n):
    names = list(INT_OPS)
    probe = {"to_f32": np.float32, "u32_div": np.uint32, "u32_rem": np.uint32, "u32_to_f32": np.float32}
    dts = [probe.get(k, np.int32) for k in names]

    def kernel(a_ref, b_ref, *outs):
        a, b = a_ref[...], b_ref[...]
        for o, f in zip(outs, INT_OPS.values()):
            o[...] = f(a, b)

    return names, _gridless(kernel, n, dts)


def pad64(*arrays):
    n = arrays[0].size
    m = -(-n // 64) * 64
    return n, tuple(np.concatenate([a, np.repeat(a[-1:], m - n)]) for a in arrays)


def same(g, w):
    """Bitwise equality, NaN compared as NaN."""
    g, w = np.asarray(g), np.asarray(w)
    if g.dtype.kind == "f":
        nan = np.isnan(w)
        if not np.array_equal(np.isnan(g), nan):
            return False
        g, w = g[~nan], w[~nan]
    return np.array_equal(np.ascontiguousarray(g).view(np.uint8), np.ascontiguousarray(w).view(np.uint8))


TRANSCENDENTAL = {
    "exp": lambda x, y: jnp.exp(x),
    "exp2": lambda x, y: jnp.exp2(x),
    "expm1": lambda x, y: jnp.expm1(x),
    "log": lambda x, y: jnp.log(x),
    "log1p": lambda x, y: jnp.log1p(x),
    "sin": lambda x, y: jnp.sin(x),
    "cos": lambda x, y: jnp.cos(x),
    "tan": lambda x, y: jnp.tan(x),
    "tanh": lambda x, y: jnp.tanh(x),
    "rsqrt": lambda x, y: lax.rsqrt(x),
    "logistic": lambda x, y: jax_logistic(x),
    "atan2": lambda x, y: jnp.arctan2(x, y),
    "pow": lambda x, y: x ** y,
}


def jax_logistic(x):
    return jnp.logistic(x) if hasattr(jnp, "logistic") else 1.0 / (1.0 + jnp.exp(-x))


def transcendental_call(n):
    names = list(TRANSCENDENTAL)

    def kernel(x_ref, y_ref, *outs):
        x, y = x_ref[...], y_ref[...]
        for o, f in zip(outs, TRANSCENDENTAL.values()):
            o[...] = f(x, y)

    return names, _gridless(kernel, n, [np.float32] * len(names))


def close(g, w, ulps=4):
    """Special results (NaN, infinities, zeros with their sign) equal;
    finite nonzero results within `ulps` float32 ulps."""
    g = np.asarray(g, np.float32)
    w = np.asarray(w, np.float32)
    if not np.array_equal(np.isnan(g), np.isnan(w)):
        return False
    m = ~np.isnan(w)
    g, w = g[m], w[m]
    special = np.isinf(w) | (w == 0) | np.isinf(g) | (g == 0)
    if not np.array_equal(g[special].view(np.uint32), w[special].view(np.uint32)):
        return False
    g, w = g[~special].astype(np.float64), w[~special].astype(np.float64)
    with np.errstate(over="ignore"):  # spacing of the largest finite float
        ulp = np.spacing(np.abs(w).astype(np.float32)).astype(np.float64)
    return bool(np.all(np.abs(g - w) <= ulps * ulp))
