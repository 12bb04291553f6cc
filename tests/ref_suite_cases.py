"""Kernels mirroring the reference's topic tests (tests/test_12_matmul.py,
test_13_reduce.py, test_14_transpose.py, test_17_robustness.py dtype
matrix), each with a NumPy closed form. Shared by the CPU (interpreter)
and GPU tests."""

import numpy as np

import palladium_amd as pa
from palladium_amd import dtypes
from palladium_amd.frontend import jnp, lax, pl

F = np.float32


def _call(kernel, out_shape, **kw):
    return pa.hip_call(kernel, out_shape=out_shape, **kw)


def _rng():
    return np.random.default_rng(17)


def matmul(m, k, n):
    def kernel(a_ref, b_ref, o_ref):
        o_ref[...] = jnp.dot(a_ref[...], b_ref[...])

    r = _rng()
    a = r.standard_normal((m, k)).astype(F)
    b = r.standard_normal((k, n)).astype(F)
    return kernel, pl.ShapeDtypeStruct((m, n), F), (a, b), lambda a, b: a.astype(np.float64) @ b


def lhs_transposed_matmul():
    def kernel(a_ref, b_ref, o_ref):
        o_ref[...] = jnp.dot(a_ref[...].T, b_ref[...])

    r = _rng()
    a = r.standard_normal((5, 3)).astype(F)
    b = r.standard_normal((5, 4)).astype(F)
    return kernel, pl.ShapeDtypeStruct((3, 4), F), (a, b), lambda a, b: a.T.astype(np.float64) @ b


def rhs_transposed_matmul():
    def kernel(a_ref, b_ref, o_ref):
        o_ref[...] = jnp.dot(a_ref[...], b_ref[...].T)

    r = _rng()
    a = r.standard_normal((3, 8)).astype(F)
    b = r.standard_normal((6, 8)).astype(F)
    return kernel, pl.ShapeDtypeStruct((3, 6), F), (a, b), lambda a, b: a.astype(np.float64) @ b.T


def contract_dim0_dot_general():
    """lhs dim 0 with rhs dim 0: the reference rejects it; here the
    operand strides absorb the layout."""
    def kernel(a_ref, b_ref, o_ref):
        o_ref[...] = lax.dot_general(a_ref[...], b_ref[...], (((0,), (0,)), ((), ())))

    r = _rng()
    a = r.standard_normal((4, 3)).astype(F)
    b = r.standard_normal((4, 5)).astype(F)
    return kernel, pl.ShapeDtypeStruct((3, 5), F), (a, b), lambda a, b: a.T.astype(np.float64) @ b


def transpose(shape):
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...].T

    x = _rng().standard_normal(shape).astype(F)
    return kernel, pl.ShapeDtypeStruct(shape[::-1], F), (x,), lambda x: x.T


def reduction(kind):
    x = _rng().standard_normal((6, 10)).astype(F)
    y = _rng().standard_normal((6, 10)).astype(F)
    table = {
        "sum_scalar": (lambda v, w: jnp.sum(v, keepdims=True).reshape(1), (1,), lambda v, w: v.astype(np.float64).sum(keepdims=True).reshape(1)),
        "sum_last": (lambda v, w: jnp.sum(v, axis=-1), (6,), lambda v, w: v.astype(np.float64).sum(-1)),
        "sum_first": (lambda v, w: jnp.sum(v, axis=0), (10,), lambda v, w: v.astype(np.float64).sum(0)),
        "mean": (lambda v, w: jnp.mean(v, axis=1, keepdims=True), (6, 1), lambda v, w: v.astype(np.float64).mean(1, keepdims=True)),
        "mse": (lambda v, w: jnp.mean(jnp.square(v - w)).reshape(1), (1,), lambda v, w: np.mean((v.astype(np.float64) - w) ** 2).reshape(1)),
        "max_scalar": (lambda v, w: jnp.max(v).reshape(1), (1,), lambda v, w: v.max().reshape(1)),
        "max_last": (lambda v, w: jnp.max(v, axis=-1), (6,), lambda v, w: v.max(-1)),
        "softmax": (lambda v, w: _softmax(v * 40.0), (6, 10), lambda v, w: _np_softmax(v.astype(np.float64) * 40.0)),
    }
    fn, oshape, ref = table[kind]

    def kernel(x_ref, y_ref, o_ref):
        o_ref[...] = fn(x_ref[...], y_ref[...])

    return kernel, pl.ShapeDtypeStruct(oshape, F), (x, y), ref


def _softmax(v):
    z = v - jnp.max(v, axis=-1, keepdims=True)
    e = jnp.exp(z)
    return e / jnp.sum(e, axis=-1, keepdims=True)


def _np_softmax(v):
    e = np.exp(v - v.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def bf16_matmul(m, k, n):
    def kernel(a_ref, b_ref, o_ref):
        o_ref[...] = jnp.dot(a_ref[...], b_ref[...])

    r = _rng()
    a = dtypes.from_float(r.standard_normal((m, k)).astype(F))
    b = dtypes.from_float(r.standard_normal((k, n)).astype(F))
    return (kernel, pl.ShapeDtypeStruct((m, n), dtypes.bfloat16), (a, b),
            lambda a, b: dtypes.to_float(a).astype(np.float64) @ dtypes.to_float(b))


def dtype_case(name):
    """Round trip + one op per dtype (reference test_17_robustness.py:85-140)."""
    r = _rng()
    cases = {
        "float32": (r.standard_normal(16).astype(np.float32), lambda v: v * 2.0 + 1.0, lambda v: v * 2 + 1),
        "float16": (r.standard_normal(16).astype(np.float16), lambda v: v * 2.0 + 1.0, lambda v: v * 2 + 1),
        "int32": (np.arange(-8, 8, dtype=np.int32), lambda v: v * 3 + 1, lambda v: v * 3 + 1),
        "uint32": (np.arange(16, dtype=np.uint32), lambda v: v ^ np.uint32(0xFF), lambda v: v ^ np.uint32(0xFF)),
        "bool": (np.array([True, False] * 8), lambda v: jnp.logical_not(v), np.logical_not),
        "float16_sum": (r.standard_normal(16).astype(np.float16), lambda v: jnp.sum(v, keepdims=True),
                        lambda v: np.sum(v.astype(np.float64), keepdims=True)),
        "int32_sum": (np.arange(16, dtype=np.int32), lambda v: jnp.sum(v, keepdims=True), lambda v: np.sum(v, keepdims=True)),
        "bfloat16": (dtypes.from_float(r.standard_normal(16).astype(np.float32)), lambda v: v * 2.0 + 1.0,
                     lambda v: dtypes.to_float(v) * 2 + 1),
        "bfloat16_sum": (dtypes.from_float(r.standard_normal(16).astype(np.float32)), lambda v: jnp.sum(v, keepdims=True),
                         lambda v: np.sum(dtypes.to_float(v).astype(np.float64), keepdims=True)),
    }
    x, op, ref = cases[name]
    oshape = (1,) if name.endswith("_sum") else x.shape

    def kernel(x_ref, o_ref):
        o_ref[...] = op(x_ref[...])

    return kernel, pl.ShapeDtypeStruct(oshape, x.dtype), (x,), ref


CASES = {
    "matmul_square": lambda: matmul(8, 8, 8),
    "matmul_rect": lambda: matmul(4, 6, 10),
    "matmul_inner1": lambda: matmul(5, 1, 3),
    "matmul_lhsT": lhs_transposed_matmul,
    "matmul_rhsT": rhs_transposed_matmul,
    "dot_general_dim0": contract_dim0_dot_general,
    "transpose_rect": lambda: transpose((3, 7)),
    "transpose_square": lambda: transpose((5, 5)),
    **{f"reduce_{k}": (lambda k=k: reduction(k)) for k in
       ("sum_scalar", "sum_last", "sum_first", "mean", "mse", "max_scalar", "max_last", "softmax")},
    **{f"dtype_{k}": (lambda k=k: dtype_case(k)) for k in
       ("float32", "float16", "int32", "uint32", "bool", "float16_sum", "int32_sum", "bfloat16", "bfloat16_sum")},
    "matmul_bfloat16": lambda: bf16_matmul(4, 16, 5),
}


def check(name, got):
    kernel, out_shape, args, ref = CASES[name]()
    want = np.asarray(ref(*args))
    got = np.asarray(got)
    assert got.shape == tuple(out_shape.shape), (got.shape, out_shape.shape)
    if dtypes.is_bf16(got.dtype):
        # the reference's bf16 tolerance (tests/test_17_robustness.py:180)
        np.testing.assert_allclose(dtypes.to_float(got).astype(np.float64), want, rtol=2e-2, atol=2e-2 * max(1.0, np.abs(want).max()))
    elif np.issubdtype(got.dtype, np.floating):
        tol = 1e-2 if got.dtype == np.float16 else 1e-4
        np.testing.assert_allclose(got.astype(np.float64), want, rtol=tol, atol=tol)
    else:
        np.testing.assert_array_equal(got, want.astype(got.dtype))
