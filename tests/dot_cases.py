"""Shared `dot_general` kernels for the CPU and GPU tests: each case is
(name, builder) where builder(rng) -> (hip_call kwargs-free callable factory, inputs)."""

import numpy as np

import palladium_amd as pa
from palladium_amd.frontend import jnp, lax, pl

F32 = np.float32


def _call(kernel, grid, in_specs, out_spec, out_shape, factory=None, **kw):
    factory = factory or pa.hip_call
    return factory(kernel, grid=grid, in_specs=in_specs, out_specs=out_spec, out_shape=out_shape, **kw)


def lane_rows(rng, b=128, k=8, n=4, rows=1024, **kw):
    """(B, K) @ (K, N) per program: lhs rows across lanes."""
    def kernel(a_ref, w_ref, o_ref):
        o_ref[...] = jnp.dot(a_ref[...], w_ref[...])
    a = rng.standard_normal((rows, k)).astype(F32)
    w = rng.standard_normal((k, n)).astype(F32)
    f = _call(kernel, (rows // b,), [pl.BlockSpec((b, k), lambda i: (i, 0)), pl.BlockSpec((k, n), lambda i: (0, 0))],
              pl.BlockSpec((b, n), lambda i: (i, 0)), pl.ShapeDtypeStruct((rows, n), F32), **kw)
    return f, (a, w)


def instance_small(rng, m=3, k=5, n=4, grid=300, **kw):
    """Per-instance (M, K) @ (K, N) with a.T-style and vector forms mixed in."""
    def kernel(a_ref, b_ref, v_ref, o_ref, p_ref, s_ref):
        a = a_ref[0]          # (M, K)
        b = b_ref[0]          # (K, N)
        v = v_ref[0]          # (K,)
        o_ref[0] = a @ b                                  # (M, N)
        p_ref[0] = lax.dot_general(b, a, (((0,), (1,)), ((), ())))  # (N, M) = b.T @ a.T
        s_ref[0] = jnp.dot(v, v) + jnp.sum(jnp.dot(a, v))  # scalar
    a = rng.standard_normal((grid, m, k)).astype(F32)
    b = rng.standard_normal((grid, k, n)).astype(F32)
    v = rng.standard_normal((grid, k)).astype(F32)
    blk = lambda *s: pl.BlockSpec((1, *s), lambda i: (i,) + (0,) * len(s))  # noqa: E731
    f = pa.hip_call(kernel, grid=(grid,), in_specs=[blk(m, k), blk(k, n), blk(k)],
                    out_specs=(blk(m, n), blk(n, m), pl.BlockSpec((1,), lambda i: (i,))),
                    out_shape=(pl.ShapeDtypeStruct((grid, m, n), F32), pl.ShapeDtypeStruct((grid, n, m), F32),
                               pl.ShapeDtypeStruct((grid,), F32)), **kw)
    return f, (a, b, v)


def long_contraction(rng, k=96, grid=256, **kw):
    """A contraction longer than the unroll limit, rhs read from the shared operand."""
    def kernel(x_ref, w_ref, o_ref):
        o_ref[...] = jnp.dot(x_ref[...], w_ref[...])
    x = rng.standard_normal((grid * 64, k)).astype(F32)
    w = rng.standard_normal((k, 2)).astype(F32)
    f = _call(kernel, (grid,), [pl.BlockSpec((64, k), lambda i: (i, 0)), pl.BlockSpec((k, 2), lambda i: (0, 0))],
              pl.BlockSpec((64, 2), lambda i: (i, 0)), pl.ShapeDtypeStruct((grid * 64, 2), F32), **kw)
    return f, (x, w)


def int_mixed(rng, grid=200, **kw):
    """int32 contraction, and an int32 contraction accumulated in float32."""
    def kernel(a_ref, b_ref, o_ref, p_ref):
        a = a_ref[0]
        b = b_ref[0]
        o_ref[0] = jnp.dot(a, b)
        p_ref[0] = jnp.dot(a, b, preferred_element_type=jnp.float32)
    a = rng.integers(-50, 50, (grid, 2, 6)).astype(np.int32)
    b = rng.integers(-50, 50, (grid, 6, 3)).astype(np.int32)
    blk = lambda *s: pl.BlockSpec((1, *s), lambda i: (i,) + (0,) * len(s))  # noqa: E731
    f = pa.hip_call(kernel, grid=(grid,), in_specs=[blk(2, 6), blk(6, 3)], out_specs=(blk(2, 3), blk(2, 3)),
                    out_shape=(pl.ShapeDtypeStruct((grid, 2, 3), np.int32), pl.ShapeDtypeStruct((grid, 2, 3), F32)), **kw)
    return f, (a, b)


CASES = {"lane_rows": lane_rows, "instance_small": instance_small, "long_contraction": long_contraction,
         "int_mixed": int_mixed}


def numpy_reference(name, inputs):
    """float64 NumPy restatement of each case (the mathematics, not the op order)."""
    if name in ("lane_rows", "long_contraction"):
        a, w = (x.astype(np.float64) for x in inputs)
        return (a @ w,)
    if name == "instance_small":
        a, b, v = (x.astype(np.float64) for x in inputs)
        o = a @ b
        p = np.einsum("ikn,imk->inm", b, a)
        s = np.einsum("ik,ik->i", v, v) + np.einsum("imk,ik->i", a, v)
        return (o, p, s)
    if name == "int_mixed":
        a, b = (x.astype(np.int64) for x in inputs)
        o = a @ b
        return (o, o.astype(np.float64))
    raise KeyError(name)
