"""bfloat16 kernels shared by the CPU and GPU tests (reference:
tests/test_17_robustness.py:143-195 covers the bf16 copy round trip, a
computed kernel with pin(), and the FFI path)."""

import numpy as np

import palladium_amd as pa
from palladium_amd import dtypes
from palladium_amd.frontend import jnp, lax, pl

BF = dtypes.bfloat16
B = 64
N = 4096


def _spec(b=B):
    return pl.BlockSpec((b,), lambda i: (i,))


def copy(n=65536, **kw):
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...]

    return pa.hip_call(kernel, grid=(n // B,), in_specs=[_spec()], out_specs=_spec(),
                       out_shape=pl.ShapeDtypeStruct((n,), BF), **kw)


def affine(n=16, **kw):
    """The reference's `x * 2.0 + 1.0` bf16 kernel (gridless)."""
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...] * 2.0 + 1.0

    return pa.hip_call(kernel, out_shape=pl.ShapeDtypeStruct((n,), BF), **kw)


def arithmetic(**kw):
    """Correctly rounded operations only (+ - * / sqrt compare select
    min max abs neg integer_pow, conversions to and from float32, float16
    and int32): each result is the bfloat16 rounding of a float32 result
    that is itself correctly rounded, so device and interpreter agree bit
    for bit under SAFE."""
    def kernel(x_ref, y_ref, o_ref, c_ref, i_ref, h_ref):
        x = x_ref[...]
        y = y_ref[...]
        z = x * y + 0.1 * x - y / (x * x + 1.0)
        z = jnp.where(z > 0, z * 3.0, jnp.abs(z) - 0.5)
        z = z + jnp.maximum(x, y) - jnp.minimum(x, -y) + lax.integer_pow(y, 3) + jnp.sqrt(jnp.abs(y))
        o_ref[...] = z
        c_ref[...] = (x.astype(jnp.float32) * 1.0001).astype(jnp.bfloat16) - x
        i_ref[...] = (y * 100.0).astype(jnp.int32)
        h_ref[...] = ((y.astype(jnp.float16) * 3.0).astype(jnp.bfloat16) + (i_ref[...] // 7).astype(jnp.bfloat16)).astype(jnp.float32)

    return pa.hip_call(kernel, grid=(N // B,), in_specs=[_spec()] * 2, out_specs=(_spec(),) * 4,
                       out_shape=(pl.ShapeDtypeStruct((N,), BF), pl.ShapeDtypeStruct((N,), BF),
                                  pl.ShapeDtypeStruct((N,), np.int32), pl.ShapeDtypeStruct((N,), np.float32)), **kw)


def transcendental(**kw):
    """exp/log/sin/tanh in bfloat16 (computed in float32, rounded once)
    and a block sum accumulated across lanes in float32."""
    def kernel(x_ref, o_ref, s_ref):
        x = x_ref[...]
        z = jnp.exp(x * 0.5) + jnp.log(jnp.abs(x) + 1.0) + jnp.sin(x) + jnp.tanh(x)
        o_ref[...] = z
        s_ref[...] = jnp.broadcast_to(jnp.sum(z), (1,))

    return pa.hip_call(kernel, grid=(N // B,), in_specs=[_spec()], out_specs=(_spec(), pl.BlockSpec((1,), lambda i: (i,))),
                       out_shape=(pl.ShapeDtypeStruct((N,), BF), pl.ShapeDtypeStruct((N // B,), BF)), **kw)


def instance_reduce(**kw):
    """Per-instance 16-element rows: a float32-accumulated bfloat16 sum, a
    max, and a 16x16 @ 16 contraction (bfloat16 in, bfloat16 out), all in
    one thread each, so the accumulation order is the emitted one."""
    R = 16

    def kernel(x_ref, m_ref, s_ref, mx_ref, d_ref):
        x = x_ref[...]
        s_ref[...] = jnp.sum(x, keepdims=True)
        mx_ref[...] = jnp.max(x, keepdims=True)
        d_ref[...] = jnp.dot(m_ref[...], x)

    rows = 64
    row = pl.BlockSpec((R,), lambda i: (i,))
    mat = pl.BlockSpec((R, R), lambda i: (0, 0))
    one = pl.BlockSpec((1,), lambda i: (i,))
    return pa.hip_call(kernel, grid=(rows,), in_specs=[row, mat], out_specs=(one, one, row),
                       out_shape=(pl.ShapeDtypeStruct((rows,), BF), pl.ShapeDtypeStruct((rows,), BF),
                                  pl.ShapeDtypeStruct((rows * R,), BF)), **kw)


def inputs(seed=0, n=N):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n).astype(np.float32) * 2
    y = rng.standard_normal(n).astype(np.float32) * 2
    x[:8] = [0.0, -0.0, 1.0, -1.0, 3.3895e38, 1.1755e-38, 9.2e-41, 2.0]  # zeros, max, min normal, subnormal
    return dtypes.from_float(x), dtypes.from_float(y)


def all_bit_patterns():
    return np.arange(65536, dtype=np.uint32).astype(np.uint16).view(BF)
