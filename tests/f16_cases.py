"""float16 kernels shared by the CPU and GPU tests."""

import numpy as np

import palladium_amd as pa
from palladium_amd.frontend import jnp, lax, pl

F16 = np.float16
B = 64
N = 4096


def _spec():
    return pl.BlockSpec((B,), lambda i: (i,))


def arithmetic(**kw):
    """Only correctly rounded float16 operations (+ - * / compare select
    min max abs integer_pow, conversions): every result is the float16
    rounding of the exact one, so the device must agree bit for bit."""
    def kernel(x_ref, y_ref, o_ref, c_ref, i_ref):
        x = x_ref[...]
        y = y_ref[...]
        z = x * y + 0.1 * x - y / (x * x + 1.0)
        z = jnp.where(z > 0, z * 3.0, jnp.abs(z) - 0.5)
        z = z + jnp.maximum(x, y) - jnp.minimum(x, -y) + lax.integer_pow(y, 3)
        o_ref[...] = z
        c_ref[...] = (x.astype(jnp.float32) * 1.0001).astype(jnp.float16) - x
        i_ref[...] = (y * 100.0).astype(jnp.int32)

    f = pa.hip_call(kernel, grid=(N // B,), in_specs=[_spec()] * 2, out_specs=(_spec(),) * 3,
                    out_shape=(pl.ShapeDtypeStruct((N,), F16), pl.ShapeDtypeStruct((N,), F16),
                               pl.ShapeDtypeStruct((N,), np.int32)), **kw)
    return f


def transcendental(**kw):
    """exp/log/sin/sqrt in float16 (computed in float32, rounded once) and a
    block sum accumulated across lanes."""
    def kernel(x_ref, o_ref, s_ref):
        x = x_ref[...]
        z = jnp.exp(x * 0.5) + jnp.log(jnp.abs(x) + 1.0) + jnp.sin(x) + jnp.sqrt(jnp.abs(x))
        o_ref[...] = z
        s_ref[...] = jnp.broadcast_to(jnp.sum(z), (1,))

    f = pa.hip_call(kernel, grid=(N // B,), in_specs=[_spec()], out_specs=(_spec(), pl.BlockSpec((1,), lambda i: (i,))),
                    out_shape=(pl.ShapeDtypeStruct((N,), F16), pl.ShapeDtypeStruct((N // B,), F16)), **kw)
    return f


def inputs(seed=0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(N) * 2).astype(F16)
    y = (rng.standard_normal(N) * 2).astype(F16)
    x[:8] = [0.0, -0.0, 1.0, -1.0, 65504.0, 6.1e-5, 6e-8, 2.0]  # zeros, max, min normal, subnormal
    return x, y
