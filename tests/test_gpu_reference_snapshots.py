"""The reference's snapshot kernels (tests/test_msl_snapshots.py:34-110 of
the reference) run on the GPU under SAFE against NumPy closed forms."""

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd.frontend import jnp, lax, pl

pytestmark = pytest.mark.gpu
F = np.float32


def test_copy_2d(rng):
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...]

    x = rng.standard_normal((16, 32)).astype(F)
    f = pa.hip_call(kernel, out_shape=pl.ShapeDtypeStruct((16, 32), F), math_mode="safe")
    np.testing.assert_array_equal(f(x), x)


def test_blocked_saxpy(rng):
    def kernel(x_ref, y_ref, o_ref):
        o_ref[...] = 2.5 * x_ref[...] + y_ref[...]

    spec_8 = pl.BlockSpec((8,), lambda i: (i,))
    f = pa.hip_call(kernel, grid=(32,), in_specs=[spec_8, spec_8], out_specs=spec_8,
                    out_shape=pl.ShapeDtypeStruct((256,), F), math_mode="safe")
    x = rng.standard_normal(256).astype(F)
    y = rng.standard_normal(256).astype(F)
    np.testing.assert_array_equal(f(x, y), F(2.5) * x + y)  # two roundings, as NumPy float32


def test_conditional_loop(rng):
    def kernel(y0_ref, r_ref, o_ref):
        r = r_ref[...]

        def step(_, y):
            grown = y + r
            return jnp.where(grown <= 1.0, grown, y)

        o_ref[...] = lax.fori_loop(0, 20, step, y0_ref[...])

    f = pa.hip_call(kernel, out_shape=pl.ShapeDtypeStruct((64,), F), math_mode="safe")
    y0 = rng.uniform(-1, 1, 64).astype(F)
    r = rng.uniform(0, 0.2, 64).astype(F)
    want = y0.copy()
    for _ in range(20):
        grown = want + r
        want = np.where(grown <= F(1.0), grown, want)
    got = f(y0, r)
    np.testing.assert_array_equal(got, want)
    # closed form: y0 + k r with k the largest count <= 20 keeping y0 + k r <= 1
    assert np.all(got <= 1.0) and np.all(got >= y0)
