"""The exact `or(shift_right_logical(x, n), C)` -> `v_alignbit_b32` rewrite
(emit/optimize.py:funnel_shifts) on the GPU: emitted kernels equal the
interpreter bit for bit under SAFE and FAST, for unsigned and signed
words, and where the constant does not fit the shifted-out field (no
rewrite) too."""

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd.frontend import jnp, lax, pl

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", ["safe", "fast"])
@pytest.mark.parametrize("n,c,signed", [(9, 0x3F800000, False), (9, 0x3F800000, True), (20, 0xABC00000, False),
                                        (9, 0x3F800001, False), (1, 0x80000000, True), (31, 0xFFFFFFFE, False)])
def test_funnel_shift_matches_interpreter(mode, n, c, signed):
    dt = np.int32 if signed else np.uint32
    size = 4096
    x = np.random.default_rng(n).integers(0, 2 ** 32, size, dtype=np.uint64).astype(np.uint32).view(dt)
    x[:4] = np.array([0, 0xFFFFFFFF, 0x80000000, 1], np.uint32).view(dt)
    cc = np.uint32(c).view(dt)

    def kernel(x_ref, o_ref):
        v = x_ref[...]
        o_ref[...] = lax.shift_right_logical(v, jnp.asarray(n, v.dtype)) | jnp.asarray(cc, v.dtype)

    s = pl.BlockSpec((1,), lambda i: (i,))
    f = pa.hip_call(kernel, grid=(size,), in_specs=[s], out_specs=s, out_shape=pl.ShapeDtypeStruct((size,), dt),
                    math_mode=mode)
    np.testing.assert_array_equal(f(x).view(np.uint32), f.interpret(x).view(np.uint32))
    np.testing.assert_array_equal(f(x).view(np.uint32), (x.view(np.uint32) >> np.uint32(n)) | np.uint32(c))
