"""Operands past 2^31 elements: the emitter switches its offsets to 64-bit
(`(long long)(pid) * block`), so an instance's block can start beyond the
reach of a 32-bit index. One float32 operand of (2^21 + 1) x 1024 elements
(2^31 + 1,024; 8.6 GB in HBM, the same out) through an elementwise kernel,
one 1,024-element row per program instance; the first, middle, last and
scattered rows are checked exactly."""

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd.frontend import pl

pytestmark = pytest.mark.gpu


def test_operand_past_two_to_the_31_elements():
    rows, cols = 2**21 + 1, 1024
    print(f"[large] {rows} x {cols} float32 ({rows * cols} elements)", flush=True)

    def k(x_ref, o_ref):
        o_ref[...] = x_ref[...] * 2.0 + 1.0

    s = pl.BlockSpec((1, cols), lambda i: (i, 0))
    f = pa.hip_call(k, grid=(rows,), in_specs=[s], out_specs=s,
                    out_shape=pl.ShapeDtypeStruct((rows, cols), np.float32))
    x = (np.arange(rows, dtype=np.float32) % np.float32(4093))[:, None] \
        + np.arange(cols, dtype=np.float32)[None, :] * np.float32(0.001)
    got = f(x)
    rng = np.random.default_rng(5)
    pick = np.concatenate([[0, 1, rows // 2, rows - 2, rows - 1], rng.integers(0, rows, 64)])
    want = x[pick] * np.float32(2.0) + np.float32(1.0)
    np.testing.assert_array_equal(got[pick], want)
