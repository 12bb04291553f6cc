"""What the backend rejects, and how (reference: tests/test_16_diagnostics.py:
97-150): the same kernels raise the same error classes with the same key
phrases, at emission, as the reference's emitter does."""

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd import EmitError, TraceError, UnsupportedPrimitiveError
from palladium_amd.frontend import jnp, lax, pl

F = np.float32


def _shaped(*s):
    return pl.ShapeDtypeStruct(s, F)


def test_batched_dot_general_rejected():
    def kernel(a_ref, b_ref, o_ref):
        o_ref[...] = lax.dot_general(a_ref[...], b_ref[...], (((2,), (1,)), ((0,), (0,))))

    a = np.zeros((2, 4, 4), F)
    with pytest.raises(EmitError, match="batch dims"):
        pa.debug_hip(kernel, a, a, out_shape=_shaped(2, 4, 4))
    with pytest.raises(EmitError, match="batch dims"):
        pa.hip_call(kernel, out_shape=_shaped(2, 4, 4)).interpret(a, a)


def test_scan_with_stacked_ys_rejected():
    def kernel(x_ref, o_ref):
        def body(c, x):
            return c + x, c

        _c, ys = lax.scan(body, x_ref[0], x_ref[...])
        o_ref[...] = ys

    x = np.zeros(8, F)
    with pytest.raises(EmitError, match="stacked ys"):
        pa.debug_hip(kernel, x, out_shape=_shaped(8))
    with pytest.raises(EmitError, match="stacked ys"):
        pa.hip_call(kernel, out_shape=_shaped(8)).interpret(x)


def test_scan_over_xs_without_ys_rejected():
    def kernel(x_ref, o_ref):
        c, _ = lax.scan(lambda c, x: (c + x, None), x_ref[0], x_ref[...])
        o_ref[0] = c

    with pytest.raises(EmitError, match="scanned xs"):
        pa.debug_hip(kernel, np.zeros(8, F), out_shape=_shaped(1))


def test_strided_ref_access_rejected():
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[::2]

    x = np.zeros(8, F)
    with pytest.raises(EmitError, match="stride"):
        pa.debug_hip(kernel, x, out_shape=_shaped(4))
    with pytest.raises(EmitError, match="stride"):
        pa.hip_call(kernel, out_shape=_shaped(4)).interpret(x)


def test_unsupported_primitive_names_it():
    from palladium_amd.frontend.core import current_builder
    from palladium_amd.ir import ShapedArray

    def kernel(x_ref, o_ref):
        x = x_ref[...]
        (y,) = current_builder().add("sort", [x], [ShapedArray(x.shape, x.dtype)], dimension=0)
        o_ref[...] = y

    with pytest.raises(UnsupportedPrimitiveError, match="sort"):
        pa.debug_hip(kernel, np.zeros(8, F), out_shape=_shaped(8))


def test_multiple_pallas_calls_rejected():
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...]

    def two_calls(x):
        y = pl.pallas_call(kernel, out_shape=_shaped(8))(x)
        return pl.pallas_call(kernel, out_shape=_shaped(8))(y)

    with pytest.raises(TraceError, match="2 pallas_call"):
        pa.trace(two_calls, np.zeros(8, F))


def test_negative_step_is_a_trace_error():
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[::-1]

    with pytest.raises(TraceError, match="step"):
        pa.debug_hip(kernel, np.zeros(8, F), out_shape=_shaped(8))
