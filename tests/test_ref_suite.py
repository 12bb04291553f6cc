"""The reference's matmul / reduce / transpose / dtype-matrix cases on the
interpreter (CPU); tests/test_gpu_ref_suite.py runs them on the GPU."""

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd.errors import EmitError, TraceError
from palladium_amd.frontend import lax, pl
from palladium_amd.trace import trace
from ref_suite_cases import CASES, check


@pytest.mark.parametrize("name", sorted(CASES))
def test_interpreter_matches_closed_form(name):
    kernel, out_shape, args, _ = CASES[name]()
    check(name, pa.hip_call(kernel, out_shape=out_shape).interpret(*args))


def test_batched_dot_general_is_rejected():
    """Batch dims stay unsupported (reference test_12_matmul.py:58-71)."""
    def kernel(a_ref, b_ref, o_ref):
        o_ref[...] = lax.dot_general(a_ref[...], b_ref[...], (((2,), (1,)), ((0,), (0,))))

    call = pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((2, 4, 4), np.float32))
    spec = trace(call, np.zeros((2, 4, 4), np.float32), np.zeros((2, 4, 4), np.float32))
    assert spec.jaxpr.eqns[-2].outvars[0].aval.shape == (2, 4, 4)  # JAX's batch-first output shape
    with pytest.raises(EmitError, match="batch dims"):
        pa.emit_hip(spec)


def test_keepdims_stages_broadcast_in_dim():
    from palladium_amd.frontend import jnp

    def kernel(x_ref, o_ref):
        o_ref[...] = jnp.sum(x_ref[...], axis=1, keepdims=True)

    spec = trace(pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((3, 1), np.float32)),
                 np.zeros((3, 4), np.float32))
    names = [e.primitive.name for e in spec.jaxpr.eqns]
    assert names[names.index("reduce_sum") + 1] == "broadcast_in_dim"


def test_function_with_one_pallas_call_traces():
    from palladium_amd.frontend import jnp

    def kernel(x_ref, o_ref):
        o_ref[...] = jnp.abs(x_ref[...])

    def wrapper(x):
        return pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((8,), np.float32))(x * 2)

    spec = trace(wrapper, np.zeros(8, np.float32))
    assert spec.name == "kernel" and spec.inputs[0].array_shape == (8,)


@pytest.mark.parametrize("n", [0, 2])
def test_zero_or_several_pallas_calls_rejected(n):
    """reference tests/test_16_diagnostics.py:135-149"""
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...]

    def calls(x):
        for _ in range(n):
            x = pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((8,), np.float32))(x)
        return x

    with pytest.raises(TraceError, match=f"found {n} pallas_call"):
        trace(calls, np.zeros(8, np.float32))


def test_preferred_element_type_accumulates_in_float32():
    """reference tests/test_16_diagnostics.py:214-233: a_i = b_i = 1 + 2^-10
    (exact in float16); each product 1 + 2^-9 + 2^-20 is exact in float32 but
    not in float16, so a kernel that multiplies in half is off by 2^-16."""
    from palladium_amd.frontend import jnp

    def kernel(a_ref, b_ref, o_ref):
        o_ref[...] = lax.dot_general(a_ref[...], b_ref[...], (((1,), (0,)), ((), ())),
                                     preferred_element_type=jnp.float32)

    k = 16
    a = np.full((7, k), 1 + 2**-10, dtype=np.float16)
    b = np.full((k, 8), 1 + 2**-10, dtype=np.float16)
    call = pa.hip_call(kernel, out_shape=pl.ShapeDtypeStruct((7, 8), np.float32))
    got = call.interpret(a, b)
    assert got.dtype == np.float32
    np.testing.assert_allclose(got, np.full((7, 8), k * (1 + 2**-9 + 2**-20)), rtol=0, atol=2**-17)
