"""The reference's matmul / reduce / transpose / dtype-matrix cases on the
interpreter (CPU); tests/test_gpu_ref_suite.py runs them on the GPU."""

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd.errors import TraceError
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
    with pytest.raises(TraceError, match="batch"):
        trace(call, np.zeros((2, 4, 4), np.float32), np.zeros((2, 4, 4), np.float32))


def test_keepdims_stages_broadcast_in_dim():
    from palladium_amd.frontend import jnp

    def kernel(x_ref, o_ref):
        o_ref[...] = jnp.sum(x_ref[...], axis=1, keepdims=True)

    spec = trace(pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((3, 1), np.float32)),
                 np.zeros((3, 4), np.float32))
    names = [e.primitive.name for e in spec.jaxpr.eqns]
    assert names[names.index("reduce_sum") + 1] == "broadcast_in_dim"
