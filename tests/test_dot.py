"""`dot_general` staging, lowering and interpretation (CPU)."""

import numpy as np
import pytest

from dot_cases import CASES, numpy_reference
from palladium_amd import runtime as rt
from palladium_amd.emit import emit_hip
from palladium_amd.emit.lanes import lane_transform
from palladium_amd.errors import TraceError
from palladium_amd.frontend import jnp, pl
from palladium_amd.trace import trace


@pytest.mark.parametrize("name", sorted(CASES))
def test_interpreter_matches_float64(name):
    f, inputs = CASES[name](np.random.default_rng(5))
    got = f.interpret(*inputs)
    got = got if isinstance(got, tuple) else (got,)
    for g, w in zip(got, numpy_reference(name, inputs)):
        if g.dtype.kind == "i":
            np.testing.assert_array_equal(g, w)
        else:
            np.testing.assert_allclose(g, w, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("name", sorted(CASES))
def test_emitted_source_compiles_for_gfx950(name):
    f, inputs = CASES[name](np.random.default_rng(5))
    spec = trace(f._staged, *inputs)
    for mode in ("safe", "fast"):
        rt.compile_code_object(emit_hip(spec, math_mode=mode), spec.name, mode)


def test_block_matmul_runs_lane_parallel():
    f, inputs = CASES["lane_rows"](np.random.default_rng(0))
    plan = lane_transform(trace(f._staged, *inputs))
    assert plan is not None and plan.lanes == 128


def test_staged_shapes_and_params():
    seen = {}

    def kernel(a_ref, b_ref, o_ref):
        a = a_ref[...]
        b = b_ref[...]
        seen["ab"] = (a @ b).shape
        seen["atb"] = jnp.dot(a.T, a).shape
        seen["vec"] = jnp.dot(b_ref[:, 0], b_ref[:, 1]).shape
        seen["mv"] = jnp.dot(a, b_ref[:, 0]).shape
        o_ref[...] = a @ b

    call = pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((3, 2), np.float32))
    spec = trace(call, np.zeros((3, 4), np.float32), np.zeros((4, 2), np.float32))
    assert seen == {"ab": (3, 2), "atb": (4, 4), "vec": (), "mv": (3,)}
    dots = [e for e in spec.jaxpr.eqns if e.primitive.name == "dot_general"]
    assert dots[-1].params["dimension_numbers"] == (((1,), (0,)), ((), ()))
    assert np.dtype(dots[-1].params["preferred_element_type"]) == np.float32


def test_mismatched_contraction_is_a_trace_error():
    def kernel(a_ref, o_ref):
        o_ref[...] = jnp.dot(a_ref[...], a_ref[...])

    call = pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((3, 3), np.float32))
    with pytest.raises(TraceError, match="contracting dims disagree"):
        trace(call, np.zeros((3, 4), np.float32))
