"""The frontend stages the reference's primitives in the reference's order.

The RK4 kernel of examples/01_ode_ensembles.py:72-103, traced by our
frontend, must reproduce op for op (primitive, operands, folded constants)
the step body of the reference's blessed emitter output
tests/golden/rk4_lotka_volterra.metal:55-293 (extracted into
tests/golden/rk4_lotka_volterra_ops.json by tests/golden/make_rk4_ops.py).
"""

import json
from pathlib import Path

import numpy as np
import pytest

from palladium_amd.errors import TraceError
from palladium_amd.frontend import jnp, lax, pl, random
from palladium_amd.ir import Literal
from palladium_amd.trace import trace
from palladium_amd.workloads import lv_rk4_kernel

GOLDEN = Path(__file__).parent / "golden" / "rk4_lotka_volterra_ops.json"


def _lv_spec(n=8, dt=0.01, steps=500):
    s1 = pl.BlockSpec((1,), lambda i: (i,))
    call = pl.pallas_call(lv_rk4_kernel(dt, steps), grid=(n,), in_specs=[s1] * 6, out_specs=(s1, s1),
                          out_shape=(pl.ShapeDtypeStruct((n,), np.float32),) * 2)
    return trace(call, *[np.zeros(n, np.float32)] * 6)


def test_rk4_body_matches_reference_golden_op_order():
    golden = json.loads(GOLDEN.read_text())
    spec = _lv_spec(dt=golden["dt"])
    (scan,) = [e for e in spec.jaxpr.eqns if e.primitive.name == "scan"]
    body = scan.params["jaxpr"].jaxpr
    consts = body.invars[:4]
    names = {consts[0]: "a", consts[1]: "b", consts[2]: "c", consts[3]: "d", body.invars[5]: "x", body.invars[6]: "y"}
    ops = []
    for e in body.eqns:
        if e.outvars[0].aval.dtype != np.float32:
            continue  # the loop-index increment

        def norm(a):
            if isinstance(a, Literal):
                return repr(float(a.val))
            return names[a]

        ops.append([e.primitive.name, norm(e.invars[0]), norm(e.invars[1])])
        names[e.outvars[0]] = f"e{len(ops) - 1}"
    assert ops == golden["ops"]
    assert len(ops) == 58


def test_scan_layout_consts_then_index_then_carries():
    spec = _lv_spec()
    (scan,) = [e for e in spec.jaxpr.eqns if e.primitive.name == "scan"]
    assert scan.params["num_consts"] == 4
    assert scan.params["num_carry"] == 3
    assert scan.params["length"] == 500
    assert isinstance(scan.invars[4], Literal) and scan.invars[4].val == 0


def test_value_indexing_is_rejected():
    def kernel(x_ref, o_ref):
        x = x_ref[...]

        def body(c):
            i, v = c
            v = lax.cond(v[0] > 1.0, lambda v: v * 0.5, lambda v: v + 1.0, v)
            return i + 1, v

        _, v = lax.while_loop(lambda c: c[0] < 10, body, (0, x))
        o_ref[...] = v

    call = pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((1,), np.float32))
    with pytest.raises(TraceError):
        trace(call, np.zeros(1, np.float32))  # value indexing is rejected, as documented


def test_weak_carry_promotes_to_strong():
    def kernel(o_ref):
        s = lax.fori_loop(0, 3, lambda i, s: s * jnp.exp(jnp.zeros((), jnp.float32)), 100.0)
        o_ref[0] = s

    spec = trace(pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((1,), np.float32)))
    (scan,) = [e for e in spec.jaxpr.eqns if e.primitive.name == "scan"]
    assert scan.outvars[1].aval.dtype == np.float32 and not scan.outvars[1].aval.weak_type


def test_random_staging_matches_jax_primitive_sequence():
    def kernel(k_ref, o_ref):
        key = random.wrap_key_data(k_ref[...])
        o_ref[...] = random.uniform(key, (4,))

    spec = trace(pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((4,), np.float32)), np.zeros(2, np.uint32))
    names = [e.primitive.name for e in spec.jaxpr.eqns]
    assert names == ["get", "random_wrap", "random_bits", "shift_right_logical", "or", "bitcast_convert_type",
                     "sub", "mul", "add", "max", "swap"]


def test_gridless_call_has_one_instance_and_full_blocks():
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...] * 2.0

    spec = trace(pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((8, 4), np.float32)), np.zeros((8, 4), np.float32))
    assert spec.grid == (1,)
    assert spec.inputs[0].block_shape == (8, 4)


def test_squeezed_block_dims_drop_from_ref_shape():
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...]

    spec = trace(pl.pallas_call(kernel, grid=(4,), in_specs=[pl.BlockSpec((None, 16), lambda i: (i, 0))],
                                out_specs=pl.BlockSpec((None, 16), lambda i: (i, 0)),
                                out_shape=pl.ShapeDtypeStruct((4, 16), np.float32)), np.zeros((4, 16), np.float32))
    assert spec.inputs[0].block_shape == (16,)
    assert spec.inputs[0].full_block() == (1, 16)


@pytest.mark.parametrize("bad", [pl.Element(4)])
def test_unsupported_block_dims_raise_trace_error(bad):
    call = pl.pallas_call(lambda x_ref, o_ref: None, grid=(2,), in_specs=[pl.BlockSpec((bad,), lambda i: (i,))],
                          out_specs=pl.BlockSpec((4,), lambda i: (i,)), out_shape=pl.ShapeDtypeStruct((8,), np.float32))
    with pytest.raises(TraceError, match="unsupported block dim"):
        trace(call, np.zeros(8, np.float32))


def test_scratch_shapes_and_prefetch_rejected():
    with pytest.raises(TraceError, match="scratch"):
        pl.pallas_call(lambda o: None, out_shape=pl.ShapeDtypeStruct((1,), np.float32), scratch_shapes=[1])
    with pytest.raises(TraceError, match="PrefetchScalarGridSpec"):
        pl.pallas_call(lambda o: None, out_shape=pl.ShapeDtypeStruct((1,), np.float32), grid_spec=object())


def test_float64_inputs_rejected():
    call = pl.pallas_call(lambda x, o: None, out_shape=pl.ShapeDtypeStruct((1,), np.float32))
    with pytest.raises(TraceError):
        trace(call, np.zeros(1, np.float64))
