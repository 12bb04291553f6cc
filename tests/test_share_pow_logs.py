"""SAFE rewrite `share_pow_logs` (palladium_amd/emit/optimize.py): a while
loop that takes the power of a carry and of the value the carry is selected
from carries the carry's double log2 beside it. Structure on the CPU here;
bit-identity with the unshared build on the GPU in
tests/test_gpu_share_pow_logs.py."""

import dataclasses

import numpy as np
import pytest

from palladium_amd.emit import emit_hip
from palladium_amd.emit.compact import plan_for
from palladium_amd.emit.core import launch_geometry
from palladium_amd.emit.optimize import share_pow_logs
from palladium_amd.frontend import jnp, lax, pl
from palladium_amd.trace import trace
from palladium_amd.workloads import BS3Config, bs3_inputs, bs3_vdp_call


def _count(jaxpr, name):
    n = 0
    for e in jaxpr.eqns:
        n += e.primitive.name == name
        for v in e.params.values():
            sub = getattr(v, "jaxpr", v)
            if hasattr(sub, "eqns"):
                n += _count(sub, name)
    return n


def _while(jaxpr):
    (e,) = [e for e in jaxpr.eqns if e.primitive.name == "while"]
    return e, getattr(e.params["body_jaxpr"], "jaxpr", e.params["body_jaxpr"])


def _controller_kernel(order, v_powered=True, carry_by_select=True):
    """prev-style carry: out += pow(c, -0.3) * pow(v, 0.7); c = select(p, c, v)."""

    def kernel(x_ref, o_ref):
        x = x_ref[...]

        def body(s):
            k, c, acc = s
            v = jnp.abs(x) * 0.5 + k.astype(jnp.float32)
            pv = v ** 0.7 if v_powered else v * 2.0
            acc = acc + c ** -0.3 * pv
            p = v > 1.5
            if carry_by_select:
                c = jnp.where(p, v, c) if order == "v_if_true" else jnp.where(p, c, v)
            else:
                c = c * 0.5 + v
            return k + 1, c, acc

        _, c, acc = lax.while_loop(lambda s: s[0] < 5, body, (jnp.int32(0), x, jnp.zeros_like(x)))
        o_ref[...] = acc + c

    return kernel


def _spec(kernel, n=64):
    x = np.linspace(-3, 3, n, dtype=np.float32)
    s = pl.BlockSpec((1,), lambda i: (i,))
    call = pl.pallas_call(kernel, grid=(n,), in_specs=[s], out_specs=s, out_shape=pl.ShapeDtypeStruct((n,), np.float32))
    return trace(call, x)


def test_bs3_controller_takes_one_log_per_attempt():
    cfg = dataclasses.replace(BS3Config(), n=128, t1=2.0)
    spec = trace(bs3_vdp_call(128, cfg)._staged, *bs3_inputs(128))
    e0, b0 = _while(spec.jaxpr)
    opt = share_pow_logs(spec.jaxpr)
    e, b = _while(opt)
    assert _count(b0, "pow") == 2
    assert _count(b, "pow") == 0 and _count(b, "pow_with_log") == 2
    assert _count(b, "pow_log") == 1                   # log2(1/err) only; log2(prev) is carried
    assert len(e.invars) == len(e0.invars) + 1 and len(e.outvars) == len(e0.outvars) + 1
    assert str(e.invars[-1].aval.dtype) == "float64"
    assert _count(opt, "pow_log") == 2                 # + the initial carry's log, before the loop
    cond = getattr(e.params["cond_jaxpr"], "jaxpr", e.params["cond_jaxpr"])
    assert len(cond.invars) == len(b.invars) - int(e.params["body_nconsts"]) + int(e.params["cond_nconsts"])


@pytest.mark.parametrize("order", ["v_if_true", "c_if_true"])
def test_either_case_order(order):
    spec = _spec(_controller_kernel(order))
    opt = share_pow_logs(spec.jaxpr)
    _, b = _while(opt)
    assert _count(b, "pow_log") == 1 and _count(b, "pow_with_log") == 2
    # the log carry is selected with the same predicate and case order
    sel_c = [x for x in b.eqns if x.primitive.name == "select_n" and x.outvars[0] is b.outvars[1]][0]
    sel_l = [x for x in b.eqns if x.primitive.name == "select_n" and x.outvars[0] is b.outvars[-1]][0]
    assert sel_l.invars[0] is sel_c.invars[0]
    carry_pos = [k for k, u in enumerate(sel_c.invars[1:]) if u is b.invars[int(_while(opt)[0].params["body_nconsts"]) + 1]]
    log_pos = [k for k, u in enumerate(sel_l.invars[1:]) if u is b.invars[-1]]
    assert carry_pos == log_pos


@pytest.mark.parametrize("v_powered,carry_by_select", [(False, True), (True, False)])
def test_unmatched_loops_are_untouched(v_powered, carry_by_select):
    spec = _spec(_controller_kernel("v_if_true", v_powered, carry_by_select))
    assert share_pow_logs(spec.jaxpr).eqns == spec.jaxpr.eqns


def test_emitter_shares_only_under_safe_and_keeps_compaction(monkeypatch):
    spec = trace(bs3_vdp_call(2048)._staged, *bs3_inputs(2048))
    def kernel_body(mode):
        return emit_hip(spec, math_mode=mode).split("__global__")[1]

    safe = kernel_body("safe")
    assert "ph_pow_log(" in safe and "ph_pow_with_log(" in safe
    assert "__syncthreads" in safe                      # still compacted, the double carry as two LDS words
    assert "__double_as_longlong" in safe and "__longlong_as_double" in safe
    assert "ph_pow_log(" not in kernel_body("fast")
    assert "ph_pow_log(" not in kernel_body("relaxed")
    monkeypatch.setenv("PALLADIUM_SHARE_POW_LOGS", "0")
    off = kernel_body("safe")
    assert "ph_pow_log(" not in off and "__syncthreads" in off


def test_compaction_counts_double_carries_in_words():
    spec = trace(bs3_vdp_call(2048)._staged, *bs3_inputs(2048))
    assert launch_geometry(spec).block == 1024
    opt = share_pow_logs(spec.jaxpr)
    assert plan_for(spec, opt, 1, None) is not None
