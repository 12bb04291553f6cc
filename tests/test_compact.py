"""Which loops get workgroup lane compaction, and the launch geometry that
goes with it (CPU: emission only)."""

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd.emit import emit_hip, launch_geometry
from palladium_amd.frontend import jnp, lax, pl
from palladium_amd.trace import trace
from palladium_amd.workloads import bs3_inputs, bs3_vdp_call


def _bs3_spec(n):
    return trace(bs3_vdp_call(n)._staged, *bs3_inputs(n))


def test_bs3_loop_is_compacted_in_1024_lane_workgroups():
    spec = _bs3_spec(4096)
    assert launch_geometry(spec).block == 1024
    src = emit_hip(spec, math_mode="fast")
    assert src.count("__syncthreads()") == 3
    assert "__launch_bounds__(1024)" in src
    # only the carries read after the loop keep a result slot: four of the
    # outputs and the attempt count the rejected count is rebuilt from
    assert "_cres" in src and "[5][1024]" in src


@pytest.mark.parametrize("n", [1000, 1536, 512])
def test_partial_workgroups_keep_their_extra_lanes(n):
    """A grid that does not fill its last workgroup: no lane returns early
    (every wavefront must meet the barriers); the extra lanes read the last
    instance's data, hold no instance and store nothing."""
    spec = _bs3_spec(n)
    geo = launch_geometry(spec)
    assert geo.block == 1024 and geo.blocks == -(-n // 1024)
    src = emit_hip(spec)
    assert "return;" not in src
    assert f"const bool _in = _flat < {n}u;" in src
    assert f"_in ? _flat : {n - 1}u" in src
    assert "(_in ? (int)threadIdx.x : -1)" in src
    # all five output stores are guarded
    assert src.count("if (_in) {") == 5


def test_whole_workgroups_need_no_guard():
    src = emit_hip(_bs3_spec(2048))
    body = src[src.index("extern \"C\""):]
    assert "_in " not in body and "return;" in body


def test_explicit_workgroup_size_and_env_switch(monkeypatch):
    spec = _bs3_spec(4096)
    assert launch_geometry(spec, 256).block == 256
    assert "__syncthreads" not in emit_hip(spec, block=256)
    assert "__syncthreads" in emit_hip(spec, block=1024)
    monkeypatch.setenv("PALLADIUM_WHILE_COMPACTION", "0")
    assert launch_geometry(spec).block == 256
    assert "__syncthreads" not in emit_hip(spec)


def _loop_kernel(use_pid=False, vector=False):
    def kernel(x_ref, o_ref):
        x = x_ref[...]
        if vector:
            x = jnp.broadcast_to(x, (1,))

        def cond(c):
            return c[0] > 1

        def body(c):
            v, k = c
            extra = pl.program_id(0) * 0 if use_pid else 0
            return jnp.where(v % 2 == 0, v // 2, 3 * v + 1) + extra, k + 1

        _, k = lax.while_loop(cond, body, (x, jnp.zeros_like(x)))
        o_ref[...] = k

    return kernel


def test_loops_reading_the_program_id_are_not_compacted():
    n = 2048
    spec_ok = trace(pl.pallas_call(_loop_kernel(), grid=(n,), in_specs=[pl.BlockSpec((1,), lambda i: (i,))],
                                   out_specs=pl.BlockSpec((1,), lambda i: (i,)),
                                   out_shape=pl.ShapeDtypeStruct((n,), np.int32)), np.ones(n, np.int32))
    assert "__syncthreads" in emit_hip(spec_ok)
    spec_pid = trace(pl.pallas_call(_loop_kernel(use_pid=True), grid=(n,),
                                    in_specs=[pl.BlockSpec((1,), lambda i: (i,))],
                                    out_specs=pl.BlockSpec((1,), lambda i: (i,)),
                                    out_shape=pl.ShapeDtypeStruct((n,), np.int32)), np.ones(n, np.int32))
    assert "__syncthreads" not in emit_hip(spec_pid)


def test_iterations_per_pass_follow_mode_and_body_size(monkeypatch):
    from palladium_amd.emit import compact

    spec = _bs3_spec(4096)
    assert compact.iterations_per_pass(emit_hip(spec, math_mode="fast")) == 32
    assert compact.iterations_per_pass(emit_hip(spec, math_mode="safe")) == 16
    assert compact.iterations_per_pass(emit_hip(spec)) == 16
    # a body that would not fit: fewer iterations per pass
    monkeypatch.setattr(compact, "EPOCH_UNROLL_OPS", 400)
    assert compact.iterations_per_pass(emit_hip(spec, math_mode="fast")) in (2, 4)
    monkeypatch.setattr(compact, "EPOCH_UNROLL_OPS", 10)
    assert compact.iterations_per_pass(emit_hip(spec, math_mode="fast")) == 1
    monkeypatch.setenv("PALLADIUM_EPOCH_UNROLL", "8")
    assert compact.iterations_per_pass(emit_hip(spec, math_mode="fast")) == 8
    monkeypatch.setenv("PALLADIUM_EPOCH_UNROLL", "3")
    with pytest.raises(ValueError, match="divide"):
        emit_hip(spec, math_mode="fast")
