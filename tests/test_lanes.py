"""Lane-parallel lowering (CPU): which kernels take it, what it emits, and
that it compiles."""

import numpy as np

from palladium_amd import runtime as rt
from palladium_amd.emit import emit_hip, launch_geometry
from palladium_amd.emit.lanes import lane_transform
from palladium_amd.frontend import jnp, lax, pl, random
from palladium_amd.trace import trace
from palladium_amd.workloads import GBMConfig, gbm_block_call, lv_inputs, lv_rk4_call

F = np.float32


def test_lv_blocks_of_256_go_across_lanes():
    call = lv_rk4_call(4096, 0.01, 10, block=256)
    spec = trace(call._staged, *lv_inputs(4096, 0))
    plan = lane_transform(spec)
    assert plan is not None and plan.lanes == 256
    geo = launch_geometry(spec)
    assert (geo.block, geo.blocks, geo.lanes) == (256, 16, 256)
    src = emit_hip(spec)
    assert "_lane" in src and "[256]" not in src.split("__launch_bounds__")[1]
    rt.compile_code_object(src, spec.name, "safe")


def test_one_lane_per_instance_kernels_are_untouched():
    call = lv_rk4_call(1000, 0.01, 10)
    spec = trace(call._staged, *lv_inputs(1000, 0))
    assert lane_transform(spec) is None
    assert launch_geometry(spec).lanes == 1


def test_iota_rows_and_cross_lane_sum():
    call = gbm_block_call(GBMConfig(n_steps=4), n_paths=2048)
    spec = trace(call._staged, random.key(1))
    plan = lane_transform(spec)
    assert plan is not None and plan.lanes == 256
    src = emit_hip(spec)
    assert "__shfl_xor" in src and "__syncthreads" in src and "if (_lane == 0)" in src
    rt.compile_code_object(src, spec.name, "fast")


def _lockstep_kernel(x_ref, o_ref, n_ref):
    x = x_ref[...]

    def cond(c):
        return jnp.any(c[0] > 1.0)

    def body(c):
        v, k = c
        active = v > 1.0
        return jnp.where(active, v * 0.5, v), k + jnp.where(active, 1, 0)

    v, k = lax.while_loop(cond, body, (x, jnp.zeros(x.shape, jnp.int32)))
    o_ref[...] = v
    n_ref[...] = k


def test_while_any_over_64_lanes_shares_workgroups():
    spec64 = pl.BlockSpec((64,), lambda i: (i,))
    call = pl.pallas_call(_lockstep_kernel, grid=(8,), in_specs=[spec64], out_specs=(spec64, spec64),
                          out_shape=(pl.ShapeDtypeStruct((512,), F), pl.ShapeDtypeStruct((512,), np.int32)))
    spec = trace(call, np.ones(512, F))
    plan = lane_transform(spec)
    assert plan is not None and plan.lanes == 64
    geo = launch_geometry(spec)
    assert geo.block == 256 and geo.blocks == 2
    src = emit_hip(spec)
    assert "__syncthreads" not in src  # one wavefront per instance: shuffles only
    rt.compile_code_object(src, spec.name, "safe")


def test_uniform_row_access_in_lane_mode():
    def kernel(x_ref, o_ref):
        i = lax.iota(jnp.int32, 64)
        o_ref[...] = x_ref[...] + i.astype(jnp.float32)
        o_ref[0] = x_ref[3]

    spec64 = pl.BlockSpec((64,), lambda i: (i,))
    spec = trace(pl.pallas_call(kernel, grid=(2,), in_specs=[spec64], out_specs=spec64,
                                out_shape=pl.ShapeDtypeStruct((128,), F)), np.zeros(128, F))
    plan = lane_transform(spec)
    assert plan is not None  # uniform row reads/writes are fine
    src = emit_hip(spec)
    rt.compile_code_object(src, spec.name, "safe")


def test_two_d_lane_blocks_with_column_stores():
    def kernel(x_ref, o_ref):
        x = x_ref[...]
        o_ref[:, 0] = x * 2.0
        o_ref[:, 1] = x + 1.0

    spec = trace(pl.pallas_call(kernel, grid=(4,), in_specs=[pl.BlockSpec((128,), lambda i: (i,))],
                                out_specs=pl.BlockSpec((128, 2), lambda i: (i, 0)),
                                out_shape=pl.ShapeDtypeStruct((512, 2), F)), np.zeros(512, F))
    plan = lane_transform(spec)
    assert plan is not None and plan.lanes == 128
    rt.compile_code_object(emit_hip(spec), spec.name, "safe")
