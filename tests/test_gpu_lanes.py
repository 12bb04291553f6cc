"""Lane-parallel kernels on the GPU against the oracle and the interpreter."""

import numpy as np
import pytest

import oracle
import palladium_amd as pa
from palladium_amd.frontend import jnp, lax, pl, random
from palladium_amd.workloads import GBMConfig, gbm_block_call, lv_inputs, lv_rk4_call

pytestmark = pytest.mark.gpu

F = np.float32


def test_lv_cfg0_layout_blocks_of_256_bit_exact():
    # Config 0's layout: grid=(N/256,), blocks of 256 trajectories.
    n = 256 * 40
    args = lv_inputs(n, 0)
    got = lv_rk4_call(n, 0.01, 1000, block=256, math_mode="safe")(*args)
    want = oracle.lv_rk4(*args, 0.01, 1000)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)


def test_lv_cfg0_exact_ragged_layout_bit_exact():
    """Config 0 exactly: N = 100,000 (not a multiple of 256), grid
    ceil(N/256) = 391 blocks of 256; the last block's 96 tail lanes are
    masked."""
    from palladium_amd.workloads import LV_CFG0

    n = LV_CFG0.n
    args = lv_inputs(n, LV_CFG0.seed)
    call = lv_rk4_call(n, LV_CFG0.dt, LV_CFG0.steps, track_max=True, block=256, math_mode="safe")
    assert call.bound(*args).geometry.blocks == 391
    got = call(*args)
    want = oracle.lv_rk4(*args, LV_CFG0.dt, LV_CFG0.steps, track_max=True)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    fast = lv_rk4_call(n, LV_CFG0.dt, LV_CFG0.steps, block=256)(*args)
    np.testing.assert_allclose(fast[0], want[0], rtol=1e-4)


def test_gbm_block_sums_match_oracle_paths():
    cfg = GBMConfig(n_steps=32)
    n = 256 * 64
    sums = gbm_block_call(cfg, n_paths=n, math_mode="safe")(random.key(cfg.seed))
    paths = oracle.gbm(cfg, n).astype(np.float64)
    want = np.exp(-cfg.r * cfg.t) * paths.reshape(-1, 256).sum(axis=1)
    np.testing.assert_allclose(sums, want, rtol=2e-5, atol=1e-3)


def _lockstep_kernel(x_ref, o_ref, n_ref, m_ref):
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
    m_ref[0] = jnp.max(v) + jnp.min(v) + jnp.all(v <= 1.0).astype(jnp.float32)


@pytest.mark.parametrize("lanes", [64, 256])
def test_lockstep_while_any_matches_interpreter(lanes):
    n = lanes * 12
    blk = pl.BlockSpec((lanes,), lambda i: (i,))
    one = pl.BlockSpec((1,), lambda i: (i,))
    call = pa.hip_call(_lockstep_kernel, grid=(12,), in_specs=[blk], out_specs=(blk, blk, one),
                       out_shape=(pl.ShapeDtypeStruct((n,), F), pl.ShapeDtypeStruct((n,), np.int32),
                                  pl.ShapeDtypeStruct((12,), F)), math_mode="safe")
    x = (10.0 ** np.random.default_rng(lanes).uniform(-1, 4, n)).astype(F)
    got = call(x)
    want = call.interpret(x)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)


def test_two_d_blocks_column_stores():
    def kernel(x_ref, o_ref):
        x = x_ref[...]
        o_ref[:, 0] = x * 2.0
        o_ref[:, 1] = x + 1.0

    call = pa.hip_call(kernel, grid=(4,), in_specs=[pl.BlockSpec((128,), lambda i: (i,))],
                       out_specs=pl.BlockSpec((128, 2), lambda i: (i, 0)),
                       out_shape=pl.ShapeDtypeStruct((512, 2), F))
    x = np.arange(512, dtype=F)
    np.testing.assert_array_equal(call(x), np.stack([x * 2.0, x + 1.0], axis=1))


def test_two_d_threadgroups_tile_the_grid_without_changing_results():
    """A 2-D threadgroup tiles a 2-D grid (x instances of program_id(0) by y
    of program_id(1) per workgroup): same results as the default tiling and
    the interpreter, for square, tall and wide tiles."""
    import palladium_amd as pa

    def k(x_ref, o_ref):
        i, j = pl.program_id(0), pl.program_id(1)
        o_ref[i, j] = x_ref[i, j] * 2.0 + (i * 128 + j).astype(jnp.float32)

    n = 128
    x = np.random.default_rng(6).standard_normal((n, n)).astype(np.float32)
    full = pl.BlockSpec((n, n), lambda i, j: (0, 0))
    kw = dict(grid=(n, n), in_specs=[full], out_specs=full, out_shape=pl.ShapeDtypeStruct((n, n), np.float32),
              math_mode="safe")
    want = pa.hip_call(k, **kw).interpret(x)
    for tg in (None, (16, 16), (8, 32), (32, 8), (4, 64)):
        print(f"[lanes] 2-D threadgroup {tg}", flush=True)
        got = pa.hip_call(k, threadgroup=tg, **kw)(x)
        np.testing.assert_array_equal(got, want)
