"""Gray-Scott stencil on the GPU against the C oracle.

Only +, -, * are involved, so SAFE math must be bit-exact against
oracle/oracle.c for any number of steps; the multi-step driver is checked
both as plain stream launches and as one captured HIP graph."""

import numpy as np
import pytest

import oracle
import palladium_amd as pa
from palladium_amd.workloads import GS_CFG, gray_scott_call, gray_scott_initial, gray_scott_run

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("graph", [False, True])
def test_safe_bit_exact_multi_step(graph):
    size, steps = 96, 150
    u0, v0 = gray_scott_initial(size)
    call = gray_scott_call(size=size, math_mode=pa.MathMode.SAFE)
    u, v, _ = gray_scott_run(call, u0, v0, steps, graph=graph)
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, steps)
    np.testing.assert_array_equal(u, wu)
    np.testing.assert_array_equal(v, wv)


def test_single_step_call_and_periodic_wrap():
    size = 128
    rng = np.random.default_rng(3)
    u0 = rng.random((size, size), dtype=np.float32)
    v0 = rng.random((size, size), dtype=np.float32)
    u, v = gray_scott_call(size=size, math_mode="safe")(u0, v0)
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, 1)
    np.testing.assert_array_equal(u, wu)
    np.testing.assert_array_equal(v, wv)


def test_uniform_state_is_fixed_point_fast():
    size = 256
    u0 = np.ones((size, size), np.float32)
    v0 = np.zeros((size, size), np.float32)
    u, v, _ = gray_scott_run(gray_scott_call(size=size), u0, v0, 20)
    np.testing.assert_array_equal(u, u0)
    np.testing.assert_array_equal(v, v0)


def test_fast_close_to_oracle():
    size, steps = 128, 200
    u0, v0 = gray_scott_initial(size)
    u, v, _ = gray_scott_run(gray_scott_call(size=size), u0, v0, steps)
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, steps)
    np.testing.assert_allclose(u, wu, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(v, wv, rtol=1e-4, atol=1e-5)


def test_full_config4_safe_bit_exact():
    """Config 4 at full size: 4096^2, 2,000 steps as one HIP graph, SAFE,
    equal to the oracle bit for bit."""
    size, steps = GS_CFG.size, GS_CFG.steps
    u0, v0 = gray_scott_initial(size)
    u, v, _ = gray_scott_run(gray_scott_call(size=size, math_mode="safe"), u0, v0, steps)
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, steps)
    np.testing.assert_array_equal(u, wu)
    np.testing.assert_array_equal(v, wv)
    assert float(np.abs(v).sum()) > 1.0  # a pattern grew


@pytest.mark.parametrize("graph", [False, True])
def test_batch_recommit_replays_the_steps(graph):
    """Committing a batch again re-runs its launches (a graph batch is
    re-captured, the old graph released): 2 commits of 6 ping-pong steps
    equal 12 steps of the oracle."""
    from palladium_amd import runtime as rt

    size, steps = 64, 6
    u0, v0 = gray_scott_initial(size)
    bound = gray_scott_call(size=size, math_mode="safe").bound(u0, v0)
    geo = bound.geometry
    bufs = [[rt.Buffer.from_numpy(u0), rt.Buffer.from_numpy(v0)],
            [rt.Buffer.empty(u0.shape, np.float32), rt.Buffer.empty(v0.shape, np.float32)]]
    batch = rt.Batch(stream=bound.stream)
    for s in range(steps):
        src, dst = bufs[s % 2], bufs[1 - s % 2]
        batch.add(bound.kernel, geo.blocks, geo.block, [b.ptr for b in src] + [b.ptr for b in dst])
    batch.commit(graph=graph).wait()
    batch.commit(graph=graph).wait()
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, 2 * steps)
    np.testing.assert_array_equal(bufs[0][0].to_numpy(bound.stream), wu)
    np.testing.assert_array_equal(bufs[0][1].to_numpy(bound.stream), wv)
