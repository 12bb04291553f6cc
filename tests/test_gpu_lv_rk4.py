"""RK4 Lotka-Volterra on the GPU against the C oracle.

SAFE math keeps IEEE op order with no contraction, so the emitted kernel
must reproduce oracle/oracle.c bit for bit; FAST contracts and reassociates,
so it is held to a relative tolerance instead (the reference's honest bar
for FAST is rtol=1e-3, tests/test_06_capstone_rk4.py:66-76; ours is 1e-4).
"""

import numpy as np
import pytest

import oracle
import palladium_amd as pa
from palladium_amd.workloads import LV_CFG0, lv_inputs, lv_rk4_call

pytestmark = pytest.mark.gpu


def test_safe_bit_exact_vs_oracle_cfg0_sample():
    n = 4096
    args = lv_inputs(n, LV_CFG0.seed)
    f = lv_rk4_call(n, LV_CFG0.dt, LV_CFG0.steps, math_mode=pa.MathMode.SAFE)
    gx, gy = f(*args)
    wx, wy = oracle.lv_rk4(*args, LV_CFG0.dt, LV_CFG0.steps)
    np.testing.assert_array_equal(gx, wx)
    np.testing.assert_array_equal(gy, wy)


def test_safe_max_abs_y_bit_exact():
    n = 1000  # ragged against the 256-lane workgroup
    args = lv_inputs(n, 1)
    f = lv_rk4_call(n, 0.005, 400, track_max=True, math_mode="safe")
    gx, gy, gm = f(*args)
    wx, wy, wm = oracle.lv_rk4(*args, 0.005, 400, track_max=True)
    np.testing.assert_array_equal(gx, wx)
    np.testing.assert_array_equal(gy, wy)
    np.testing.assert_array_equal(gm, wm)


def test_fast_within_tolerance():
    n = 8192
    args = lv_inputs(n, 0)
    f = lv_rk4_call(n, 0.01, 1000)
    gx, gy = f(*args)
    wx, wy = oracle.lv_rk4(*args, 0.01, 1000)
    np.testing.assert_allclose(gx, wx, rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(gy, wy, rtol=1e-4, atol=1e-6)


def test_full_config1_safe_bit_exact_and_fast_tolerance():
    """Config 1 at full size (N=1e6, dt=0.005, 4000 steps, max|y| carried)."""
    from palladium_amd.workloads import LV_CFG1

    cfg = LV_CFG1
    args = lv_inputs(cfg.n, cfg.seed)
    want = oracle.lv_rk4(*args, cfg.dt, cfg.steps, track_max=True)
    safe = lv_rk4_call(cfg.n, cfg.dt, cfg.steps, track_max=True, math_mode="safe")(*args)
    for g, w in zip(safe, want):
        np.testing.assert_array_equal(g, w)
    fast = lv_rk4_call(cfg.n, cfg.dt, cfg.steps, track_max=True)(*args)
    rel = [np.abs(g - w) / np.abs(w) for g, w in zip(fast, want)]
    print("FAST relative deviation (x, y, max|y|): max", [float(r.max()) for r in rel],
          "median", [float(np.median(r)) for r in rel])
    # FAST contracts and reassociates the 58-op step; over 4000 steps that
    # moves the final state by at most ~1.4e-4 relative (measured on MI355X).
    assert max(float(r.max()) for r in rel) < 3e-4
    assert max(float(np.median(r)) for r in rel) < 1e-5


def test_full_config1_fast_as_accurate_as_safe_against_float64():
    """The stated tolerance for FAST, made precise: on config 1 FAST's
    deviation from the SAFE oracle (up to ~1.4e-4 relative) is fp32's own
    drift over 4,000 steps, not a FAST error. On the 2,000 trajectories
    where FAST and SAFE differ most, and on 2,000 random ones, FAST is no
    further from a float64 evaluation (same float32 step constants) than
    SAFE is (measured: max 1.14e-4 vs 1.18e-4 on the worst set, medians
    2.6e-6 vs 2.7e-6 on the random set)."""
    from oracle.ref64 import lv_rk4_f64
    from palladium_amd.workloads import LV_CFG1

    cfg = LV_CFG1
    args = lv_inputs(cfg.n, cfg.seed)
    safe = oracle.lv_rk4(*args, cfg.dt, cfg.steps)
    fast = lv_rk4_call(cfg.n, cfg.dt, cfg.steps)(*args)

    def rel(a, b):
        return np.maximum(np.abs(a[0] - b[0]) / np.abs(b[0]), np.abs(a[1] - b[1]) / np.abs(b[1]))

    dev = rel(fast, safe)
    consts = (np.float32(0.5 * cfg.dt), np.float32(cfg.dt), np.float32(cfg.dt / 6))
    rng = np.random.default_rng(0)
    for idx in (np.argsort(dev)[-2000:], rng.choice(cfg.n, 2000, replace=False)):
        r64 = lv_rk4_f64(*[a[idx] for a in args], cfg.dt, cfg.steps, consts=consts)
        e_safe = rel((safe[0][idx], safe[1][idx]), r64)
        e_fast = rel((fast[0][idx], fast[1][idx]), r64)
        assert e_fast.max() <= 1.25 * e_safe.max()
        assert np.median(e_fast) <= 1.25 * np.median(e_safe)
