"""df32 RK4 LV on the GPU: bit-exact against the C oracle's df32 (same
operation sequence under SAFE math) and ~1e4x closer to float64 than fp32."""

import numpy as np
import pytest

import oracle
from palladium_amd.df32 import lv_rk4_df32
from palladium_amd.workloads import lv_inputs

pytestmark = pytest.mark.gpu


def test_df32_lv_bit_exact_vs_oracle():
    args = lv_inputs(3000, 1)
    got = lv_rk4_df32(*args, 0.005, 400)
    want = oracle.lv_rk4_df32(*args, 0.005, 400)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)


def test_df32_more_accurate_than_fp32():
    args = lv_inputs(2048, 0)
    xh, xl, _, _ = lv_rk4_df32(*args, 0.01, 500)
    wxh, wxl, _, _ = oracle.lv_rk4_df32(*args, 0.01, 500)
    x32, _ = oracle.lv_rk4(*args, 0.01, 500)
    ref = wxh.astype(np.float64) + wxl
    assert np.max(np.abs(xh.astype(np.float64) + xl - ref)) == 0.0
    assert np.max(np.abs(x32 - ref)) > 1e3 * 1e-10


def test_full_config4b_bit_exact_on_a_sample():
    """Config 4b at full size (N = 1e6, config-1 inputs, dt = 0.005, 4,000
    steps, SAFE); the first 16,384 trajectories against the oracle."""
    from palladium_amd.workloads import LV_CFG1

    cfg = LV_CFG1
    args = lv_inputs(cfg.n, cfg.seed)
    got = lv_rk4_df32(*args, cfg.dt, cfg.steps)
    m = 16384
    want = oracle.lv_rk4_df32(*(a[:m] for a in args), cfg.dt, cfg.steps)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g[:m], w)
    assert all(np.all(np.isfinite(g)) for g in got)
