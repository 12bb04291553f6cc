"""Adaptive BS3(2)+PI Van der Pol on the GPU against the C oracle.

Under SAFE math the device kernel runs the same IEEE op sequence as
oracle/oracle.c (including the deterministic pow), so final states and the
accepted/rejected step counts must match exactly. Under FAST, accept
decisions can flip on ulp-level differences, so the bar is the reference's
(tests/test_08_adaptive.py:174-189: counts within 20, states within a
loose tolerance)."""

import dataclasses

import numpy as np
import pytest

import oracle
import palladium_amd as pa
from palladium_amd.workloads import BS3_CFG, bs3_inputs, bs3_vdp_call

pytestmark = pytest.mark.gpu


def test_safe_exact_states_and_counts():
    n = 2048
    x0, v0, mu = bs3_inputs(n, seed=BS3_CFG.seed)
    f = bs3_vdp_call(n, math_mode=pa.MathMode.SAFE)
    got = f(x0, v0, mu)
    want = oracle.bs3_vdp(x0, v0, mu, BS3_CFG)
    for g, w, name in zip(got, want, ["t", "x", "v", "accepted", "rejected"]):
        np.testing.assert_array_equal(g, w, err_msg=name)
    assert np.all(got[0] == np.float32(BS3_CFG.t1))
    assert got[3].std() > 0  # adaptivity is per lane


def test_fast_reaches_t1_and_tracks_oracle():
    n = 4096
    x0, v0, mu = bs3_inputs(n, seed=5)
    t, x, v, acc, rej = bs3_vdp_call(n)(x0, v0, mu)
    wt, wx, wv, wacc, wrej = oracle.bs3_vdp(x0, v0, mu, BS3_CFG)
    np.testing.assert_allclose(t, BS3_CFG.t1, rtol=0, atol=1e-4)
    mild = mu < 5.0
    # FAST uses the approximate device pow and division, which shifts a
    # few controller decisions over T1=20 (twice the reference's horizon).
    np.testing.assert_allclose(acc[mild], wacc[mild], rtol=0.05, atol=20)
    assert np.mean(np.abs(acc[mild] - wacc[mild]) <= 20) > 0.99
    np.testing.assert_allclose(x[mild], wx[mild], rtol=1e-2, atol=1e-2)


def test_attempt_cap_ends_every_lane():
    # A cap far below what the stiff lanes need: every lane must still exit
    # (t < T1 for the capped ones) and match the oracle's capped run.
    cfg = dataclasses.replace(BS3_CFG, max_attempts=50)
    n = 512
    x0, v0, mu = bs3_inputs(n, seed=9)
    got = bs3_vdp_call(n, cfg, math_mode="safe")(x0, v0, mu)
    want = oracle.bs3_vdp(x0, v0, mu, cfg)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    assert np.all(got[3] + got[4] <= 50)


def test_reference_lockstep_formulation_matches_while_loop():
    """The reference's fixed-trip, self-stalling loop
    (tests/test_08_adaptive.py:33-142) ends in the same state: after T1 a
    lane only attempts zero steps. Its `steps` counter includes those idle
    accepts, so it equals max_steps - rejected."""
    from palladium_amd.workloads import bs3_vdp_lockstep_call

    n = 2048
    x0, v0, mu = bs3_inputs(n, seed=BS3_CFG.seed)
    want = oracle.bs3_vdp(x0, v0, mu, BS3_CFG)
    max_steps = int((want[3] + want[4]).max()) + 16
    t, x, v, steps, rej = bs3_vdp_lockstep_call(n, max_steps, math_mode=pa.MathMode.SAFE)(x0, v0, mu)
    np.testing.assert_array_equal(t, want[0])
    np.testing.assert_array_equal(x, want[1])
    np.testing.assert_array_equal(v, want[2])
    np.testing.assert_array_equal(rej, want[4].astype(np.float32))
    np.testing.assert_array_equal(steps, (max_steps - want[4]).astype(np.float32))


def test_full_config2_safe_states_and_counts_exact():
    """Config 2 at its full size (N = 262,144, mu log-uniform in [0.1, 100]):
    final states and accepted/rejected counts equal the oracle's exactly."""
    n = BS3_CFG.n
    x0, v0, mu = bs3_inputs(n, seed=BS3_CFG.seed)
    got = bs3_vdp_call(n, math_mode=pa.MathMode.SAFE)(x0, v0, mu)
    want = oracle.bs3_vdp(x0, v0, mu, BS3_CFG)
    for g, w, name in zip(got, want, ["t", "x", "v", "accepted", "rejected"]):
        np.testing.assert_array_equal(g, w, err_msg=name)
    assert got[3].sum() > 2e8  # the full workload ran: ~2.5e8 accepted steps
