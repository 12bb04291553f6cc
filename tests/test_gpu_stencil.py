"""The temporal-blocking Gray-Scott pass (palladium_amd/stencil.py) on the
GPU: under SAFE the fields after any number of steps equal the C oracle's
and the emitted per-step kernel's bit for bit (halo cells are recomputed,
not approximated); under FAST it stays within the per-step kernel's
tolerance of the oracle."""

import numpy as np
import pytest

import oracle
from palladium_amd import stencil
from palladium_amd.workloads import GS_CFG, gray_scott_call, gray_scott_initial, gray_scott_run

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("k,th,tw,single", [(4, 32, 64, True), (2, 16, 64, False), (3, 16, 32, True)])
@pytest.mark.parametrize("steps", [12, 13])
def test_safe_bit_exact_against_oracle(k, th, tw, single, steps):
    n = 256
    print(f"[stencil] safe k={k} tile={th}x{tw} single={single} steps={steps}", flush=True)
    u0, v0 = gray_scott_initial(n)
    f = stencil.FusedGrayScott(n, k, th, tw, math_mode="safe", single_buffer=single)
    u, v, _ = stencil.gray_scott_fused_run(f, u0, v0, steps)
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, steps)
    np.testing.assert_array_equal(u, wu)
    np.testing.assert_array_equal(v, wv)


def test_full_config4_safe_equals_the_per_step_kernel():
    """Config 4 at full size, 2,000 steps (500 passes of 4): bit for bit
    the emitted per-step kernel's fields, which equal the oracle's
    (tests/test_gpu_gray_scott.py::test_full_config4_safe_bit_exact)."""
    n, steps = GS_CFG.size, GS_CFG.steps
    u0, v0 = gray_scott_initial(n)
    fu, fv, _ = stencil.gray_scott_fused_run(stencil.FusedGrayScott(n, math_mode="safe"), u0, v0, steps)
    pu, pv, _ = gray_scott_run(gray_scott_call(size=n, math_mode="safe"), u0, v0, steps)
    np.testing.assert_array_equal(fu, pu)
    np.testing.assert_array_equal(fv, pv)
    assert float(np.abs(fv).sum()) > 1.0


def test_fast_close_to_oracle():
    n, steps = 256, 200
    u0, v0 = gray_scott_initial(n)
    u, v, _ = stencil.gray_scott_fused_run(stencil.FusedGrayScott(n), u0, v0, steps)
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, steps)
    np.testing.assert_allclose(u, wu, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(v, wv, rtol=1e-4, atol=1e-5)


def test_uniform_state_is_a_fixed_point():
    n = 256
    u0 = np.ones((n, n), np.float32)
    v0 = np.zeros((n, n), np.float32)
    u, v, _ = stencil.gray_scott_fused_run(stencil.FusedGrayScott(n), u0, v0, 20)
    np.testing.assert_array_equal(u, u0)
    np.testing.assert_array_equal(v, v0)
