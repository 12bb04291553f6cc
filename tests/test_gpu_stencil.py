"""The temporal-blocking Gray-Scott passes (palladium_amd/stencil.py) on the
GPU, both the LDS-tiled one and the register one: under SAFE the fields
after any number of steps equal the C oracle's and the emitted per-step
kernel's bit for bit (halo cells are recomputed, not approximated); under
FAST they stay within the per-step kernel's tolerance of the oracle."""

import numpy as np
import pytest

import oracle
from palladium_amd import stencil
from palladium_amd.workloads import GS_CFG, gray_scott_call, gray_scott_initial, gray_scott_run

pytestmark = pytest.mark.gpu

KINDS = {
    "lds": lambda n, **kw: stencil.FusedGrayScott(n, **kw),
    "regs": lambda n, **kw: stencil.RegisterGrayScott(n, **kw),
    "regs4": lambda n, **kw: stencil.RegisterGrayScott(n, k=4, rows=32, group=2, cols=4, **kw),
}


@pytest.mark.parametrize("k,th,tw,single", [(4, 32, 64, True), (2, 16, 64, False), (3, 16, 32, True)])
@pytest.mark.parametrize("steps", [12, 13])
def test_lds_safe_bit_exact_against_oracle(k, th, tw, single, steps):
    n = 256
    print(f"[stencil] lds safe k={k} tile={th}x{tw} single={single} steps={steps}", flush=True)
    u0, v0 = gray_scott_initial(n)
    f = stencil.FusedGrayScott(n, k, th, tw, math_mode="safe", single_buffer=single)
    u, v, _ = stencil.gray_scott_fused_run(f, u0, v0, steps)
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, steps)
    np.testing.assert_array_equal(u, wu)
    np.testing.assert_array_equal(v, wv)


_REGS_CASES = [(256, 6, 64, 4, 1), (256, 4, 40, 8, 1), (256, 8, 27, 3, 1), (192, 1, 64, 8, 1), (80, 3, 22, 5, 1),
               (64, 12, 16, 8, 1),
               # two and four columns per lane: 64-/128-bit rows (K, n multiples of the columns)
               # and 32-bit ones (odd K), strips that divide the grid and ragged ones
               (256, 6, 64, 4, 2), (192, 4, 40, 8, 2), (160, 3, 27, 3, 2), (128, 1, 64, 8, 2), (256, 8, 30, 2, 4)]


@pytest.mark.parametrize("n,k,rows,group,cols", _REGS_CASES)
@pytest.mark.parametrize("steps", [12, 13])
def test_regs_safe_bit_exact_against_oracle(n, k, rows, group, cols, steps):
    """Strips that divide the grid and strips that do not (the last strip of
    a column or row reaches past the grid), K from 1 to 12, one, two and
    four columns per lane."""
    print(f"[stencil] regs safe n={n} k={k} rows={rows} group={group} steps={steps} cols={cols}", flush=True)
    u0, v0 = gray_scott_initial(n)
    f = stencil.RegisterGrayScott(n, k, rows, group, math_mode="safe", cols=cols)
    u, v, _ = stencil.gray_scott_fused_run(f, u0, v0, steps)
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, steps)
    np.testing.assert_array_equal(u, wu)
    np.testing.assert_array_equal(v, wv)


@pytest.mark.parametrize("kind", sorted(KINDS))
def test_full_config4_safe_equals_the_per_step_kernel(kind):
    """Config 4 at full size, 2,000 steps: bit for bit the emitted per-step
    kernel's fields, which equal the oracle's
    (tests/test_gpu_gray_scott.py::test_full_config4_safe_bit_exact)."""
    n, steps = GS_CFG.size, GS_CFG.steps
    print(f"[stencil] {kind} full config 4 safe", flush=True)
    u0, v0 = gray_scott_initial(n)
    fu, fv, _ = stencil.gray_scott_fused_run(KINDS[kind](n, math_mode="safe"), u0, v0, steps)
    pu, pv, _ = gray_scott_run(gray_scott_call(size=n, math_mode="safe"), u0, v0, steps)
    np.testing.assert_array_equal(fu, pu)
    np.testing.assert_array_equal(fv, pv)
    assert float(np.abs(fv).sum()) > 1.0


@pytest.mark.parametrize("kind", sorted(KINDS))
def test_fast_close_to_oracle(kind):
    n, steps = 256, 200
    u0, v0 = gray_scott_initial(n)
    u, v, _ = stencil.gray_scott_fused_run(KINDS[kind](n), u0, v0, steps)
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, steps)
    np.testing.assert_allclose(u, wu, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(v, wv, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("kind", sorted(KINDS))
def test_uniform_state_is_a_fixed_point(kind):
    n = 256
    u0 = np.ones((n, n), np.float32)
    v0 = np.zeros((n, n), np.float32)
    u, v, _ = stencil.gray_scott_fused_run(KINDS[kind](n), u0, v0, 20)
    np.testing.assert_array_equal(u, u0)
    np.testing.assert_array_equal(v, v0)
