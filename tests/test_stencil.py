"""The temporal-blocking Gray-Scott pass (palladium_amd/stencil.py) on the
CPU: its tiling (tile + K-cell periodic halo, K updates on a region that
shrinks by one cell per side, the tile written back) restated in NumPy
float32 with the kernel's op order, against the C oracle bit for bit; and
the generated source's shape. The GPU runs of the kernel itself are in
tests/test_gpu_stencil.py."""

import numpy as np
import pytest

import oracle
from palladium_amd import runtime as rt
from palladium_amd import stencil
from palladium_amd.workloads import GS_CFG, gray_scott_initial

F = np.float32


def _update(u, v, cfg):
    """One step on the interior of (u, v) (arrays with a one-cell border),
    in the oracle's op order."""
    du, dv, f, fk, dt = (F(x) for x in (cfg.du, cfg.dv, cfg.f, cfg.f + cfg.k, cfg.dt))
    uc, vc = u[1:-1, 1:-1], v[1:-1, 1:-1]
    lu = u[2:, 1:-1] + u[:-2, 1:-1]
    lu = lu + u[1:-1, 2:]
    lu = lu + u[1:-1, :-2]
    lu = lu - F(4.0) * uc
    lv = v[2:, 1:-1] + v[:-2, 1:-1]
    lv = lv + v[1:-1, 2:]
    lv = lv + v[1:-1, :-2]
    lv = lv - F(4.0) * vc
    uvv = (uc * vc) * vc
    a = du * lu
    a = a - uvv
    a = a + f * (F(1.0) - uc)
    b = dv * lv
    b = b + uvv
    b = b - fk * vc
    return uc + dt * a, vc + dt * b


def _fused_pass(u, v, k, th, tw, cfg):
    n = u.shape[0]
    uo, vo = np.empty_like(u), np.empty_like(v)
    for i0 in range(0, n, th):
        for j0 in range(0, n, tw):
            rows = np.arange(i0 - k, i0 + th + k) % n
            cols = np.arange(j0 - k, j0 + tw + k) % n
            tu, tv = u[np.ix_(rows, cols)], v[np.ix_(rows, cols)]
            for _ in range(k):   # the region shrinks by one cell per side
                tu, tv = _update(tu, tv, cfg)
            uo[i0:i0 + th, j0:j0 + tw] = tu
            vo[i0:i0 + th, j0:j0 + tw] = tv
    return uo, vo


@pytest.mark.parametrize("k,th,tw,steps", [(4, 16, 32, 8), (4, 16, 32, 9), (2, 8, 16, 6), (3, 16, 16, 7)])
def test_tiling_restated_matches_oracle(k, th, tw, steps):
    n = 64
    u0, v0 = gray_scott_initial(n)
    u, v = u0.copy(), v0.copy()
    for kk in [k] * (steps // k) + [1] * (steps % k):
        u, v = _fused_pass(u, v, kk, th, tw, GS_CFG)
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, steps)
    np.testing.assert_array_equal(u, wu)
    np.testing.assert_array_equal(v, wv)


def test_launch_plan_covers_every_step():
    f = stencil.FusedGrayScott.__new__(stencil.FusedGrayScott)
    f.k = 4
    assert f.launches(2000) == [4] * 500
    assert f.launches(7) == [4, 1, 1, 1]


@pytest.mark.parametrize("single", [True, False])
def test_source_compiles_with_its_lds_budget(single):
    src = stencil.fused_source(4096, 4, 32, 64, 0.16, 0.08, 0.037, 0.097, 1.0, single_buffer=single)
    from palladium_amd.diagnostics import code_object_resources

    res = code_object_resources(rt.compile_code_object(src, "gray_scott_fused", "fast"), "gray_scott_fused")
    assert res.lds_bytes == (1 if single else 2) * 2 * 40 * 72 * 4
    assert res.vgpr_spills == 0 and res.scratch_bytes == 0


def test_bad_tiles_are_refused():
    with pytest.raises(ValueError, match="must divide"):
        stencil.fused_source(100, 2, 32, 64, 0.16, 0.08, 0.037, 0.097, 1.0)
    with pytest.raises(ValueError, match="out of range"):
        stencil.fused_source(4096, 9, 16, 64, 0.16, 0.08, 0.037, 0.097, 1.0)
