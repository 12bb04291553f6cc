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


def _register_pass(u, v, k, rows, group, cfg, cols=1):
    """The register kernel's schedule, lane for lane: a wave's 64 lanes of
    `cols` columns each walk down their columns (up, in odd bands of
    strips), each step keeping two rows of the step before; a column's
    inner neighbours are its lane's own columns and the lane's outer ones
    come from the adjacent lanes rotated across the whole wave (np.roll),
    the windows start at zero, row and column indices wrap, and only owner
    columns and rows K .. K + rows - 1 of step K are stored."""
    du, dv, f, fk, dt = (F(x) for x in (cfg.du, cfg.dv, cfg.f, cfg.f + cfg.k, cfg.dt))
    n = u.shape[0]
    C = cols
    w = 64 * C - 2 * k
    h = rows + 2 * k
    total = -(-h // group) * group
    uo, vo = np.full_like(u, np.nan), np.full_like(v, np.nan)
    sc = np.arange(64 * C).reshape(64, C)          # strip column of lane l, column c
    for band, i0 in enumerate(range(0, n, rows)):
        up = band % 2 == 1  # odd bands walk up the grid
        for j0 in range(0, -(-n // w) * w, w):
            gj = (j0 - k + sc) % n
            owner = (sc >= k) & (sc < 64 * C - k) & (j0 + sc - k < n)
            win = [[np.zeros((64, C), F) for _ in range(4)] for _ in range(k)]  # pu2, pu1, pv2, pv1

            def neighbours(x):
                """(right, left) of every column of (64, C) values x."""
                right, left = np.empty_like(x), np.empty_like(x)
                right[:, :-1], left[:, 1:] = x[:, 1:], x[:, :-1]
                right[:, -1] = np.roll(x[:, 0], -1)
                left[:, 0] = np.roll(x[:, -1], 1)
                return right, left

            for r in range(total):
                p = min(r, h - 1)  # past the strip's end: its last row again
                gi = (i0 + rows - 1 + k - p) % n if up else (i0 - k + p) % n
                cu, cv = u[gi, gj], v[gi, gj]
                for t in range(k):
                    pu2, pu1, pv2, pv1 = win[t]
                    with np.errstate(all="ignore"):
                        ru, lu_ = neighbours(pu1)
                        rv, lv_ = neighbours(pv1)
                        lu = cu + pu2
                        lu = lu + ru
                        lu = lu + lu_
                        lu = lu - F(4.0) * pu1
                        lv = cv + pv2
                        lv = lv + rv
                        lv = lv + lv_
                        lv = lv - F(4.0) * pv1
                        uvv = (pu1 * pv1) * pv1
                        a = du * lu
                        a = a - uvv
                        a = a + f * (F(1.0) - pu1)
                        b = dv * lv
                        b = b + uvv
                        b = b - fk * pv1
                        yu, yv = pu1 + dt * a, pv1 + dt * b
                    win[t] = [pu1, cu, pv1, cv]
                    cu, cv = yu, yv
                a_row = r - 2 * k
                ga = i0 + rows - 1 - a_row if up else i0 + a_row
                if 0 <= a_row < rows and ga < n:
                    cols_g = j0 + sc[owner] - k
                    assert np.all(np.isnan(uo[ga, cols_g])), "a cell stored twice"
                    uo[ga, cols_g] = cu[owner]
                    vo[ga, cols_g] = cv[owner]
    assert not np.isnan(uo).any() and not np.isnan(vo).any(), "a cell never stored"
    return uo, vo


@pytest.mark.parametrize("n,k,rows,group,steps", [(64, 4, 16, 8, 8), (64, 4, 16, 8, 9), (64, 3, 32, 5, 6),
                                                   (64, 8, 16, 8, 16), (124, 1, 62, 4, 3), (96, 4, 20, 8, 8),
                                                   (80, 6, 27, 8, 12), (80, 3, 22, 5, 7)])
def test_register_schedule_restated_matches_oracle(n, k, rows, group, steps):
    u0, v0 = gray_scott_initial(n)
    u, v = u0.copy(), v0.copy()
    for kk in [k] * (steps // k) + [1] * (steps % k):
        u, v = _register_pass(u, v, kk, rows, group, GS_CFG)
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, steps)
    np.testing.assert_array_equal(u, wu)
    np.testing.assert_array_equal(v, wv)


@pytest.mark.parametrize("n,k,rows,group,steps,cols", [(128, 4, 24, 4, 9, 2), (160, 6, 32, 4, 13, 2),
                                                        (256, 3, 40, 2, 7, 4), (128, 1, 64, 8, 2, 2)])
def test_register_schedule_with_several_columns_per_lane(n, k, rows, group, steps, cols):
    u0, v0 = gray_scott_initial(n)
    u, v = u0.copy(), v0.copy()
    for kk in [k] * (steps // k) + [1] * (steps % k):
        u, v = _register_pass(u, v, kk, rows, group, GS_CFG, cols)
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, steps)
    np.testing.assert_array_equal(u, wu)
    np.testing.assert_array_equal(v, wv)


@pytest.mark.parametrize("k,rows", [(4, 64), (8, 64)])
def test_register_source_compiles_without_lds_or_spills(k, rows):
    src = stencil.register_source(4096, k, rows, 0.16, 0.08, 0.037, 0.097, 1.0)
    from palladium_amd.diagnostics import code_object_resources

    res = code_object_resources(rt.compile_code_object(src, "gray_scott_regs", "fast"), "gray_scott_regs")
    assert res.lds_bytes == 0 and res.vgpr_spills == 0 and res.scratch_bytes == 0
    assert res.vgprs <= 128


def test_register_bad_shapes_are_refused():
    with pytest.raises(ValueError, match="positive"):
        stencil.register_source(4096, 4, 0, 0.16, 0.08, 0.037, 0.097, 1.0)
    with pytest.raises(ValueError, match="out of range"):
        stencil.register_source(4096, 32, 64, 0.16, 0.08, 0.037, 0.097, 1.0)
    with pytest.raises(ValueError, match="too small"):
        stencil.register_source(32, 2, 16, 0.16, 0.08, 0.037, 0.097, 1.0)
    with pytest.raises(ValueError, match="too small"):
        stencil.register_source(96, 2, 16, 0.16, 0.08, 0.037, 0.097, 1.0, cols=2)


def test_runner_checks_its_arguments_before_touching_a_device():
    f = stencil.FusedGrayScott.__new__(stencil.FusedGrayScott)
    f.n = 64
    u0 = np.ones((64, 64), np.float32)
    with pytest.raises(ValueError, match="64x64"):
        stencil.gray_scott_fused_run(f, u0[:32], u0, 4)
    with pytest.raises(ValueError, match="non-negative"):
        stencil.gray_scott_fused_run(f, u0, u0, -1)
    u, v, t = stencil.gray_scott_fused_run(f, u0, 2 * u0, 0)
    assert t == 0.0 and np.array_equal(u, u0) and np.array_equal(v, 2 * u0) and u is not u0
