"""The oracle's pins can fail: plausible mistakes move results far beyond
the tolerances the pin tests use (the reference's doctrine of sabotaging a
rule to prove its test can fail, `docs/extending.md:53-69`).

Each mutant is the float64 restatement with one mistake of the kind a
restatement could make (a dropped term, a wrong sign, transposed operands,
a wrong weight or coefficient, a wrong stencil index). If the C oracle
carried that mistake it would track the mutant, and its pin test
(tests/test_oracle.py, same inputs and tolerance) would fail; so every
mutant must sit outside that tolerance of the oracle.
"""

import numpy as np
import pytest

import oracle
from palladium_amd.workloads import GS_CFG, BS3Config, bs3_inputs, gray_scott_initial, lv_inputs

# ---------------------------------------------------------------------------
# RK4 Lotka-Volterra: pin = max relative error < 1e-4 against float64 RK4.

LV_TOL = 1e-4


def _lv_mutant(x0, y0, a, b, c, d, dt, steps, mutation):
    x, y = x0.astype(np.float64), y0.astype(np.float64)
    a, b, c, d = (v.astype(np.float64) for v in (a, b, c, d))

    def rhs(x, y):
        fx = a * x - b * x * y
        fy = c * x * y - d * y
        if mutation == "drop_bxy":
            fx = a * x
        elif mutation == "sign_bxy":
            fx = a * x + b * x * y
        elif mutation == "swap_cd":
            fy = d * x * y - c * y
        elif mutation == "transpose_dy":
            fy = c * x * y - d * x
        return fx, fy

    w2 = 1.0 if mutation == "weight_k2" else 2.0
    h2 = dt if mutation == "stage_full_dt" else 0.5 * dt
    for _ in range(steps):
        k1 = rhs(x, y)
        k2 = rhs(x + h2 * k1[0], y + h2 * k1[1])
        k3 = rhs(x + h2 * k2[0], y + h2 * k2[1])
        k4 = rhs(x + dt * k3[0], y + dt * k3[1])
        x = x + dt / 6.0 * (k1[0] + w2 * k2[0] + 2 * k3[0] + k4[0])
        y = y + dt / 6.0 * (k1[1] + w2 * k2[1] + 2 * k3[1] + k4[1])
    return x, y


@pytest.mark.parametrize("mutation", ["drop_bxy", "sign_bxy", "swap_cd", "transpose_dy", "weight_k2", "stage_full_dt"])
def test_lv_pin_detects(mutation):
    args = lv_inputs(2000, 0)
    x, y = oracle.lv_rk4(*args, 0.01, 1000)
    with np.errstate(all="ignore"):  # some mutants blow up; that counts as detected
        mx, my = _lv_mutant(*args, 0.01, 1000, mutation)
        rel = max(np.max(np.abs(x - mx) / np.abs(mx)), np.max(np.abs(y - my) / np.abs(my)))
    assert not rel < 10 * LV_TOL  # NaN/inf from a blown-up mutant also counts as detected


# ---------------------------------------------------------------------------
# Gray-Scott: pin = max absolute error < 1e-5 against the float64 np.roll form.

GS_TOL = 1e-5


def _gs_mutant(u, v, cfg, steps, mutation):
    u, v = u.astype(np.float64), v.astype(np.float64)

    def lap(z):
        n, s, e, w = np.roll(z, 1, 0), np.roll(z, -1, 0), np.roll(z, 1, 1), np.roll(z, -1, 1)
        if mutation == "neighbour_twice":
            s = n
        if mutation == "no_centre":
            return n + s + e + w
        return n + s + e + w - 4.0 * z

    du, dv = (cfg.dv, cfg.du) if mutation == "swap_diffusion" else (cfg.du, cfg.dv)
    for _ in range(steps):
        uvv = u * v * v
        feed = cfg.f * u if mutation == "feed_sign" else cfg.f * (1.0 - u)
        react = -uvv if mutation == "reaction_sign" else uvv
        u, v = (u + cfg.dt * (du * lap(u) - react + feed),
                v + cfg.dt * (dv * lap(v) + react - (cfg.f + cfg.k) * v))
    return u, v


@pytest.mark.parametrize("mutation", ["neighbour_twice", "no_centre", "swap_diffusion", "feed_sign", "reaction_sign"])
def test_gray_scott_pin_detects(mutation):
    u0, v0 = gray_scott_initial(64)
    u, v = oracle.gray_scott(u0, v0, GS_CFG, 50)
    with np.errstate(all="ignore"):
        mu, mv = _gs_mutant(u0, v0, GS_CFG, 50, mutation)
    with np.errstate(all="ignore"):
        d = max(np.max(np.abs(u - mu)), np.max(np.abs(v - mv)))
    assert not d <= 10 * GS_TOL  # NaN from a blown-up mutant also counts as detected


# ---------------------------------------------------------------------------
# BS3(2)+PI: pin = final x within rtol/atol 2e-3 and accepted counts within
# 5 % / 5 of the float64 restatement.


def _bs3_mutant(x0, v0, mu, cfg, mutation):
    out = []
    c1 = (cfg.icoeff + cfg.pcoeff) / 3
    c2 = (+1 if mutation == "controller_sign" else -1) * cfg.pcoeff / 3
    cs = (0.5, 0.5) if mutation == "node_c3" else (0.5, 0.75)
    b3 = (1 / 4, 1 / 3, 5 / 12) if mutation == "weights_b3" else (2 / 9, 1 / 3, 4 / 9)
    for x, v, m in zip(x0.astype(float), v0.astype(float), mu.astype(float)):
        f = lambda x, v: (v, m * (1 - x * x) * v - x)  # noqa: E731
        t, dt, prev = 0.0, cfg.dt0, 1.0
        k1 = f(x, v)
        acc = attempts = 0
        while t < cfg.t1 and attempts < 20_000:
            attempts += 1
            dt = min(dt, cfg.t1 - t)
            k2 = f(x + cs[0] * dt * k1[0], v + cs[0] * dt * k1[1])
            k3 = f(x + cs[1] * dt * k2[0], v + cs[1] * dt * k2[1])
            y3 = [s + dt * (b3[0] * a + b3[1] * b + b3[2] * c) for s, a, b, c in zip((x, v), k1, k2, k3)]
            k4 = f(*y3)
            y2 = [s + dt * (7 / 24 * a + 1 / 4 * b + 1 / 3 * c + 1 / 8 * d) for s, a, b, c, d in zip((x, v), k1, k2, k3, k4)]
            scale = y2 if mutation == "norm_scale_y2" else y3
            terms = [abs(y3[i] - y2[i]) / (cfg.atol + cfg.rtol * abs(scale[i])) for i in range(2)]
            err = sum(terms) if mutation == "norm_sum" else max(terms)
            accept = err <= 1.0
            if accept:
                t, x, v, k1 = t + dt, y3[0], y3[1], k4
                acc += 1
            err = max(err, 1e-9)
            inv = 1 / err
            factor = 0.9 * inv**c1 * prev**c2
            if accept:
                prev = inv
            dt = dt * min(10.0, max(0.2, factor))
        out.append((x, acc))
    return [np.array(c) for c in zip(*out)]


@pytest.mark.parametrize("mutation", ["controller_sign", "node_c3", "weights_b3"])
def test_bs3_pin_detects(mutation):
    x0, v0, mu = (a[:12] for a in bs3_inputs(48, seed=11))
    mu = np.minimum(mu, np.float32(5.0))
    cfg = BS3Config()
    _, x, _, acc, _ = oracle.bs3_vdp(x0, v0, mu, cfg)
    mx, macc = _bs3_mutant(x0, v0, mu, cfg, mutation)
    x_off = np.any(np.abs(x - mx) > 2e-3 + 2e-3 * np.abs(mx))
    acc_off = np.any(np.abs(acc - macc) > 5 + 0.05 * np.abs(macc))
    assert x_off or acc_off


# The stiff pin (tests/test_oracle.py: 12 trajectories with mu in [50, 100],
# final x within 2e-5 relative, accepted counts within 3 % / 3) catches the
# same mistakes on the stiff trajectories. Two mistakes stay below every pin
# and are listed so that stays visible: scaling the norm by |y2| instead of
# |y3| (the two agree to rtol, so it is the same method to 1e-5), and summing
# the two components instead of taking the larger (it shifts accepted counts
# by under 1 %, inside the float32-vs-float64 spread of correct code).
UNDETECTED_BY_FINAL_STATE = ("norm_scale_y2", "norm_sum")


@pytest.mark.parametrize("mutation", ["controller_sign", "node_c3", "weights_b3"])
def test_bs3_stiff_pin_detects(mutation):
    x0, v0, mu = bs3_inputs(4096, seed=11)
    sel = np.where(mu >= 50)[0][:12]
    x0, v0, mu = x0[sel], v0[sel], mu[sel]
    cfg = BS3Config()
    _, x, _, acc, _ = oracle.bs3_vdp(x0, v0, mu, cfg)
    mx, macc = _bs3_mutant(x0, v0, mu, cfg, mutation)
    x_off = np.any(np.abs(x - mx) > 2e-5 * np.abs(mx))
    acc_off = np.any(np.abs(acc - macc) > 3 + 0.03 * np.abs(macc))
    assert x_off or acc_off
