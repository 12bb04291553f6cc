"""float64 NumPy references (test infrastructure only).

`lv_rk4_f64` restates examples/05_df32_precision.py:95-109: RK4 on the
reference rhs with every operand promoted to float64. `bs3_vdp_f64` is the
adaptive BS3(2)+PI Van der Pol loop of tests/test_08_adaptive.py:76-122 in
Python floats.
"""

from __future__ import annotations

import numpy as np


def lv_rk4_f64(x0, y0, a, b, c, d, dt: float, steps: int, consts=None):
    """`consts` = (half, full, sixth) replaces (dt/2, dt, dt/6), e.g. with
    the float32-rounded step constants a float32 kernel actually uses."""
    half, full, sixth = consts if consts is not None else (0.5 * dt, dt, dt / 6.0)
    x, y = x0.astype(np.float64), y0.astype(np.float64)
    a, b, c, d = (v.astype(np.float64) for v in (a, b, c, d))

    def rhs(x, y):
        return a * x - b * x * y, c * x * y - d * y

    for _ in range(steps):
        k1x, k1y = rhs(x, y)
        k2x, k2y = rhs(x + half * k1x, y + half * k1y)
        k3x, k3y = rhs(x + half * k2x, y + half * k2y)
        k4x, k4y = rhs(x + full * k3x, y + full * k3y)
        x = x + sixth * (k1x + 2 * k2x + 2 * k3x + k4x)
        y = y + sixth * (k1y + 2 * k2y + 2 * k3y + k4y)
    return x, y


def bs3_vdp_f64(x0, v0, mu, cfg):
    """Independent float64 BS3(2)+PI restatement (tests/test_08_adaptive.py:76-122),
    one trajectory at a time in Python floats: (t, x, v, accepted, rejected)."""
    out = []
    c1 = (cfg.icoeff + cfg.pcoeff) / 3
    c2 = -cfg.pcoeff / 3
    for x, v, m in zip(x0.astype(float), v0.astype(float), mu.astype(float)):
        f = lambda x, v: (v, m * (1 - x * x) * v - x)  # noqa: E731
        t, dt, prev = 0.0, cfg.dt0, 1.0
        k1 = f(x, v)
        acc = rej = 0
        while t < cfg.t1:
            dt = min(dt, cfg.t1 - t)
            k2 = f(x + 0.5 * dt * k1[0], v + 0.5 * dt * k1[1])
            k3 = f(x + 0.75 * dt * k2[0], v + 0.75 * dt * k2[1])
            y3 = [s + dt * (2 / 9 * a + 1 / 3 * b + 4 / 9 * c) for s, a, b, c in zip((x, v), k1, k2, k3)]
            k4 = f(*y3)
            y2 = [s + dt * (7 / 24 * a + 1 / 4 * b + 1 / 3 * c + 1 / 8 * d) for s, a, b, c, d in zip((x, v), k1, k2, k3, k4)]
            err = max(abs(y3[i] - y2[i]) / (cfg.atol + cfg.rtol * abs(y3[i])) for i in range(2))
            accept = err <= 1.0
            if accept:
                t, x, v, k1 = t + dt, y3[0], y3[1], k4
                acc += 1
            else:
                rej += 1
            err = max(err, 1e-9)
            inv = 1 / err
            factor = 0.9 * inv**c1 * prev**c2
            if accept:
                prev = inv
            dt = dt * min(10.0, max(0.2, factor))
        out.append((t, x, v, acc, rej))
    return [np.array(c) for c in zip(*out)]
