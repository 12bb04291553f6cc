"""float64 NumPy references (test infrastructure only).

`lv_rk4_f64` restates examples/05_df32_precision.py:95-109: RK4 on the
reference rhs with every operand promoted to float64.
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
