"""float64 NumPy references (test infrastructure only).

`lv_rk4_f64` restates examples/05_df32_precision.py:95-109: RK4 on the
reference rhs with every operand promoted to float64.
"""

from __future__ import annotations

import numpy as np


def lv_rk4_f64(x0, y0, a, b, c, d, dt: float, steps: int):
    x, y = x0.astype(np.float64), y0.astype(np.float64)
    a, b, c, d = (v.astype(np.float64) for v in (a, b, c, d))

    def rhs(x, y):
        return a * x - b * x * y, c * x * y - d * y

    for _ in range(steps):
        k1x, k1y = rhs(x, y)
        k2x, k2y = rhs(x + 0.5 * dt * k1x, y + 0.5 * dt * k1y)
        k3x, k3y = rhs(x + 0.5 * dt * k2x, y + 0.5 * dt * k2y)
        k4x, k4y = rhs(x + dt * k3x, y + dt * k3y)
        x = x + dt / 6.0 * (k1x + 2 * k2x + 2 * k3x + k4x)
        y = y + dt / 6.0 * (k1y + 2 * k2y + 2 * k3y + k4y)
    return x, y
