"""The hot-path kernels, authored as ordinary Pallas kernels.

These are the five workloads the backend is measured on. Each is written
against `palladium_amd.frontend` exactly as a user would write it for the
reference (the same jnp/lax calls, hence the same staged op order), and
runs through `hip_call` like any other kernel:

- `lv_rk4`: RK4 Lotka-Volterra ensemble, one trajectory per program
  instance (`examples/01_ode_ensembles.py:72-103`,
  `tests/test_06_capstone_rk4.py:20-53`), optionally carrying the running
  max |y|.
- `bs3_vdp`: adaptive Bogacki-Shampine 3(2) with a PI controller on a Van
  der Pol ensemble, one `while_loop` per instance
  (`tests/test_08_adaptive.py:33-142` restated with a data-dependent loop).
- `gbm`: geometric Brownian motion Monte Carlo with in-kernel Threefry
  bits and Box-Muller normals (`examples/03_sde_montecarlo.py:97-119`).
- `gray_scott`: one explicit Euler step of Gray-Scott reaction-diffusion
  with a periodic 5-point Laplacian through indexed refs
  (`examples/04_reaction_diffusion.py:61-74`).

Input generators reproduce the configurations the backend is benchmarked
on (seeded `numpy.random.default_rng`).
"""

from __future__ import annotations

import dataclasses
import math
from typing import Any

import numpy as np

from palladium_amd.frontend import jnp, lax, pl, random

F32 = np.float32

# ---------------------------------------------------------------------------
# RK4 Lotka-Volterra


def lv_rk4_kernel(dt: float, steps: int, track_max: bool = False):
    """Kernel: refs (x0, y0, a, b, c, d) -> (x, y[, max|y|]).

    rhs(x, y) = (a x - b x y, c x y - d y), classic RK4 with the stage
    constants folded by Python as in the reference (0.5*DT, DT, DT/6)."""

    def kernel(x_ref, y_ref, a_ref, b_ref, c_ref, d_ref, xo_ref, yo_ref, *rest):
        a, b, c, d = a_ref[...], b_ref[...], c_ref[...], d_ref[...]

        def rhs(x, y):
            return a * x - b * x * y, c * x * y - d * y

        def rk4(x, y):
            k1x, k1y = rhs(x, y)
            k2x, k2y = rhs(x + 0.5 * dt * k1x, y + 0.5 * dt * k1y)
            k3x, k3y = rhs(x + 0.5 * dt * k2x, y + 0.5 * dt * k2y)
            k4x, k4y = rhs(x + dt * k3x, y + dt * k3y)
            return (
                x + dt / 6.0 * (k1x + 2.0 * k2x + 2.0 * k3x + k4x),
                y + dt / 6.0 * (k1y + 2.0 * k2y + 2.0 * k3y + k4y),
            )

        x0, y0 = x_ref[...], y_ref[...]
        if track_max:
            def step(_, carry):
                x, y, m = carry
                x, y = rk4(x, y)
                return x, y, jnp.maximum(m, jnp.abs(y))

            x, y, m = lax.fori_loop(0, steps, step, (x0, y0, jnp.abs(y0)))
            rest[0][...] = m
        else:
            def step(_, carry):
                return rk4(*carry)

            x, y = lax.fori_loop(0, steps, step, (x0, y0))
        xo_ref[...] = x
        yo_ref[...] = y

    kernel.__name__ = "lv_rk4"
    return kernel


def lv_rk4_call(n: int, dt: float, steps: int, track_max: bool = False, block: int = 1, **kw: Any):
    """`hip_call` of the LV ensemble over `n` trajectories; `block`
    trajectories per program instance (1 = one lane each)."""
    import palladium_amd as pa

    if n % block:
        raise ValueError(f"n={n} is not a multiple of block={block}")
    spec = pl.BlockSpec((block,), lambda i: (i,))
    n_out = 3 if track_max else 2
    return pa.hip_call(
        lv_rk4_kernel(dt, steps, track_max),
        grid=(n // block,),
        in_specs=[spec] * 6,
        out_specs=tuple([spec] * n_out),
        out_shape=tuple(pl.ShapeDtypeStruct((n,), F32) for _ in range(n_out)),
        name="lv_rk4",
        **kw,
    )


def lv_inputs(n: int, seed: int) -> tuple[np.ndarray, ...]:
    """(x0, y0, a, b, c, d) for the benchmark configurations.

    Draw order alpha~U(0.5,1.5), beta~U(0.5,1.5), gamma~U(1,3),
    delta~U(0.5,1.5), x0~U(0.5,2), y0~U(0.5,2); mapped onto the reference
    rhs (a x - b x y, c x y - d y) as a=alpha, b=beta, c=delta, d=gamma
    (x' = alpha x - beta x y, y' = delta x y - gamma y)."""
    rng = np.random.default_rng(seed)
    alpha = rng.uniform(0.5, 1.5, n).astype(F32)
    beta = rng.uniform(0.5, 1.5, n).astype(F32)
    gamma = rng.uniform(1.0, 3.0, n).astype(F32)
    delta = rng.uniform(0.5, 1.5, n).astype(F32)
    x0 = rng.uniform(0.5, 2.0, n).astype(F32)
    y0 = rng.uniform(0.5, 2.0, n).astype(F32)
    return x0, y0, alpha, beta, delta, gamma


@dataclasses.dataclass(frozen=True)
class LVConfig:
    n: int
    dt: float
    steps: int
    seed: int


LV_CFG0 = LVConfig(100_000, 0.01, 1000, 0)
LV_CFG1 = LVConfig(1_000_000, 0.005, 4000, 1)

# Algorithmic floating-point work of one RK4 LV step: the 58 elementwise
# float ops of the staged step body (an FMA counts as two).
LV_FLOP_PER_STEP = 58
LV_BYTES_PER_TRAJ = 6 * 4 + 3 * 4
