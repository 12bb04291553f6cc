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


def lv_rk4_call(n: int, dt: float, steps: int, track_max: bool = False, block: int = 1, name: str = "lv_rk4",
                **kw: Any):
    """`hip_call` of the LV ensemble over `n` trajectories; `block`
    trajectories per program instance (1 = one lane each). The grid is
    ceil(n / block), as config 0 states it (N = 100,000 in blocks of 256):
    a ragged last block is lowered lane-parallel with its tail masked."""
    import palladium_amd as pa

    spec = pl.BlockSpec((block,), lambda i: (i,))
    n_out = 3 if track_max else 2
    return pa.hip_call(
        lv_rk4_kernel(dt, steps, track_max),
        grid=(-(-n // block),),
        in_specs=[spec] * 6,
        out_specs=tuple([spec] * n_out),
        out_shape=tuple(pl.ShapeDtypeStruct((n,), F32) for _ in range(n_out)),
        name=name,
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


# ---------------------------------------------------------------------------
# Adaptive Bogacki-Shampine 3(2) + PI controller, Van der Pol


@dataclasses.dataclass(frozen=True)
class BS3Config:
    n: int = 262_144
    t1: float = 20.0
    dt0: float = 0.01
    rtol: float = 1e-5
    atol: float = 1e-8
    pcoeff: float = 0.4
    icoeff: float = 0.3
    max_attempts: int = 2_000_000
    seed: int = 2


BS3_CFG = BS3Config()


def _bs3_attempt(cfg: BS3Config, mu: Any, t: Any, dt: Any, x: Any, v: Any, k1x: Any, k1v: Any,
                 prev_inv_err: Any) -> tuple:
    """One BS3(2)+FSAL+PI attempt (`tests/test_08_adaptive.py:76-122`):
    returns (accept, t, dt, x, v, k1x, k1v, prev_inv_err) after it. The
    step clamps to T1 first, so a lane at T1 attempts a zero step, which
    is accepted and changes nothing."""
    t1, rtol, atol = cfg.t1, cfg.rtol, cfg.atol
    error_order = 3
    coeff1 = (cfg.icoeff + cfg.pcoeff) / error_order
    coeff2 = -cfg.pcoeff / error_order
    safety, factormin, factormax = 0.9, 0.2, 10.0

    def rhs(x, v):
        return v, mu * (1.0 - x**2) * v - x

    dt = jnp.minimum(dt, t1 - t)
    k2x, k2v = rhs(x + 0.5 * dt * k1x, v + 0.5 * dt * k1v)
    k3x, k3v = rhs(x + 0.75 * dt * k2x, v + 0.75 * dt * k2v)
    y3 = (
        x + dt * (2 / 9 * k1x + 1 / 3 * k2x + 4 / 9 * k3x),
        v + dt * (2 / 9 * k1v + 1 / 3 * k2v + 4 / 9 * k3v),
    )
    k4x, k4v = rhs(*y3)
    y2 = (
        x + dt * (7 / 24 * k1x + 1 / 4 * k2x + 1 / 3 * k3x + 1 / 8 * k4x),
        v + dt * (7 / 24 * k1v + 1 / 4 * k2v + 1 / 3 * k3v + 1 / 8 * k4v),
    )
    err_x, err_v = y3[0] - y2[0], y3[1] - y2[1]
    x3, v3 = y3
    err_norm = jnp.maximum(
        jnp.abs(err_x) / (atol + rtol * jnp.abs(x3)),
        jnp.abs(err_v) / (atol + rtol * jnp.abs(v3)),
    )
    accept = err_norm <= 1.0
    t2 = jnp.where(accept, t + dt, t)
    x2 = jnp.where(accept, y3[0], x)
    v2 = jnp.where(accept, y3[1], v)
    nk1x = jnp.where(accept, k4x, k1x)
    nk1v = jnp.where(accept, k4v, k1v)
    err_norm = jnp.maximum(err_norm, 1e-9)
    inv_err = 1 / err_norm
    factor = safety * inv_err**coeff1 * prev_inv_err**coeff2
    prev_inv_err = jnp.where(accept, inv_err, prev_inv_err)
    dt = dt * jnp.clip(factor, factormin, factormax)
    return accept, t2, dt, x2, v2, nk1x, nk1v, prev_inv_err


def _bs3_rhs(mu: Any, x: Any, v: Any) -> tuple:
    return v, mu * (1.0 - x**2) * v - x


def bs3_vdp_kernel(cfg: BS3Config):
    """Kernel: refs (x0, v0, mu) -> (t, x, v, accepted, rejected).

    The reference's adaptive step inside a `while_loop` that runs until t
    reaches T1 (bounded by `max_attempts`), so each lane takes exactly the
    attempts it needs; accepted/rejected are int32 counts of real
    attempts."""

    def kernel(x0_ref, v0_ref, mu_ref, to_ref, xo_ref, vo_ref, acc_ref, rej_ref):
        mu = mu_ref[...]

        def cond(c):
            t, it = c[0], c[9]
            return jnp.logical_and(t < cfg.t1, it < cfg.max_attempts)

        def body(c):
            t, dt, x, v, k1x, k1v, prev_inv_err, acc, rej, it = c
            accept, t, dt, x, v, k1x, k1v, prev_inv_err = _bs3_attempt(cfg, mu, t, dt, x, v, k1x, k1v, prev_inv_err)
            acc = acc + jnp.where(accept, 1, 0)
            rej = rej + jnp.where(accept, 0, 1)
            return (t, dt, x, v, k1x, k1v, prev_inv_err, acc, rej, it + 1)

        x0, v0 = x0_ref[...], v0_ref[...]
        k1x, k1v = _bs3_rhs(mu, x0, v0)
        zeros_i = jnp.zeros(x0.shape, jnp.int32)
        init = (
            jnp.zeros_like(x0), jnp.full_like(x0, cfg.dt0), x0, v0, k1x, k1v,
            jnp.ones_like(x0), zeros_i, zeros_i, zeros_i,
        )
        t, _, x, v, _, _, _, acc, rej, _ = lax.while_loop(cond, body, init)
        to_ref[...] = t
        xo_ref[...] = x
        vo_ref[...] = v
        acc_ref[...] = acc
        rej_ref[...] = rej

    kernel.__name__ = "bs3_vdp"
    return kernel


def bs3_vdp_lockstep_kernel(cfg: BS3Config, max_steps: int):
    """The reference's own formulation (`tests/test_08_adaptive.py:33-142`):
    the same attempt in a fixed-trip `fori_loop` of `max_steps`; a lane
    that reaches T1 keeps attempting zero steps, which change nothing.
    Outputs (t, x, v, steps, rejected) as float32 counters; `steps` counts
    accepted attempts including the idle ones after T1."""

    def kernel(x0_ref, v0_ref, mu_ref, to_ref, xo_ref, vo_ref, steps_ref, rej_ref):
        mu = mu_ref[...]

        def step(_, c):
            t, dt, x, v, k1x, k1v, prev_inv_err, steps, rej = c
            accept, t, dt, x, v, k1x, k1v, prev_inv_err = _bs3_attempt(cfg, mu, t, dt, x, v, k1x, k1v, prev_inv_err)
            steps = steps + jnp.where(accept, 1.0, 0.0)
            rej = rej + jnp.where(accept, 0.0, 1.0)
            return (t, dt, x, v, k1x, k1v, prev_inv_err, steps, rej)

        x0, v0 = x0_ref[...], v0_ref[...]
        k1x, k1v = _bs3_rhs(mu, x0, v0)
        init = (jnp.zeros_like(x0), jnp.full_like(x0, cfg.dt0), x0, v0, k1x, k1v, jnp.ones_like(x0),
                jnp.zeros_like(x0), jnp.zeros_like(x0))
        t, _, x, v, _, _, _, steps, rej = lax.fori_loop(0, max_steps, step, init)
        to_ref[...] = t
        xo_ref[...] = x
        vo_ref[...] = v
        steps_ref[...] = steps
        rej_ref[...] = rej

    kernel.__name__ = "bs3_vdp_lockstep"
    return kernel


def bs3_vdp_call(n: int, cfg: BS3Config = BS3_CFG, name: str = "bs3_vdp", **kw: Any):
    import palladium_amd as pa

    spec = pl.BlockSpec((1,), lambda i: (i,))
    return pa.hip_call(
        bs3_vdp_kernel(cfg),
        grid=(n,),
        in_specs=[spec] * 3,
        out_specs=tuple([spec] * 5),
        out_shape=(
            pl.ShapeDtypeStruct((n,), F32), pl.ShapeDtypeStruct((n,), F32), pl.ShapeDtypeStruct((n,), F32),
            pl.ShapeDtypeStruct((n,), np.int32), pl.ShapeDtypeStruct((n,), np.int32),
        ),
        name=name,
        **kw,
    )


def bs3_vdp_lockstep_call(n: int, max_steps: int, cfg: BS3Config = BS3_CFG, **kw: Any):
    import palladium_amd as pa

    spec = pl.BlockSpec((1,), lambda i: (i,))
    return pa.hip_call(
        bs3_vdp_lockstep_kernel(cfg, max_steps),
        grid=(n,),
        in_specs=[spec] * 3,
        out_specs=tuple([spec] * 5),
        out_shape=tuple(pl.ShapeDtypeStruct((n,), F32) for _ in range(5)),
        name="bs3_vdp_lockstep",
        **kw,
    )


def bs3_inputs(n: int, seed: int = BS3_CFG.seed) -> tuple[np.ndarray, ...]:
    """(x0, v0, mu): mu log-uniform in [0.1, 100], (x0, v0) ~ U(-2, 2)^2."""
    rng = np.random.default_rng(seed)
    mu = (10.0 ** rng.uniform(-1.0, 2.0, n)).astype(F32)
    x0 = rng.uniform(-2.0, 2.0, n).astype(F32)
    v0 = rng.uniform(-2.0, 2.0, n).astype(F32)
    return x0, v0, mu


# ---------------------------------------------------------------------------
# GBM Monte Carlo


@dataclasses.dataclass(frozen=True)
class GBMConfig:
    n_paths: int = 4_194_304
    n_steps: int = 252
    s0: float = 100.0
    r: float = 0.05
    sigma: float = 0.2
    t: float = 1.0
    strike: float = 105.0
    seed: int = 42

    @property
    def dt(self) -> float:
        return self.t / self.n_steps

    @property
    def drift_dt(self) -> float:
        return (self.r - self.sigma**2 / 2) * self.dt

    @property
    def vol_sqdt(self) -> float:
        return self.sigma * math.sqrt(self.dt)


GBM_CFG = GBMConfig()


def gbm_kernel(cfg: GBMConfig):
    """Kernel: refs (key u32[2]) -> payoff per path.

    One Threefry-2x32-20 block per (path, step) counter supplies both
    uniforms (bits -> float exactly as `jax.random.uniform`), Box-Muller
    gives z, and the log-Euler GBM update multiplies s by
    exp(drift*dt + sigma*sqrt(dt)*z) (`examples/03_sde_montecarlo.py:97-119`
    with the configured counter layout)."""
    drift, vol = cfg.drift_dt, cfg.vol_sqdt

    def kernel(key_ref, o_ref):
        path = pl.program_id(0).astype(jnp.uint32)
        k0, k1 = key_ref[0], key_ref[1]

        def step(i, s):
            b0, b1 = random.threefry2x32_p(k0, k1, path, i.astype(jnp.uint32))
            u1 = jnp.maximum(random.bits_to_uniform(b0), 1e-7)
            u2 = random.bits_to_uniform(b1)
            z = jnp.sqrt(-2.0 * jnp.log(u1)) * jnp.cos(2.0 * jnp.pi * u2)
            return s * jnp.exp(drift + vol * z)

        s = lax.fori_loop(0, cfg.n_steps, step, cfg.s0)
        o_ref[0] = jnp.maximum(s - cfg.strike, 0.0)

    kernel.__name__ = "gbm_paths"
    return kernel


def gbm_call(cfg: GBMConfig = GBM_CFG, n_paths: int | None = None, **kw: Any):
    import palladium_amd as pa

    n = n_paths or cfg.n_paths
    return pa.hip_call(
        gbm_kernel(cfg),
        grid=(n,),
        in_specs=[pl.BlockSpec((2,), lambda i: (0,))],
        out_specs=pl.BlockSpec((1,), lambda i: (i,)),
        out_shape=pl.ShapeDtypeStruct((n,), F32),
        **{"name": "gbm_paths", **kw},
    )


def gbm_fold_in_kernel(cfg: GBMConfig, record_steps: int = 0):
    """The reference's own derivation (`examples/03_sde_montecarlo.py:95-117`):
    key0 = fold_in(key, path); per step i, u1 from fold_in(key0, 2i) and u2
    from fold_in(key0, 2i + 1), each through `random.uniform` (four Threefry
    blocks per step, against the one-block counter form of `gbm_kernel`).
    With `record_steps`, the first steps' (u1, u2) are also written out, so
    the raw uniforms can be checked bit for bit."""
    drift, vol = cfg.drift_dt, cfg.vol_sqdt

    def kernel(key_ref, o_ref, *u_refs):
        base = random.wrap_key_data(key_ref[...])
        key0 = random.fold_in(base, pl.program_id(0))

        def uniforms(i):
            k1 = random.fold_in(key0, 2 * i)
            k2 = random.fold_in(key0, 2 * i + 1)
            return jnp.maximum(random.uniform(k1, ()), 1e-7), random.uniform(k2, ())

        def step(i, s):
            u1, u2 = uniforms(i)
            z = jnp.sqrt(-2.0 * jnp.log(u1)) * jnp.cos(2.0 * jnp.pi * u2)
            return s * jnp.exp(drift + vol * z)

        s = lax.fori_loop(0, cfg.n_steps, step, cfg.s0)
        o_ref[0] = jnp.maximum(s - cfg.strike, 0.0)
        for j in range(record_steps):
            u1, u2 = uniforms(j)
            u_refs[0][0, j] = u1
            u_refs[1][0, j] = u2

    kernel.__name__ = "gbm_fold_in"
    return kernel


def gbm_fold_in_call(cfg: GBMConfig = GBM_CFG, n_paths: int | None = None, record_steps: int = 0, **kw: Any):
    import palladium_amd as pa

    n = n_paths or cfg.n_paths
    out_specs = [pl.BlockSpec((1,), lambda i: (i,))]
    out_shape = [pl.ShapeDtypeStruct((n,), F32)]
    if record_steps:
        rec = pl.BlockSpec((1, record_steps), lambda i: (i, 0))
        out_specs += [rec, rec]
        out_shape += [pl.ShapeDtypeStruct((n, record_steps), F32)] * 2
    return pa.hip_call(
        gbm_fold_in_kernel(cfg, record_steps),
        grid=(n,),
        in_specs=[pl.BlockSpec((2,), lambda i: (0,))],
        out_specs=tuple(out_specs) if record_steps else out_specs[0],
        out_shape=tuple(out_shape) if record_steps else out_shape[0],
        name="gbm_fold_in",
        **kw,
    )


def black_scholes_call(s0: float, k: float, t: float, r: float, sigma: float) -> float:
    """Closed-form European call (`examples/03_sde_montecarlo.py:73-76`)."""
    d1 = (math.log(s0 / k) + (r + sigma**2 / 2) * t) / (sigma * math.sqrt(t))
    d2 = d1 - sigma * math.sqrt(t)
    ncdf = lambda x: 0.5 * (1.0 + math.erf(x / math.sqrt(2.0)))  # noqa: E731
    return s0 * ncdf(d1) - k * math.exp(-r * t) * ncdf(d2)


# ---------------------------------------------------------------------------
# Gray-Scott


@dataclasses.dataclass(frozen=True)
class GrayScottConfig:
    size: int = 4096
    steps: int = 2000
    du: float = 0.16
    dv: float = 0.08
    f: float = 0.037
    k: float = 0.06
    dt: float = 1.0
    seed: int = 4


GS_CFG = GrayScottConfig()


def gray_scott_kernel(cfg: GrayScottConfig, size: int):
    """Kernel: refs (u, v) full arrays -> (u', v'), one cell per instance,
    periodic 5-point Laplacian via indexed refs
    (`examples/04_reaction_diffusion.py:61-74`)."""
    DU, DV, F, KK, DT = cfg.du, cfg.dv, cfg.f, cfg.k, cfg.dt

    def kernel(u_ref, v_ref, uo_ref, vo_ref):
        i, j = pl.program_id(0), pl.program_id(1)
        n = size
        ip = jnp.where(i == n - 1, 0, i + 1)
        im = jnp.where(i == 0, n - 1, i - 1)
        jp = jnp.where(j == n - 1, 0, j + 1)
        jm = jnp.where(j == 0, n - 1, j - 1)
        u, v = u_ref[i, j], v_ref[i, j]
        lap_u = u_ref[ip, j] + u_ref[im, j] + u_ref[i, jp] + u_ref[i, jm] - 4.0 * u
        lap_v = v_ref[ip, j] + v_ref[im, j] + v_ref[i, jp] + v_ref[i, jm] - 4.0 * v
        uvv = u * v * v
        uo_ref[i, j] = u + DT * (DU * lap_u - uvv + F * (1.0 - u))
        vo_ref[i, j] = v + DT * (DV * lap_v + uvv - (F + KK) * v)

    kernel.__name__ = "gray_scott"
    return kernel


def gray_scott_call(cfg: GrayScottConfig = GS_CFG, size: int | None = None, **kw: Any):
    import palladium_amd as pa

    n = size or cfg.size
    full = pl.BlockSpec((n, n), lambda i, j: (0, 0))
    return pa.hip_call(
        gray_scott_kernel(cfg, n),
        grid=(n, n),
        in_specs=[full, full],
        out_specs=(full, full),
        out_shape=(pl.ShapeDtypeStruct((n, n), F32), pl.ShapeDtypeStruct((n, n), F32)),
        name="gray_scott",
        **kw,
    )


def gray_scott_initial(size: int, seed: int = GS_CFG.seed) -> tuple[np.ndarray, np.ndarray]:
    """U=1, V=0, a central 64x64 square (scaled for small grids) of U=0.5,
    V=0.25, plus 1% uniform noise on U."""
    rng = np.random.default_rng(seed)
    u = np.ones((size, size), F32)
    v = np.zeros((size, size), F32)
    half = min(32, size // 8)
    m = size // 2
    u[m - half : m + half, m - half : m + half] = 0.5
    v[m - half : m + half, m - half : m + half] = 0.25
    u += (0.01 * rng.random((size, size))).astype(F32)
    return u, v


# Algorithmic HBM traffic of one Gray-Scott cell-step: read u, v and write
# u', v' once each (halo re-reads excluded).
GS_BYTES_PER_CELL_STEP = 16


def gray_scott_run(call, u0: np.ndarray, v0: np.ndarray, steps: int, graph: bool = True):
    """Run `steps` Gray-Scott steps on the GPU, ping-ponging two buffer pairs,
    all launches queued as one batch (one HIP graph when `graph`); the
    multi-launch driver of `examples/04_reaction_diffusion.py:77-109`.
    Returns (u, v, device seconds)."""
    from palladium_amd import runtime as rt

    bound = call.bound(u0, v0)
    geo = bound.geometry
    bufs = [
        [rt.Buffer.from_numpy(u0), rt.Buffer.from_numpy(v0)],
        [rt.Buffer.empty(u0.shape, F32), rt.Buffer.empty(v0.shape, F32)],
    ]
    batch = rt.Batch(stream=bound.stream)
    src = 0
    for _ in range(steps):
        dst = 1 - src
        batch.add(bound.kernel, geo.blocks, geo.block, [b.ptr for b in bufs[src]] + [b.ptr for b in bufs[dst]])
        src = dst
    batch.commit(graph=graph)
    batch.wait()
    return bufs[src][0].to_numpy(bound.stream), bufs[src][1].to_numpy(bound.stream), batch.gpu_time


def gbm_block_kernel(cfg: GBMConfig, block: int):
    """Kernel: refs (key u32[2]) -> one discounted-payoff *sum* per block of
    `block` paths ("reduced per block"). The block's paths are the rows of
    a (block,) value, which the emitter spreads across `block` lanes; the
    closing `jnp.sum` is a cross-lane reduction."""
    drift, vol = cfg.drift_dt, cfg.vol_sqdt
    disc = math.exp(-cfg.r * cfg.t)

    def kernel(key_ref, o_ref):
        k0, k1 = key_ref[0], key_ref[1]
        first = pl.program_id(0) * block
        path = (first + lax.iota(jnp.int32, block)).astype(jnp.uint32)

        def step(i, s):
            b0, b1 = random.threefry2x32_p(k0, k1, path, i.astype(jnp.uint32))
            u1 = jnp.maximum(random.bits_to_uniform(b0), 1e-7)
            u2 = random.bits_to_uniform(b1)
            z = jnp.sqrt(-2.0 * jnp.log(u1)) * jnp.cos(2.0 * jnp.pi * u2)
            return s * jnp.exp(drift + vol * z)

        s = lax.fori_loop(0, cfg.n_steps, step, jnp.full((block,), cfg.s0, jnp.float32))
        o_ref[0] = jnp.sum(disc * jnp.maximum(s - cfg.strike, 0.0))

    kernel.__name__ = "gbm_block_sums"
    return kernel


def gbm_block_call(cfg: GBMConfig = GBM_CFG, block: int = 256, n_paths: int | None = None, **kw: Any):
    import palladium_amd as pa

    n = n_paths or cfg.n_paths
    if n % block:
        raise ValueError(f"n_paths={n} is not a multiple of block={block}")
    return pa.hip_call(
        gbm_block_kernel(cfg, block),
        grid=(n // block,),
        in_specs=[pl.BlockSpec((2,), lambda i: (0,))],
        out_specs=pl.BlockSpec((1,), lambda i: (i,)),
        out_shape=pl.ShapeDtypeStruct((n // block,), F32),
        name="gbm_block_sums",
        **kw,
    )
