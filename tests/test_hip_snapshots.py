"""Golden HIP snapshots: pin the emitted text, not only its values (the
reference's tests/test_msl_snapshots.py, same four kernels, plus the
benchmark kernels). Unintended codegen drift (a lost offset factor, a
changed launch remap, an extra copy, a rewrite that stopped firing) shows
up as a reviewable diff. The emitter's name counter is deterministic.

Regenerate after an intended emitter change:

    PALLADIUM_REGEN_GOLDEN=1 python -m pytest tests/test_hip_snapshots.py

No GPU needed (pure text)."""

import os
from pathlib import Path

import numpy as np
import pytest

from palladium_amd.emit import emit_hip
from palladium_amd.frontend import jnp, lax, pl
from palladium_amd.trace import trace
from palladium_amd.workloads import (
    BS3_CFG,
    GBMConfig,
    bs3_inputs,
    bs3_vdp_call,
    gbm_call,
    gray_scott_call,
    lv_inputs,
    lv_rk4_call,
)

GOLDEN = Path(__file__).parent / "golden"
DT, STEPS = 0.01, 500
F = np.float32


def _copy_2d():
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...]

    f = pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((16, 32), F))
    return trace(f, np.zeros((16, 32), F))


def _blocked_saxpy():
    def kernel(x_ref, y_ref, o_ref):
        o_ref[...] = 2.5 * x_ref[...] + y_ref[...]

    spec_8 = pl.BlockSpec((8,), lambda i: (i,))
    f = pl.pallas_call(kernel, grid=(32,), in_specs=[spec_8, spec_8], out_specs=spec_8,
                       out_shape=pl.ShapeDtypeStruct((256,), F))
    x = np.zeros(256, F)
    return trace(f, x, x)


def _rk4_lotka_volterra():
    def kernel(x_ref, y_ref, a_ref, b_ref, c_ref, d_ref, xo_ref, yo_ref):
        a, b, c, d = a_ref[...], b_ref[...], c_ref[...], d_ref[...]

        def rhs(x, y):
            return a * x - b * x * y, c * x * y - d * y

        def step(_, carry):
            x, y = carry
            k1x, k1y = rhs(x, y)
            k2x, k2y = rhs(x + 0.5 * DT * k1x, y + 0.5 * DT * k1y)
            k3x, k3y = rhs(x + 0.5 * DT * k2x, y + 0.5 * DT * k2y)
            k4x, k4y = rhs(x + DT * k3x, y + DT * k3y)
            return (x + DT / 6.0 * (k1x + 2.0 * k2x + 2.0 * k3x + k4x),
                    y + DT / 6.0 * (k1y + 2.0 * k2y + 2.0 * k3y + k4y))

        x, y = lax.fori_loop(0, STEPS, step, (x_ref[...], y_ref[...]))
        xo_ref[...] = x
        yo_ref[...] = y

    n = 64
    spec_1 = pl.BlockSpec((1,), lambda i: (i,))
    f = pl.pallas_call(kernel, grid=(n,), in_specs=[spec_1] * 6, out_specs=(spec_1, spec_1),
                       out_shape=(pl.ShapeDtypeStruct((n,), F),) * 2)
    return trace(f, *[np.zeros(n, F)] * 6)


def _conditional_loop():
    def kernel(y0_ref, r_ref, o_ref):
        r = r_ref[...]

        def step(_, y):
            grown = y + r
            return jnp.where(grown <= 1.0, grown, y)

        o_ref[...] = lax.fori_loop(0, 20, step, y0_ref[...])

    f = pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((64,), F))
    x = np.zeros(64, F)
    return trace(f, x, x)


def _bench_lv():
    return trace(lv_rk4_call(1_000_000, 0.005, 4000, track_max=True)._staged, *lv_inputs(8, 1))


def _bench_gray_scott():
    z = np.zeros((4096, 4096), F)
    return trace(gray_scott_call(size=4096)._staged, z, z)


def _bench_gbm():
    from palladium_amd.frontend import random

    return trace(gbm_call(GBMConfig())._staged, random.key(42))


def _bench_bs3():
    return trace(bs3_vdp_call(BS3_CFG.n)._staged, *bs3_inputs(8))


# (spec builder, math mode): the reference's four under SAFE (the traced op
# order, no FAST rewrites), the benchmark kernels as benchmarked (FAST).
SNAPSHOTS = {
    "copy_2d": (_copy_2d, "safe"),
    "blocked_saxpy": (_blocked_saxpy, "safe"),
    "rk4_lotka_volterra": (_rk4_lotka_volterra, "safe"),
    "conditional_loop": (_conditional_loop, "safe"),
    "bench_lv_rk4_fast": (_bench_lv, "fast"),
    "bench_gray_scott_fast": (_bench_gray_scott, "fast"),
    "bench_gbm_fast": (_bench_gbm, "fast"),
    "bench_bs3_fast": (_bench_bs3, "fast"),
}


def _body(src: str) -> str:
    # The shared device prelude is pinned by its own tests; snapshot the kernel.
    return src[src.index('extern "C"'):]


@pytest.mark.parametrize("name", SNAPSHOTS)
def test_emitted_hip_matches_golden(name):
    build, mode = SNAPSHOTS[name]
    spec = build()
    hip = _body(emit_hip(spec, math_mode=mode))
    path = GOLDEN / f"{name}.hip.golden"
    if os.environ.get("PALLADIUM_REGEN_GOLDEN") == "1":
        path.write_text(hip)
        pytest.skip(f"regenerated {path.name}")
    assert path.exists(), f"missing snapshot {path.name}; bless it with PALLADIUM_REGEN_GOLDEN=1"
    assert hip == path.read_text(), (
        f"emitted HIP for '{name}' drifted from its snapshot; if the change is intended, "
        "regenerate with PALLADIUM_REGEN_GOLDEN=1 and review the diff"
    )
