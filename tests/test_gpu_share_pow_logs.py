"""The SAFE carried-log rewrite on the GPU: kernels built with it equal the
same kernels built without it (PALLADIUM_SHARE_POW_LOGS=0) bit for bit,
including bases that are zero, negative, infinite, NaN or subnormal, with
and without while-loop compaction. Config 2's SAFE states and counts, built
with the rewrite, are checked against the C oracle in tests/test_gpu_bs3.py."""

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd.frontend import jnp, lax, pl

pytestmark = pytest.mark.gpu

F = np.float32


def _kernel(order):
    def kernel(x_ref, o_ref, c_ref):
        x = x_ref[...]

        def body(s):
            k, c, acc = s
            v = x * 0.5 + (k.astype(jnp.float32) - 2.0)
            # the powers see every special base; their NaNs are selected away
            # so the sum stays informative
            pc, pv = c ** -0.3, v ** 0.7
            acc = acc + jnp.where(c > 0, pc, 0.0) * jnp.where(v > 0, pv, 1.0) + jnp.where(v > 0, v ** 2.5, 0.0)
            p = v > 0.25
            c = jnp.where(p, v, c) if order == 0 else jnp.where(p, c, v)
            return k + 1, c, acc

        _, c, acc = lax.while_loop(lambda s: s[0] < 6, body, (jnp.int32(0), x, jnp.zeros_like(x)))
        o_ref[...] = acc
        c_ref[...] = c

    return kernel


def _inputs(n):
    r = np.random.default_rng(7)
    x = r.uniform(-4, 4, n).astype(F)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-42, -1e-42, 1.0, -1.0, 3e38, 4.5, 0.25],
                       F)
    x[: special.size] = special
    return x


@pytest.mark.parametrize("order", [0, 1])
@pytest.mark.parametrize("compaction", ["1", "0"])
def test_shared_logs_equal_unshared(order, compaction, monkeypatch):
    n = 4096
    print(f"[share_pow_logs] order={order} compaction={compaction}", flush=True)
    monkeypatch.setenv("PALLADIUM_WHILE_COMPACTION", compaction)
    x = _inputs(n)
    s = pl.BlockSpec((1,), lambda i: (i,))
    shapes = (pl.ShapeDtypeStruct((n,), F),) * 2

    def build():
        return pa.hip_call(_kernel(order), grid=(n,), in_specs=[s], out_specs=(s, s), out_shape=shapes,
                           math_mode="safe")

    on = build()
    assert "ph_pow_log(" in on.bound(x).hip_source.split("__global__")[1]
    got = on(x)
    monkeypatch.setenv("PALLADIUM_SHARE_POW_LOGS", "0")
    off = build()
    assert "ph_pow_log(" not in off.bound(x).hip_source.split("__global__")[1]
    want = off(x)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g.view(np.uint32), w.view(np.uint32))
    assert np.isfinite(got[0]).sum() > n // 2 and np.unique(got[0]).size > n // 4
