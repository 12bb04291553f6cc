"""Random while loops in the shape the SAFE carried-log rewrite looks for
(carries powered and updated by selecting between themselves and another
powered value), built with and without the rewrite on the GPU: equal bit
for bit, special bases included, with while-loop compaction on."""

import os

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd.emit.optimize import share_pow_logs
from palladium_amd.frontend import jnp, lax, pl
from palladium_amd.trace import trace

pytestmark = pytest.mark.gpu

F = np.float32
EXPONENTS = [0.5, -0.3, 0.2333, 2.0, -1.0, 3.0, 0.75, -2.5, 1e-3, 7.0]


def _program(seed):
    r = np.random.default_rng(seed)
    n_carries = int(r.integers(1, 4))
    trips = int(r.integers(1, 9))
    exps = [[float(F(r.choice(EXPONENTS))) for _ in range(2)] for _ in range(n_carries)]
    scales = [float(F(r.uniform(-1.5, 1.5))) for _ in range(n_carries)]
    thresholds = [float(F(r.uniform(-1, 2))) for _ in range(n_carries)]
    flips = [bool(r.integers(2)) for _ in range(n_carries)]

    def kernel(x_ref, o_ref):
        x = x_ref[...]

        def body(s):
            k, *cs = s
            kf = k.astype(jnp.float32)
            new, acc = [], s[-1]
            for i, c in enumerate(cs[:-1]):
                v = x * scales[i] + (kf - 1.5)
                pc, pv = c ** exps[i][0], v ** exps[i][1]
                acc = acc + jnp.where(pc == pc, pc, 0.0) * 0.5 + jnp.where(pv == pv, pv, 0.0)
                p = v > thresholds[i]
                new.append(jnp.where(p, v, c) if flips[i] else jnp.where(p, c, v))
            return (k + 1, *new, acc)

        init = (jnp.int32(0),) + tuple(x * (0.5 + i) for i in range(n_carries)) + (jnp.zeros_like(x),)
        out = lax.while_loop(lambda s: s[0] < trips, body, init)
        o_ref[...] = out[-1] + sum(out[1:-1])

    return kernel


def _inputs(n, seed):
    x = np.random.default_rng(seed).uniform(-3, 3, n).astype(F)
    x[:12] = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 1e-40, 3e38, 0.5, 2.0, -2.0], F)
    return x


@pytest.mark.parametrize("seed", range(int(os.environ.get("PALLADIUM_FUZZ_SEEDS", os.environ.get("PALLADIUM_FUZZ_EXAMPLES", "12")))))
def test_random_loop_shared_equals_unshared(seed, monkeypatch):
    n = 2048
    print(f"[share_pow_logs fuzz] seed={seed}", flush=True)
    x = _inputs(n, seed)
    s = pl.BlockSpec((1,), lambda i: (i,))

    def build():
        return pa.hip_call(_program(seed), grid=(n,), in_specs=[s], out_specs=s,
                           out_shape=pl.ShapeDtypeStruct((n,), F), math_mode="safe")

    on = build()
    spec = trace(on._staged, x)
    assert share_pow_logs(spec.jaxpr).eqns != spec.jaxpr.eqns, "the generator must hit the rewrite"
    got = on(x)
    monkeypatch.setenv("PALLADIUM_SHARE_POW_LOGS", "0")
    want = build()(x)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
