"""Predicated while loops run several iterations per machine-loop pass,
each with its own exit test (palladium_amd/emit/compact.py, rules.py).
Loops of 0 to 70 iterations, lanes of mixed trip counts, with and without
compaction, every math mode: results equal the interpreter (SAFE) and the
build with one iteration per pass."""

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd.frontend import jnp, lax, pl

pytestmark = pytest.mark.gpu


def _kernel(x_ref, trips_ref, o_ref, k_ref):
    x, trips = x_ref[...], trips_ref[...]

    def body(c):
        k, v = c
        return k + 1, v * 0.75 + 0.125 * (v * v) - 0.0625  # IEEE basic ops: SAFE equals the interpreter

    k, v = lax.while_loop(lambda c: c[0] < trips, body, (jnp.zeros_like(trips), x))
    o_ref[...] = v
    k_ref[...] = k


@pytest.mark.parametrize("mode", ["safe", "fast"])
@pytest.mark.parametrize("compaction", ["1", "0"])
@pytest.mark.parametrize("trips", ["short", "mixed"])
def test_iteration_counts_and_states(mode, compaction, trips, monkeypatch):
    n = 4096
    print(f"[while passes] mode={mode} compaction={compaction} trips={trips}", flush=True)
    monkeypatch.setenv("PALLADIUM_WHILE_COMPACTION", compaction)
    r = np.random.default_rng(3)
    x = r.uniform(-2, 2, n).astype(np.float32)
    hi = 4 if trips == "short" else 71
    t = r.integers(0, hi, n).astype(np.int32)
    s = pl.BlockSpec((1,), lambda i: (i,))

    def build():
        return pa.hip_call(_kernel, grid=(n,), in_specs=[s, s], out_specs=(s, s),
                           out_shape=(pl.ShapeDtypeStruct((n,), np.float32), pl.ShapeDtypeStruct((n,), np.int32)),
                           math_mode=mode)

    got = build()(x, t)
    np.testing.assert_array_equal(got[1], t)
    monkeypatch.setenv("PALLADIUM_EPOCH_UNROLL", "1")
    one = build()(x, t)
    for g, w in zip(got, one):
        np.testing.assert_array_equal(np.asarray(g).view(np.uint32), np.asarray(w).view(np.uint32))
    if mode == "safe":
        want = build().interpret(x, t)
        for g, w in zip(got, want):
            np.testing.assert_array_equal(g, w)
