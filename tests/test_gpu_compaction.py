"""Workgroup lane compaction of divergent while loops on the GPU: each
instance runs the same operations as without compaction, so results are
bit-identical to the uncompacted kernel, the interpreter and the oracle."""

import os

import numpy as np
import pytest

import oracle
import palladium_amd as pa
from palladium_amd.frontend import jnp, lax, pl
from palladium_amd.workloads import BS3_CFG, bs3_inputs, bs3_vdp_call

pytestmark = pytest.mark.gpu


def _collatz(n):
    """Integer, float, unsigned and bool carries; trip counts from 0 to a
    few hundred, so lanes finish at very different times."""
    def kernel(x_ref, f_ref, o_ref, s_ref, h_ref, b_ref):
        x = x_ref[...]
        f0 = f_ref[...]

        def cond(c):
            return c[0] > 1

        def body(c):
            v, k, s, h, odd = c
            is_odd = v % 2 == 1
            v2 = jnp.where(is_odd, 3 * v + 1, v // 2)
            return v2, k + 1, s * 0.75 + f0, h * jnp.uint32(2654435761) + v2.astype(jnp.uint32), odd | is_odd

        init = (x, jnp.zeros_like(x), jnp.zeros_like(f0), jnp.zeros(x.shape, jnp.uint32), x < 0)
        _, k, s, h, odd = lax.while_loop(cond, body, init)
        o_ref[...] = k
        s_ref[...] = s
        h_ref[...] = h
        b_ref[...] = odd.astype(jnp.int32)

    spec = pl.BlockSpec((1,), lambda i: (i,))
    shapes = (pl.ShapeDtypeStruct((n,), np.int32), pl.ShapeDtypeStruct((n,), np.float32),
              pl.ShapeDtypeStruct((n,), np.uint32), pl.ShapeDtypeStruct((n,), np.int32))
    return pa.hip_call(kernel, grid=(n,), in_specs=[spec, spec], out_specs=(spec,) * 4, out_shape=shapes,
                       math_mode="safe")


@pytest.mark.parametrize("n", [8192, 3000, 100])
def test_collatz_compacted_matches_interpreter_and_uncompacted(monkeypatch, n):
    """8,192 fills whole workgroups; 3,000 and 100 leave extra lanes in the
    last one, which must store nothing."""
    rng = np.random.default_rng(3 + n)
    x = rng.integers(1, 200_000, n).astype(np.int32)
    x[::97] = 1  # lanes that never enter the loop
    f = rng.standard_normal(n).astype(np.float32)
    call = _collatz(n)
    src = call.bound(x, f).hip_source
    assert "__syncthreads" in src
    got = call(x, f)
    want = call.interpret(x, f)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    assert got[0].max() > 100 and got[0].min() == 0
    monkeypatch.setenv("PALLADIUM_WHILE_COMPACTION", "0")
    plain = _collatz(n)
    assert "__syncthreads" not in plain.bound(x, f).hip_source
    for g, p in zip(got, plain(x, f)):
        np.testing.assert_array_equal(g, p)


@pytest.mark.parametrize("mode", ["safe", "fast"])
def test_bs3_compacted_equals_uncompacted(monkeypatch, mode):
    n = 65536
    args = bs3_inputs(n)
    f = bs3_vdp_call(n, math_mode=mode)
    assert "__syncthreads" in f.bound(*args).hip_source
    got = f(*args)
    monkeypatch.setenv("PALLADIUM_WHILE_COMPACTION", "0")
    g = bs3_vdp_call(n, math_mode=mode, name="bs3_vdp_plain")
    assert "__syncthreads" not in g.bound(*args).hip_source
    for a, b, name in zip(got, g(*args), ["t", "x", "v", "accepted", "rejected"]):
        np.testing.assert_array_equal(a, b, err_msg=name)
    if mode == "safe":
        want = oracle.bs3_vdp(*args, BS3_CFG)
        for a, w in zip(got, want):
            np.testing.assert_array_equal(a, w)


def _fuzz_kernel(seed):
    """A data-dependent while loop over random float/int carries: each lane
    runs until its own accumulator passes a threshold read from its input,
    so trip counts spread from 0 to a few hundred."""
    from test_gpu_emitter_fuzz import _expr, _tame

    def kernel(x_ref, y_ref, o_ref, p_ref):
        x, y = x_ref[...], y_ref[...]
        lim = jnp.abs(y) * 40.0 + 1.0

        def cond(c):
            acc, k, a, b = c
            return jnp.logical_and(acc < lim, k < 400)

        def body(c):
            acc, k, a, b = c
            r = np.random.default_rng(seed)
            na = _tame(_expr(r, [a, b, x], 3), np.dtype(np.float32))
            nb = _tame(_expr(r, [b, na, y], 2), np.dtype(np.float32))
            step = jnp.abs(na) * 0.25 + 0.05
            return acc + step, k + 1 + (k % 3), na, nb

        acc, k, a, b = lax.while_loop(cond, body, (jnp.zeros_like(x), jnp.zeros(x.shape, jnp.int32), x, y))
        o_ref[...] = a + b * 0.5
        p_ref[...] = acc + k.astype(jnp.float32)

    return kernel


@pytest.mark.parametrize("seed", range(int(os.environ.get("PALLADIUM_FUZZ_SEEDS", os.environ.get("PALLADIUM_FUZZ_EXAMPLES", "12")))))
def test_random_compacted_loops_bit_exact_vs_interpreter(seed):
    n = 2048
    rng = np.random.default_rng(700 + seed)
    x = rng.uniform(-3, 3, n).astype(np.float32)
    y = rng.uniform(-3, 3, n).astype(np.float32)
    spec = pl.BlockSpec((1,), lambda i: (i,))
    call = pa.hip_call(_fuzz_kernel(seed), grid=(n,), in_specs=[spec, spec], out_specs=(spec, spec),
                       out_shape=(pl.ShapeDtypeStruct((n,), np.float32),) * 2, math_mode="safe")
    assert "__syncthreads" in call.bound(x, y).hip_source
    got = call(x, y)
    want = call.interpret(x, y)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
