"""The exact counter fold (palladium_amd.emit.optimize.fold_counters): an
adaptive loop's accepted and rejected counts beside its attempt count."""

import dataclasses

import numpy as np
import pytest

from palladium_amd.emit.optimize import fold_counters
from palladium_amd.frontend import jnp, lax, pl
from palladium_amd.interpret import interpret_spec
from palladium_amd.trace import trace
from palladium_amd.workloads import bs3_inputs, bs3_vdp_call


def _counter_kernel(step=1, a_cases=(0, 1), b_cases=(1, 0), cond_reads_counts=False):
    def kernel(x_ref, a_ref, b_ref, n_ref):
        x = x_ref[...]

        def cond(c):
            k, v, a, b, n = c
            go = (v > 0.05) & (n < 40)
            return go & (a < 1000) & (b < 1000) if cond_reads_counts else go

        def body(c):
            k, v, a, b, n = c
            p = v * 7.0 - jnp.floor(v * 7.0) < 0.5          # a data-dependent accept
            v = jnp.where(p, v * 0.5, v * 0.9)
            a = a + jnp.where(p, a_cases[1], a_cases[0])
            b = b + jnp.where(p, b_cases[1], b_cases[0])
            return k, v, a, b, n + step

        init = [jnp.full_like(x, c, jnp.int32) for c in (3, -5, 11)]
        _, _, a, b, n = lax.while_loop(cond, body, (jnp.int32(0), x, *init))
        a_ref[...] = a
        b_ref[...] = b
        n_ref[...] = n

    return kernel


def _spec(kernel, n=256):
    x = np.random.default_rng(17).uniform(0.0, 1.0, n).astype(np.float32)
    s = pl.BlockSpec((1,), lambda i: (i,))
    call = pl.pallas_call(kernel, grid=(n,), in_specs=[s], out_specs=(s, s, s),
                          out_shape=(pl.ShapeDtypeStruct((n,), np.int32),) * 3)
    return trace(call, x), x


def _while(jaxpr):
    (w,) = [e for e in jaxpr.eqns if e.primitive.name == "while"]
    return w


def _dropped(before, after):
    """Indices of the loop results the fold took out of the loop."""
    kept = {id(v) for v in _while(after).outvars}
    return [k for k, v in enumerate(_while(before).outvars) if id(v) not in kept]


@pytest.mark.parametrize("step,a_cases,b_cases", [(1, (0, 1), (1, 0)), (2, (0, 2), (2, 0)), (2, (1, 2), (1, 0))])
def test_fold_is_exact_and_drops_one_counter(step, a_cases, b_cases):
    spec, x = _spec(_counter_kernel(step, a_cases, b_cases))
    opt = dataclasses.replace(spec, jaxpr=fold_counters(spec.jaxpr))
    assert _dropped(spec.jaxpr, opt.jaxpr) in ([2], [3])     # a or b, whichever is found first
    got, want = interpret_spec(opt, x), interpret_spec(spec, x)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    # the counts themselves, from a plain restatement of the loop
    a_np, b_np, n_np = [], [], []
    for v in x:
        v, a, b, n = np.float32(v), 3, -5, 11
        while v > np.float32(0.05) and n < 40:
            p = v * np.float32(7) - np.floor(v * np.float32(7)) < 0.5
            v = v * np.float32(0.5) if p else v * np.float32(0.9)
            a, b, n = a + a_cases[int(p)], b + b_cases[int(p)], n + step
        a_np.append(a), b_np.append(b), n_np.append(n)
    np.testing.assert_array_equal(got[0], a_np)
    np.testing.assert_array_equal(got[1], b_np)
    np.testing.assert_array_equal(got[2], n_np)
    assert len(set(b_np)) > 3  # the counts vary from lane to lane


@pytest.mark.parametrize("kw", [dict(a_cases=(0, 1), b_cases=(1, 1)),        # a + b - n not invariant
                                dict(step=2),                                 # increments sum to 1, not 2
                                dict(cond_reads_counts=True)])                # both are read by the condition
def test_fold_leaves_loops_it_cannot_prove(kw):
    spec, _ = _spec(_counter_kernel(**kw))
    assert fold_counters(spec.jaxpr).eqns == spec.jaxpr.eqns


def test_fold_takes_the_counter_the_condition_does_not_read():
    def kernel(x_ref, a_ref, b_ref, n_ref):
        x = x_ref[...]

        def body(c):
            v, a, b, n = c
            p = v * 3.0 - jnp.floor(v * 3.0) < 0.5
            return v * 0.8, a + jnp.where(p, 1, 0), b + jnp.where(p, 0, 1), n + 1

        init = [jnp.full_like(x, 0, jnp.int32) for _ in range(3)]
        _, a, b, n = lax.while_loop(lambda c: (c[0] > 0.1) & (c[2] < 7), body, (x, *init))
        a_ref[...], b_ref[...], n_ref[...] = a, b, n

    spec, x = _spec(kernel)
    assert _dropped(spec.jaxpr, fold_counters(spec.jaxpr)) == [1]   # a, not the b the condition reads
    opt = dataclasses.replace(spec, jaxpr=fold_counters(spec.jaxpr))
    for g, want in zip(interpret_spec(opt, x), interpret_spec(spec, x)):
        np.testing.assert_array_equal(g, want)


def test_bs3_counts_fold_bit_identically():
    args = bs3_inputs(512)
    spec = trace(bs3_vdp_call(512)._staged, *args)
    opt = dataclasses.replace(spec, jaxpr=fold_counters(spec.jaxpr))
    assert len(_dropped(spec.jaxpr, opt.jaxpr)) == 1
    for g, w in zip(interpret_spec(opt, *args), interpret_spec(spec, *args)):
        np.testing.assert_array_equal(g, w)


def _random_counter_kernel(seed):
    """A while loop with 3-5 integer counters, each stepping by a select of
    two small literals on one of two predicates, or by a fixed literal; the
    condition reads the float state and, sometimes, one counter."""
    r = np.random.default_rng(seed)
    m = int(r.integers(3, 6))
    kinds = []
    for _ in range(m):
        if r.random() < 0.3:
            kinds.append(("step", int(r.integers(-2, 4))))
        else:
            kinds.append(("sel", int(r.integers(0, 2)), int(r.integers(-2, 4)), int(r.integers(-2, 4))))
    if r.random() < 0.7:  # plant a complementary pair
        i, j = r.choice(m, 2, replace=False)
        s = int(r.integers(1, 4))
        a0 = int(r.integers(-2, 4))
        a1 = int(r.integers(-2, 4))
        p = int(r.integers(0, 2))
        kinds[i] = ("sel", p, a0, a1)
        kinds[j] = ("sel", p, s - a0, s - a1)
        kinds.append(("step", s))
    init = [int(v) for v in r.integers(-50, 50, len(kinds))]
    cond_reads = int(r.integers(-1, len(kinds)))
    cap = int(r.integers(5, 40))

    def kernel(x_ref, *outs):
        x = x_ref[...]

        def cond(c):
            v, cs = c[0], c[1:]
            go = (v > 0.02) & (cs[-1] < cap + 1000)
            return go & (cs[cond_reads] < 10_000) if cond_reads >= 0 else go

        def body(c):
            v, cs = c[0], list(c[1:])
            p0 = v * 7.0 - jnp.floor(v * 7.0) < 0.5
            p1 = v * 3.0 - jnp.floor(v * 3.0) < 0.3
            for k, kind in enumerate(kinds):
                if kind[0] == "step":
                    cs[k] = cs[k] + kind[1]
                else:
                    cs[k] = cs[k] + jnp.where((p0, p1)[kind[1]], kind[3], kind[2])
            return (jnp.where(p0, v * 0.5, v * 0.85), *cs)

        res = lax.while_loop(cond, body, (x, *[jnp.full_like(x, c, jnp.int32) for c in init]))
        for o, c in zip(outs, res[1:]):
            o[...] = c

    return kernel, len(kinds)


@pytest.mark.parametrize("seed", range(60))
def test_fold_fuzz_bit_identical(seed):
    kernel, m = _random_counter_kernel(seed)
    n = 64
    x = np.random.default_rng(seed).uniform(0.0, 1.0, n).astype(np.float32)
    s = pl.BlockSpec((1,), lambda i: (i,))
    call = pl.pallas_call(kernel, grid=(n,), in_specs=[s], out_specs=(s,) * m,
                          out_shape=(pl.ShapeDtypeStruct((n,), np.int32),) * m)
    spec = trace(call, x)
    folded = fold_counters(spec.jaxpr)
    opt = dataclasses.replace(spec, jaxpr=folded)
    for g, w in zip(interpret_spec(opt, x), interpret_spec(spec, x)):
        np.testing.assert_array_equal(g, w)


def test_fold_fuzz_fires_on_most_planted_pairs():
    fired = 0
    for seed in range(60):
        kernel, m = _random_counter_kernel(seed)
        x = np.zeros(64, np.float32)
        s = pl.BlockSpec((1,), lambda i: (i,))
        call = pl.pallas_call(kernel, grid=(64,), in_specs=[s], out_specs=(s,) * m,
                              out_shape=(pl.ShapeDtypeStruct((64,), np.int32),) * m)
        spec = trace(call, x)
        fired += bool(_dropped(spec.jaxpr, fold_counters(spec.jaxpr)))
    assert fired >= 35   # 41 of these 60 seeds plant a pair the fold can prove


def test_fold_on_unsigned_counters_wraps_like_the_loop():
    """uint32 counts starting near 2**32: the rebuilt count wraps exactly as
    the carried one would have."""
    def kernel(x_ref, a_ref, b_ref, n_ref):
        x = x_ref[...]

        def body(c):
            v, a, b, n = c
            p = v * 5.0 - jnp.floor(v * 5.0) < 0.5
            one, zero = jnp.uint32(1), jnp.uint32(0)
            return v * 0.8, a + jnp.where(p, one, zero), b + jnp.where(p, zero, one), n + jnp.uint32(1)

        init = [jnp.full_like(x, c, jnp.uint32) for c in (0xFFFFFFF0, 0xFFFFFFFA, 7)]
        _, a, b, n = lax.while_loop(lambda c: c[0] > 0.05, body, (x, *init))
        a_ref[...], b_ref[...], n_ref[...] = a, b, n

    n = 64
    x = np.random.default_rng(2).uniform(0.1, 1.0, n).astype(np.float32)
    s = pl.BlockSpec((1,), lambda i: (i,))
    call = pl.pallas_call(kernel, grid=(n,), in_specs=[s], out_specs=(s, s, s),
                          out_shape=(pl.ShapeDtypeStruct((n,), np.uint32),) * 3)
    spec = trace(call, x)
    opt = dataclasses.replace(spec, jaxpr=fold_counters(spec.jaxpr))
    assert len(_dropped(spec.jaxpr, opt.jaxpr)) == 1
    got, want = interpret_spec(opt, x), interpret_spec(spec, x)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    assert (got[1] < 100).any() and (got[1] > 0xFFFFFF00).any()   # some wrapped, some not


def _boundary_kernel(nx):
    """A loop carrying v, accepted, rejected and attempt counts plus `nx`
    float carries, all read after the loop: 9 + 2 nx LDS words per lane
    before the fold, one carry (two words) fewer after it."""

    def kernel(x_ref, *outs):
        x = x_ref[...]

        def cond(c):
            return (c[0] > 0.05) & (c[3] < 40)

        def body(c):
            v, a, b, n = c[:4]
            fs = c[4:]
            p = v * 7.0 - jnp.floor(v * 7.0) < 0.5
            v = jnp.where(p, v * 0.5, v * 0.9)
            fs = tuple(f * 0.5 + v for f in fs)
            return (v, a + jnp.where(p, 1, 0), b + jnp.where(p, 0, 1), n + 1, *fs)

        zi = jnp.zeros(x.shape, jnp.int32)
        init = (x, zi, zi, zi, *[x * float(k + 1) for k in range(nx)])
        res = lax.while_loop(cond, body, init)
        for ref, val in zip(outs, res):
            ref[...] = val

    return kernel


def test_fold_does_not_move_a_loop_across_the_compaction_budget():
    """With six float carries the traced loop is over compaction's LDS
    budget and the fold would bring it under; the emitter must keep the
    launch geometry's choice (no compaction) and still emit and run."""
    from palladium_amd.emit.compact import plan_for
    from palladium_amd.emit.core import emit_hip, launch_geometry

    nx, n = 6, 256
    x = np.random.default_rng(5).uniform(0.0, 1.0, n).astype(np.float32)
    s = pl.BlockSpec((1,), lambda i: (i,))
    shapes = (pl.ShapeDtypeStruct((n,), np.float32),) + (pl.ShapeDtypeStruct((n,), np.int32),) * 3 \
        + (pl.ShapeDtypeStruct((n,), np.float32),) * nx
    call = pl.pallas_call(_boundary_kernel(nx), grid=(n,), in_specs=[s], out_specs=(s,) * (4 + nx),
                          out_shape=shapes)
    spec = trace(call, x)
    assert plan_for(spec, spec.jaxpr, 1, None) is None
    assert plan_for(spec, fold_counters(spec.jaxpr), 1, None) is not None
    assert launch_geometry(spec).block != 1024
    for mode in ("safe", "relaxed", "fast"):
        src = emit_hip(spec, math_mode=mode)
        assert "__shared__" not in src
    ref = interpret_spec(spec, [x])
    assert int(np.sum(ref[1]) + np.sum(ref[2])) == int(np.sum(ref[3]))
