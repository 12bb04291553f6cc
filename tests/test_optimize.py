"""FAST-only jaxpr rewrite `factor_common_products` (CPU, interpreter)."""

import dataclasses

import numpy as np
import pytest

from palladium_amd.emit import emit_hip
from palladium_amd.emit.optimize import factor_common_products
from palladium_amd.frontend import jnp, lax, pl
from palladium_amd.interpret import interpret_spec
from palladium_amd.trace import trace
from palladium_amd.workloads import (
    BS3Config,
    bs3_inputs,
    bs3_vdp_call,
    gray_scott_call,
    gray_scott_initial,
    lv_inputs,
    lv_rk4_call,
)


def _count(jaxpr, name):
    n = 0
    for e in jaxpr.eqns:
        n += e.primitive.name == name
        for v in e.params.values():
            sub = getattr(v, "jaxpr", v)
            if hasattr(sub, "eqns"):
                n += _count(sub, name)
    return n


def _rewritten(spec):
    return dataclasses.replace(spec, jaxpr=factor_common_products(spec.jaxpr))


def test_lv_rhs_is_factored_and_agrees_within_rounding():
    args = lv_inputs(2000, 3)
    spec = trace(lv_rk4_call(2000, 0.01, 100, track_max=True)._staged, *args)
    opt = _rewritten(spec)
    # Two products per rhs component and four rhs evaluations: one mul saved
    # per component per stage.
    assert _count(opt.jaxpr, "mul") == _count(spec.jaxpr, "mul") - 8
    want = interpret_spec(spec, *args)
    got = interpret_spec(opt, *args)
    for g, w in zip(got, want):
        np.testing.assert_allclose(g, w, rtol=2e-5)


def test_rewrite_keeps_multi_use_products():
    def kernel(a_ref, x_ref, o_ref, p_ref):
        a = a_ref[...]
        x = x_ref[...]
        ax = a * x
        o_ref[...] = ax - x * x
        p_ref[...] = ax  # second use: ax must survive

    a = np.linspace(1, 2, 64, dtype=np.float32)
    x = np.linspace(-1, 3, 64, dtype=np.float32)
    call = pl.pallas_call(kernel, out_shape=(pl.ShapeDtypeStruct((64,), np.float32),) * 2)
    spec = trace(call, a, x)
    opt = _rewritten(spec)
    assert _count(opt.jaxpr, "mul") == _count(spec.jaxpr, "mul")
    for g, w in zip(interpret_spec(opt, a, x), interpret_spec(spec, a, x)):
        np.testing.assert_array_equal(g, w)


def test_rewrite_factors_literal_and_var_chains():
    def kernel(x_ref, y_ref, o_ref):
        x = x_ref[...]
        y = y_ref[...]
        o_ref[...] = (2.0 * x) * y + (3.0 * y) * x

    x = np.linspace(1, 2, 64, dtype=np.float32)
    y = np.linspace(-1, 3, 64, dtype=np.float32)
    call = pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((64,), np.float32))
    spec = trace(call, x, y)
    opt = _rewritten(spec)
    assert _count(opt.jaxpr, "mul") == _count(spec.jaxpr, "mul") - 1
    np.testing.assert_allclose(interpret_spec(opt, x, y)[0], 5 * x * y, rtol=1e-6)


def test_integer_arithmetic_is_untouched():
    def kernel(x_ref, o_ref):
        x = x_ref[...]
        o_ref[...] = x * 3 - x * 5

    x = np.arange(64, dtype=np.int32)
    call = pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((64,), np.int32))
    spec = trace(call, x)
    assert _count(_rewritten(spec).jaxpr, "mul") == _count(spec.jaxpr, "mul")


def test_gray_scott_and_bs3_agree_after_rewrite():
    u0, v0 = gray_scott_initial(32)
    spec = trace(gray_scott_call(size=32)._staged, u0, v0)
    opt = _rewritten(spec)
    for g, w in zip(interpret_spec(opt, u0, v0), interpret_spec(spec, u0, v0)):
        np.testing.assert_allclose(g, w, rtol=1e-5, atol=1e-6)
    cfg = dataclasses.replace(BS3Config(), n=128, t1=2.0)
    args = bs3_inputs(128)
    spec = trace(bs3_vdp_call(128, cfg)._staged, *args)
    opt = _rewritten(spec)
    got = interpret_spec(opt, *args)
    want = interpret_spec(spec, *args)
    np.testing.assert_allclose(got[0], want[0], rtol=1e-3, atol=1e-4)


def test_emitter_applies_rewrite_only_under_fast(monkeypatch):
    # the common-factor rewrite alone: the affine-shift reuse trades a
    # product of the shifted state for a product of the shift
    monkeypatch.setenv("PALLADIUM_AFFINE_SHIFTS", "0")
    args = lv_inputs(256, 0)
    spec = trace(lv_rk4_call(256, 0.01, 10)._staged, *args)
    safe = emit_hip(spec, math_mode="safe")
    fast = emit_hip(spec, math_mode="fast")
    assert safe == emit_hip(spec)
    assert fast.count(" * ") < safe.count(" * ")


def _poly_kernel(seed):
    """A random branch-free sum of signed products over three inputs and
    literals: the shape the common-factor rewrite targets, at random."""
    def kernel(x_ref, y_ref, z_ref, o_ref, s_ref):
        r = np.random.default_rng(seed)
        leaves = [x_ref[...], y_ref[...], z_ref[...]]

        def product():
            p = leaves[r.integers(3)]
            for _ in range(r.integers(0, 3)):
                p = p * (leaves[r.integers(3)] if r.random() < 0.7 else float(np.float32(r.uniform(0.5, 2))))
            return p

        acc = product()
        for _ in range(r.integers(1, 6)):
            acc = acc + product() if r.random() < 0.5 else acc - product()
        o_ref[...] = acc
        # Magnitude bound: the same terms, all added in absolute value.
        r = np.random.default_rng(seed)
        leaves = [jnp.abs(v) for v in leaves]
        mag = product()
        for _ in range(r.integers(1, 6)):
            r.random()
            mag = mag + product()
        s_ref[...] = mag

    return kernel


@pytest.mark.parametrize("seed", range(40))
def test_rewrite_fuzz_random_sums_of_products(seed):
    rng = np.random.default_rng(seed)
    args = [rng.uniform(-2, 2, 64).astype(np.float32) for _ in range(3)]
    call = pl.pallas_call(_poly_kernel(seed), out_shape=(pl.ShapeDtypeStruct((64,), np.float32),) * 2)
    spec = trace(call, *args)
    want, mag = interpret_spec(spec, *args)
    got, _ = interpret_spec(_rewritten(spec), *args)
    # Reassociation moves each result by a few float32 ulps of the terms.
    assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-5 * (mag.astype(np.float64) + 1e-30))


def test_rewrite_fuzz_is_not_vacuous():
    fired = 0
    for seed in range(40):
        spec = trace(pl.pallas_call(_poly_kernel(seed), out_shape=(pl.ShapeDtypeStruct((64,), np.float32),) * 2),
                     *[np.zeros(64, np.float32)] * 3)
        fired += _count(_rewritten(spec).jaxpr, "mul") < _count(spec.jaxpr, "mul")
    assert fired >= 10


# ---------------------------------------------------------------------------
# power-law rewrite: pow by non-integer literals -> exp2 of a sum of log2s

from palladium_amd.emit.optimize import power_laws_to_exp2  # noqa: E402


def _pl(spec):
    return dataclasses.replace(spec, jaxpr=power_laws_to_exp2(spec.jaxpr))


def test_bs3_controller_becomes_one_exp2():
    cfg = dataclasses.replace(BS3Config(), n=128, t1=2.0)
    args = bs3_inputs(128)
    spec = trace(bs3_vdp_call(128, cfg)._staged, *args)
    opt = _pl(spec)
    assert _count(spec.jaxpr, "pow") == 2
    assert _count(opt.jaxpr, "pow") == 0
    assert _count(opt.jaxpr, "exp2") == 1        # both powers and the safety factor in one exp2
    assert _count(opt.jaxpr, "log2") == 2        # log2(err) on the chain, log2(prev) off it
    # no -inf guard: prev starts at 1 and is only ever replaced by 1/max(err, 1e-9)
    assert _count(opt.jaxpr, "select_n") == _count(spec.jaxpr, "select_n")
    assert _count(opt.jaxpr, "div") == _count(spec.jaxpr, "div")  # 1/err still feeds the carry
    got = interpret_spec(opt, *args)
    want = interpret_spec(spec, *args)
    np.testing.assert_allclose(got[0], want[0], rtol=1e-5)
    np.testing.assert_allclose(got[1], want[1], rtol=1e-3, atol=1e-4)
    # accept/reject decisions near err = 1 may flip and shift a lane's
    # count by a few attempts; the totals stay put
    assert np.all(np.abs(got[3].astype(int) - want[3]) <= 0.1 * want[3] + 5)
    assert abs(int(got[3].sum()) - int(want[3].sum())) <= 0.02 * want[3].sum()


def _power_kernel(c1, c2, k):
    def kernel(x_ref, y_ref, o_ref, p_ref):
        x, y = x_ref[...], y_ref[...]
        o_ref[...] = k * (1.0 / x) ** c1 * y ** c2
        p_ref[...] = x ** c1
    return kernel


def test_power_law_rewrite_special_operands():
    """pow(x, c) for non-integer c and exp2(c log2 x) agree on zeros,
    infinities, NaN and negative bases. (Finite bases stay where no single
    power overflows: a product whose factors overflow and underflow is
    finite in the fused form, as reassociation allows.)"""
    vals = np.array([0.0, -0.0, np.inf, 1.0, 2.0, 0.5, 1e-3, 3e3, -1.0, -np.inf, np.nan, 7.0], np.float32)
    x, y = np.meshgrid(vals, vals)
    x, y = x.ravel().copy(), y.ravel().copy()
    n = x.size
    for c1, c2, k in ((0.2333, -0.1333, 0.9), (1.5, 0.5, 2.0), (-0.7, 2.5, 1.0)):
        call = pl.pallas_call(_power_kernel(c1, c2, k), out_shape=(pl.ShapeDtypeStruct((n,), np.float32),) * 2)
        spec = trace(call, x, y)
        opt = _pl(spec)
        assert _count(opt.jaxpr, "pow") == 0
        for g, w in zip(interpret_spec(opt, x, y), interpret_spec(spec, x, y)):
            same_class = (np.isnan(g) == np.isnan(w)) & (np.isinf(g) == np.isinf(w)) & ((g == 0) == (w == 0))
            ok = same_class
            assert ok.all(), (c1, c2, x[~ok], y[~ok], g[~ok], w[~ok])
            fin = np.isfinite(w) & (w != 0) & (np.abs(w) < 1e37) & (np.abs(w) > 1e-37)
            np.testing.assert_allclose(g[fin], w[fin], rtol=5e-6)


def test_power_law_rewrite_leaves_integer_exponents_and_shared_values():
    def kernel(x_ref, o_ref, p_ref):
        x = x_ref[...]
        q = x ** 0.5
        o_ref[...] = x ** 2.0 * q      # integer power untouched
        p_ref[...] = q                  # q has a second use: the product keeps its own exp2

    x = np.linspace(-2, 2, 64, dtype=np.float32)
    spec = trace(pl.pallas_call(kernel, out_shape=(pl.ShapeDtypeStruct((64,), np.float32),) * 2), x)
    opt = _pl(spec)
    assert _count(opt.jaxpr, "pow") == 1
    assert _count(opt.jaxpr, "exp2") == 1
    for g, w in zip(interpret_spec(opt, x), interpret_spec(spec, x)):
        np.testing.assert_allclose(g, w, rtol=5e-6)


# ---------------------------------------------------------------------------
# redundant clamps: jax.random.uniform's max(minval, .) after the bit trick

from palladium_amd.emit.optimize import drop_redundant_clamps  # noqa: E402
from palladium_amd.frontend import random  # noqa: E402


@pytest.mark.parametrize("lo,hi", [(0.0, 1.0), (-3.0, 5.0), (1e-7, 2.0), (2.5, 2.5000002)])
def test_uniform_clamp_is_dropped_and_results_unchanged(lo, hi):
    def kernel(b_ref, o_ref, p_ref):
        b = b_ref[...]
        o_ref[...] = random.bits_to_uniform(b, lo, hi)
        p_ref[...] = jnp.maximum(random.bits_to_uniform(b, lo, hi), hi)  # acts on every value: kept

    edge = np.array([0, 1, 511, 512, 0x7FFFFFFF, 0x80000000, 0xFFFFFE00, 0xFFFFFFFF], np.uint32)
    b = np.concatenate([edge, np.random.default_rng(1).integers(0, 2**32, 4088, dtype=np.uint64).astype(np.uint32)])
    call = pl.pallas_call(kernel, out_shape=(pl.ShapeDtypeStruct((b.size,), np.float32),) * 2)
    spec = trace(call, b)
    opt = dataclasses.replace(spec, jaxpr=drop_redundant_clamps(spec.jaxpr))
    assert _count(spec.jaxpr, "max") == 3
    assert _count(opt.jaxpr, "max") == 1  # both uniforms' clamps go, the one that can act stays
    for g, w in zip(interpret_spec(opt, b), interpret_spec(spec, b)):
        np.testing.assert_array_equal(g, w)


def test_carry_that_can_turn_negative_keeps_the_guard():
    def kernel(x_ref, o_ref, p_ref):
        x = x_ref[...]

        def body(c):
            k, a, b = c
            return k + 1, a * 0.5 + 0.25, b - 0.75     # a stays >= 0, b goes negative

        _, a, b = lax.while_loop(lambda c: c[0] < 4, body, (jnp.int32(0), jnp.abs(x), jnp.abs(x)))
        o_ref[...] = a ** 0.3 + b ** 0.7

    x = np.linspace(-2, 2, 64, dtype=np.float32)
    call = pl.pallas_call(kernel, grid=(64,), in_specs=[pl.BlockSpec((1,), lambda i: (i,))],
                          out_specs=(pl.BlockSpec((1,), lambda i: (i,)),) * 2,
                          out_shape=(pl.ShapeDtypeStruct((64,), np.float32),) * 2)
    spec = trace(call, x)
    opt = _pl(spec)
    assert _count(opt.jaxpr, "pow") == 0
    # only b's power gets the -inf guard (one eq + one select); a's is proven
    assert _count(opt.jaxpr, "select_n") == _count(spec.jaxpr, "select_n") + 1
    for g, w in zip(interpret_spec(opt, x), interpret_spec(spec, x)):
        np.testing.assert_allclose(g, w, rtol=5e-6)


def test_bs3_prev_carry_becomes_its_log():
    from palladium_amd.emit.optimize import carry_logs, power_laws_to_exp2

    cfg = dataclasses.replace(BS3Config(), n=128, t1=2.0)
    args = bs3_inputs(128)
    spec = trace(bs3_vdp_call(128, cfg)._staged, *args)
    pl_only = power_laws_to_exp2(spec.jaxpr)
    opt = carry_logs(pl_only)
    (w0,) = [e for e in pl_only.eqns if e.primitive.name == "while"]
    (w,) = [e for e in opt.eqns if e.primitive.name == "while"]
    body0, body = w0.params["body_jaxpr"].jaxpr, w.params["body_jaxpr"].jaxpr
    assert _count(body0, "log2") == 2 and _count(body, "log2") == 1
    assert _count(body, "neg") == 1                      # log2(1 / err) = -log2(err)
    assert len(w.invars) == len(w0.invars)               # the carry is replaced, not added
    assert _count(opt, "log2") == 2                      # + log2 of the initial prev, before the loop
    got = interpret_spec(dataclasses.replace(spec, jaxpr=opt), *args)
    want = interpret_spec(dataclasses.replace(spec, jaxpr=pl_only), *args)
    np.testing.assert_allclose(got[0], want[0], rtol=1e-5)
    np.testing.assert_allclose(got[1], want[1], rtol=1e-3, atol=1e-4)
    # log2(1/err) and -log2(err) round differently; the controller is chaotic
    # on a few lanes (up to 14 % more or fewer attempts here), the totals not
    assert np.all(np.abs(got[3].astype(int) - want[3]) <= 0.2 * want[3] + 5)
    assert abs(int(got[3].sum()) - int(want[3].sum())) <= 0.01 * want[3].sum()


@pytest.mark.parametrize("read_after", [True, False])
def test_carry_read_elsewhere_is_kept(read_after):
    from palladium_amd.emit.optimize import carry_logs, power_laws_to_exp2

    def kernel(x_ref, o_ref, p_ref):
        x = x_ref[...]

        def body(s):
            k, c = s
            v = 1.0 / (jnp.abs(x + k.astype(jnp.float32)) + 1.0)
            f = v ** 0.3 * c ** 0.2                   # log2(v), log2(c) after the power-law rewrite
            return k + 1, jnp.where(f < 0.5, v, c)

        _, c = lax.while_loop(lambda s: s[0] < 4, body, (jnp.int32(0), jnp.abs(x) + 1.0))
        o_ref[...] = c if read_after else x   # read after the loop: must stay the value, not its log
        p_ref[...] = x

    x = np.linspace(-2, 2, 64, dtype=np.float32)
    s = pl.BlockSpec((1,), lambda i: (i,))
    call = pl.pallas_call(kernel, grid=(64,), in_specs=[s], out_specs=(s, s),
                          out_shape=(pl.ShapeDtypeStruct((64,), np.float32),) * 2)
    spec = trace(call, x)
    j = power_laws_to_exp2(spec.jaxpr)
    assert _count(j, "log2") == 2 and _count(j, "eq") == 0   # c and v proven non-negative: no guards
    assert (carry_logs(j).eqns == j.eqns) == read_after


def _funnel_kernel(n, c, signed):
    def kernel(x_ref, o_ref):
        x = x_ref[...]
        o_ref[...] = lax.shift_right_logical(x, jnp.asarray(n, x.dtype)) | jnp.asarray(c, x.dtype)
    return kernel


def _funnel_spec(n, c, signed, size=256):
    dt = np.int32 if signed else np.uint32
    x = np.random.default_rng(n).integers(0, 2 ** 32, size, dtype=np.uint64).astype(np.uint32).view(dt)
    s = pl.BlockSpec((1,), lambda i: (i,))
    call = pl.pallas_call(_funnel_kernel(n, np.uint32(c).view(dt), signed), grid=(size,), in_specs=[s], out_specs=s,
                          out_shape=pl.ShapeDtypeStruct((size,), dt))
    return trace(call, x), x


@pytest.mark.parametrize("n,c,signed,rewritten", [
    (9, 0x3F800000, False, True),          # jax.random.uniform's float32 construction
    (9, 0x3F800000, True, True),
    (20, 0xABC00000, False, True),
    (9, 0x3F800001, False, False),         # a bit below the shifted field: not a funnel shift
    (1, 0x80000000, True, True),
])
def test_or_of_a_logical_shift_becomes_alignbit(n, c, signed, rewritten):
    from palladium_amd.emit.optimize import funnel_shifts

    spec, x = _funnel_spec(n, c, signed)
    opt = funnel_shifts(spec.jaxpr)
    assert (_count(opt, "alignbit") == 1) == rewritten
    if rewritten:
        (e,) = [q for q in opt.eqns if q.primitive.name == "alignbit"]
        hi, amt = int(e.invars[0].val), int(e.invars[2].val)
        xu = x.view(np.uint32).astype(np.uint64)
        # alignbit(hi, lo, s) = low word of ((hi << 32) | lo) >> s
        got = (((np.uint64(hi) << np.uint64(32)) | xu) >> np.uint64(amt)) & np.uint64(0xFFFFFFFF)
        want = (xu >> np.uint64(n)) | np.uint64(c)
        np.testing.assert_array_equal(got, want)


def test_carry_returned_as_another_carry_is_kept():
    """`prev` also becomes the next value of a second carry: it is read as a
    value there, so it must not turn into its log."""
    from palladium_amd.emit.optimize import carry_logs, power_laws_to_exp2

    def kernel(x_ref, o_ref):
        x = x_ref[...]

        def body(s):
            k, c, d = s
            v = 1.0 / (jnp.abs(x + k.astype(jnp.float32)) + 1.0)
            f = v ** 0.3 * c ** 0.2
            return k + 1, jnp.where(f < 0.5, v, c), c        # d' = c
        _, c, d = lax.while_loop(lambda s: s[0] < 4, body, (jnp.int32(0), jnp.abs(x) + 1.0, jnp.abs(x)))
        o_ref[...] = d

    x = np.linspace(-2, 2, 64, dtype=np.float32)
    s = pl.BlockSpec((1,), lambda i: (i,))
    call = pl.pallas_call(kernel, grid=(64,), in_specs=[s], out_specs=s,
                          out_shape=pl.ShapeDtypeStruct((64,), np.float32))
    spec = trace(call, x)
    j = power_laws_to_exp2(spec.jaxpr)
    assert carry_logs(j).eqns == j.eqns
    got = interpret_spec(dataclasses.replace(spec, jaxpr=carry_logs(j)), x)[0]
    np.testing.assert_array_equal(got, interpret_spec(dataclasses.replace(spec, jaxpr=j), x)[0])


from palladium_amd.emit.optimize import reuse_affine_shifts  # noqa: E402


def _shift_kernel(h, reorder=False):
    """One explicit stage of the LV right-hand side at y and at y + h k."""
    def kernel(x_ref, y_ref, a_ref, b_ref, o_ref, p_ref):
        x, y, a, b = x_ref[...], y_ref[...], a_ref[...], b_ref[...]
        f0 = a - b * y              # the unshifted value
        g0 = b * x - a
        k, j = x * f0, y * g0
        y2 = (y + h * k) if not reorder else (k * h + y)
        x2 = x + h * j
        o_ref[...] = x2 * (a - b * y2)
        p_ref[...] = y2 * ((x2 * b if reorder else b * x2) - a)
    return kernel


def _shift_spec(h, x, y, a, b, reorder=False):
    s = pl.BlockSpec((1,), lambda i: (i,))
    call = pl.pallas_call(_shift_kernel(h, reorder), grid=(x.size,), in_specs=[s] * 4, out_specs=(s, s),
                          out_shape=(pl.ShapeDtypeStruct(x.shape, np.float32),) * 2)
    return trace(call, x, y, a, b)


@pytest.mark.parametrize("reorder", [False, True])
def test_affine_shift_reuse_is_exact_where_arithmetic_is(reorder):
    # small integers and h = 1/2: every product and sum is exact in float32,
    # so the reassociated form must agree bit for bit; a dropped term, a
    # wrong sign or the wrong base value would not
    r = np.random.default_rng(3)
    x, y, a, b = (r.integers(-8, 9, 256).astype(np.float32) for _ in range(4))
    spec = _shift_spec(0.5, x, y, a, b, reorder)
    opt = dataclasses.replace(spec, jaxpr=reuse_affine_shifts(spec.jaxpr))
    # both shifted right-hand sides now start from the unshifted ones
    subs = [e for e in opt.jaxpr.eqns if e.primitive.name in ("sub", "add")]
    assert _count(opt.jaxpr, "sub") == _count(spec.jaxpr, "sub") - 1
    assert _count(opt.jaxpr, "mul") == _count(spec.jaxpr, "mul") + 2     # b h, c h and their uses; 2 dead gone
    assert len(subs) == len([e for e in spec.jaxpr.eqns if e.primitive.name in ("sub", "add")])
    for g, w in zip(interpret_spec(opt, x, y, a, b), interpret_spec(spec, x, y, a, b)):
        np.testing.assert_array_equal(g, w)
    # and against the closed form evaluated in float64
    xf, yf, af, bf = (v.astype(np.float64) for v in (x, y, a, b))
    y2 = yf + 0.5 * xf * (af - bf * yf)
    x2 = xf + 0.5 * yf * (bf * xf - af)
    got = interpret_spec(opt, x, y, a, b)
    np.testing.assert_array_equal(got[0], (x2 * (af - bf * y2)).astype(np.float32))
    np.testing.assert_array_equal(got[1], (y2 * (bf * x2 - af)).astype(np.float32))


def test_affine_shift_needs_the_unshifted_value():
    def kernel(y_ref, a_ref, b_ref, k_ref, o_ref):
        y, a, b, k = y_ref[...], a_ref[...], b_ref[...], k_ref[...]
        o_ref[...] = a - b * (y + 0.5 * k)      # a - b y never computed: nothing to reuse

    v = np.linspace(1, 2, 64, dtype=np.float32)
    call = pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((64,), np.float32))
    spec = trace(call, v, v, v, v)
    assert reuse_affine_shifts(spec.jaxpr).eqns == spec.jaxpr.eqns


def test_affine_shift_reuse_on_lv_rk4_within_fast_tolerance():
    args = lv_inputs(512, 1)
    spec = trace(lv_rk4_call(512, 0.005, 400)._staged, *args)
    # the traced x a - b x y becomes x (a - b y) under the common-factor rewrite first
    fac = factor_common_products(spec.jaxpr)
    opt = dataclasses.replace(spec, jaxpr=reuse_affine_shifts(fac))
    assert opt.jaxpr.eqns != fac.eqns
    for g, w in zip(interpret_spec(opt, *args), interpret_spec(spec, *args)):
        np.testing.assert_allclose(g, w, rtol=2e-5, atol=1e-6)


def test_affine_shift_needs_the_same_coefficient_and_offset():
    def kernel(x_ref, y_ref, a_ref, b_ref, o_ref, p_ref):
        x, y, a, b = x_ref[...], y_ref[...], a_ref[...], b_ref[...]
        f0 = a - b * y                          # a - b y exists ...
        k = x * f0
        o_ref[...] = (a + 1.0) - b * (y + 0.5 * k)   # ... but this offset differs
        p_ref[...] = a - x * (y + 0.5 * k)           # ... and this coefficient

    v = np.linspace(1, 2, 64, dtype=np.float32)
    s = pl.BlockSpec((1,), lambda i: (i,))
    call = pl.pallas_call(kernel, grid=(64,), in_specs=[s] * 4, out_specs=(s, s),
                          out_shape=(pl.ShapeDtypeStruct((64,), np.float32),) * 2)
    spec = trace(call, v, v, v, v)
    assert reuse_affine_shifts(spec.jaxpr).eqns == spec.jaxpr.eqns


from palladium_amd.emit.optimize import drop_dead_code  # noqa: E402


def test_dead_code_is_dropped_stores_and_loop_carries_kept():
    """An unread pure value goes, at the top level and inside a loop body;
    stores, loops and every value a result reads stay, and the results are
    unchanged."""

    def kernel(x_ref, o_ref, p_ref):
        x = x_ref[...]
        unused = jnp.exp(x) * 3.0  # noqa: F841 - read by nothing

        def body(i, c):
            dead = c / (c + 1.0)  # noqa: F841 - read by nothing
            return c * 0.5 + x

        o_ref[...] = lax.fori_loop(0, 8, body, x)
        p_ref[...] = x + 1.0

    x = np.linspace(0.5, 2.0, 64, dtype=np.float32)
    s = pl.BlockSpec((1,), lambda i: (i,))
    call = pl.pallas_call(kernel, grid=(64,), in_specs=[s], out_specs=[s, s],
                          out_shape=(pl.ShapeDtypeStruct((64,), np.float32),) * 2)
    spec = trace(call, x)
    pruned = dataclasses.replace(spec, jaxpr=drop_dead_code(spec.jaxpr))
    assert _count(spec.jaxpr, "exp") == 1 and _count(pruned.jaxpr, "exp") == 0
    assert _count(spec.jaxpr, "div") == 1 and _count(pruned.jaxpr, "div") == 0
    assert _count(pruned.jaxpr, "swap") == _count(spec.jaxpr, "swap") == 2
    assert _count(pruned.jaxpr, "scan") + _count(pruned.jaxpr, "while") == 1
    for g, w in zip(interpret_spec(pruned, x), interpret_spec(spec, x)):
        np.testing.assert_array_equal(g, w)
    src = emit_hip(spec, math_mode="safe")
    body = src[src.index('extern "C"'):]
    assert "expf" not in body and "ph_exp(" not in body
