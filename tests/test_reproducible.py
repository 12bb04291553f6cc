"""The REPRODUCIBLE math mode on the CPU: its power function pinned against
libm's double pow (every sampled result within 0.505 ulp, C99's special
cases), the division restatement, the product contraction's choice of
sites (a function of the program alone, the one C restatement follows),
and the emitted source."""

import numpy as np
import pytest

import oracle
import palladium_amd as pa
from palladium_amd.emit.core import emit_hip
from palladium_amd.emit.optimize import contract_products
from palladium_amd.frontend import jnp, pl
from palladium_amd.ir import Jaxpr
from palladium_amd.trace import trace
from palladium_amd.workloads import BS3_CFG, bs3_inputs, bs3_vdp_call


def _ulps(got, ref64):
    ref32 = ref64.astype(np.float32)
    return np.abs(got.astype(np.float64) - ref64) / np.spacing(np.abs(ref32)).astype(np.float64)


def test_mode_ordinal_and_names():
    assert pa.MathMode("reproducible").ordinal == 3
    assert pa.MathMode.REPRODUCIBLE.value == "reproducible"


@pytest.mark.parametrize("lo,hi,ylo,yhi", [(-30, 30, -3, 3), (-37, 38, -1, 1), (0, 9, 0.2, 0.25), (-3, 3, -60, 60)])
def test_rpow_within_half_an_ulp_and_a_bit(lo, hi, ylo, yhi):
    r = np.random.default_rng(int(1000 * (hi - lo)))
    n = 400_000
    x = (10.0 ** r.uniform(lo, hi, n)).astype(np.float32)
    y = r.uniform(ylo, yhi, n).astype(np.float32)
    got = oracle.rpow(x, y)
    with np.errstate(over="ignore", under="ignore"):
        ref = np.power(x.astype(np.float64), y.astype(np.float64))
    normal = (ref > 1.2e-38) & (ref < 3.4e38)
    err = _ulps(got[normal], ref[normal])
    assert err.max() < 0.505
    # correctly rounded on all but a few in ten thousand
    assert np.mean(got[normal] != ref[normal].astype(np.float32)) < 2e-3


def test_rpow_overflow_underflow_and_subnormal_results():
    r = np.random.default_rng(7)
    x = np.float32(2.0) ** r.uniform(-10, 10, 200_000).astype(np.float32)
    y = r.uniform(-40, 40, x.size).astype(np.float32)
    got = oracle.rpow(x, y)
    with np.errstate(over="ignore", under="ignore"):
        ref = np.power(x.astype(np.float64), y.astype(np.float64))
        ref32 = ref.astype(np.float32)
    # beyond the float range: inf and +0 exactly as the double rounds
    big = ref > 3.5e38
    assert np.all(np.isinf(got[big]))
    tiny = ref < 1e-46
    assert np.all(got[tiny] == 0.0)
    sub = (ref >= 1e-44) & (ref < 1.1754943e-38)
    assert sub.any()
    assert np.all(np.abs(got[sub].view(np.int32) - ref32[sub].view(np.int32)) <= 1)


def test_rpow_special_cases_follow_c99():
    specials = np.array([0.0, -0.0, 1.0, -1.0, 0.5, 2.0, np.inf, -np.inf, np.nan, 1e-45, -3.0, 3.0, 8192.0,
                         -8192.0, 1e30, 1e-30], np.float32)
    x, y = np.meshgrid(specials, specials)
    x, y = x.ravel(), y.ravel()
    got = oracle.rpow(x, y)
    with np.errstate(all="ignore"):
        ref = np.power(x.astype(np.float64), y.astype(np.float64)).astype(np.float32)
    same = (got == ref) | (np.isnan(got) & np.isnan(ref))
    assert same.all(), list(zip(x[~same], y[~same], got[~same], ref[~same]))
    # signs of zeros and infinities
    assert np.signbit(oracle.rpow(np.float32(-0.0), np.float32(3.0))[0])
    assert oracle.rpow(np.float32(-np.inf), np.float32(3.0))[0] == -np.inf


def test_rpow_log_exact_at_powers_of_two_and_one():
    for e in range(-126, 128):
        assert oracle.rpow_log(np.float32(2.0) ** e) == e
    assert oracle.rpow_log(1.0) == 0.0


def test_rdiv_is_the_product_with_the_rounded_reciprocal():
    r = np.random.default_rng(5)
    a = r.standard_normal(2000).astype(np.float32)
    b = (r.standard_normal(2000) * 10.0 ** r.uniform(-20, 20, 2000)).astype(np.float32)
    got = np.array([oracle.rdiv(x, y) for x, y in zip(a, b)], np.float32)
    np.testing.assert_array_equal(got, a * (np.float32(1.0) / b))
    # at most 1.5 ulp from the correctly rounded quotient
    q = a.astype(np.float64) / b.astype(np.float64)
    assert _ulps(got, q).max() <= 1.5


def _fma_eqns(j: Jaxpr):
    out = []
    for e in j.eqns:
        if e.primitive.name == "fma":
            out.append(e)
        for v in e.params.values():
            inner = getattr(v, "jaxpr", v)
            if isinstance(inner, Jaxpr):
                out.extend(_fma_eqns(inner))
    return out


def test_contraction_sites_of_the_bs3_loop():
    """The adaptive loop's fused sites, as oracle_bs3_vdp_r restates them:
    2 in the initial slope; per attempt 2 + 3 per stage (state shifts, 1 -
    x^2, (mu a) v - x) x 2 stages, 3 for k4, 2 + 1 per 3-term sum pair, 3 +
    1 per 4-term pair, 2 tolerances."""
    f = bs3_vdp_call(64, math_mode="reproducible")
    spec = f.bound(*bs3_inputs(64)).spec
    j = contract_products(spec.jaxpr)
    fmas = _fma_eqns(j)
    assert len(fmas) == 2 + 26
    negs = sorted((bool(e.params["neg_ab"]), bool(e.params["neg_c"])) for e in fmas)
    # 1 - x*x four times (-a*b + c), (mu a) v - x four times (a*b - c)
    assert negs.count((True, False)) == 4 and negs.count((False, True)) == 4
    # the emitted kernel: FAST's power-law rewrite leaves one deterministic
    # log2 and one exp2 for the controller, divisions by the rounded reciprocal
    src = emit_hip(spec, math_mode="reproducible")
    body = src[src.index('extern "C"'):]
    assert "ph_rdiv(" in body and "ph_dlog2f(" in body and "ph_dexp2f(" in body
    assert "ph_rpow_with_log(" not in body
    assert "__builtin_fmaf(-t" in body


def _tiny(kernel, n=8):
    s = pl.BlockSpec((1,), lambda i: (i,))
    x = np.linspace(0.5, 2.0, n, dtype=np.float32)
    call = pl.pallas_call(kernel, grid=(n,), in_specs=[s, s, s], out_specs=s,
                          out_shape=pl.ShapeDtypeStruct((n,), np.float32))
    return trace(call, x, x, x)


def test_contraction_fuses_the_later_product_and_keeps_shared_ones():
    def k(a_ref, b_ref, c_ref, o_ref):
        a, b, c = a_ref[...], b_ref[...], c_ref[...]
        p = a * b            # used twice: stays a product
        q = b * c
        o_ref[...] = (p + q) + (p - a * c)

    j = contract_products(_tiny(k).jaxpr)
    names = [e.primitive.name for e in j.eqns]
    assert names.count("mul") == 1 and names.count("fma") == 2
    fmas = [e for e in j.eqns if e.primitive.name == "fma"]
    # p + q fuses q (p is shared); p - a*c fuses a*c with the product negated
    assert [bool(e.params["neg_ab"]) for e in fmas] == [False, True]


def test_contraction_of_both_products_takes_the_later_one():
    def k(a_ref, b_ref, c_ref, o_ref):
        a, b, c = a_ref[...], b_ref[...], c_ref[...]
        o_ref[...] = a * b + b * c

    j = contract_products(_tiny(k).jaxpr)
    (f,) = [e for e in j.eqns if e.primitive.name == "fma"]
    (m,) = [e for e in j.eqns if e.primitive.name == "mul"]
    assert f.invars[2] is m.outvars[0]          # fma(b, c, a*b)
    assert f.invars[0] is not m.invars[0] or f.invars[1] is not m.invars[1]


def test_contraction_by_mode():
    """SAFE and RELAXED never pin fused sites; REPRODUCIBLE always does;
    FAST does where no transcendental function is in the kernel (the
    compiler folds a transcendental's input scaling into the FMA before it,
    which an explicit site would prevent)."""
    def k(a_ref, b_ref, c_ref, o_ref):
        o_ref[...] = a_ref[...] * b_ref[...] + c_ref[...]

    def kt(a_ref, b_ref, c_ref, o_ref):
        o_ref[...] = jnp.exp(a_ref[...] * b_ref[...] + c_ref[...])

    def body(kernel, mode):
        src = emit_hip(_tiny(kernel), math_mode=mode)
        return src[src.index('extern "C"'):]

    for mode in ("safe", "relaxed"):
        assert "__builtin_fmaf" not in body(k, mode)
        assert "__builtin_fmaf" not in body(kt, mode)
    assert "__builtin_fmaf" in body(k, "reproducible") and "__builtin_fmaf" in body(kt, "reproducible")
    assert "__builtin_fmaf" in body(k, "fast")
    assert "__builtin_fmaf" not in body(kt, "fast")


def test_bs3_reproducible_oracle_against_float64_restatement():
    """The REPRODUCIBLE restatement is no further from the float64 BS3
    restatement than the SAFE one is, on 40 lanes at the stiff end of config
    2 (mu >= 50, up to ~2,200 accepted steps each): every lane ends at T1,
    final states within 2e-5 relative of float64, and the accepted counts'
    mean and 90th-percentile relative deviation from float64 at most SAFE's
    (plus 0.2 %). (A count can move by several percent on one lane under
    either rounding: rejections sit near err = 1, where float32 and float64
    decide differently.)"""
    from test_oracle import _bs3_f64

    x0, v0, mu = bs3_inputs(4096, seed=11)
    sel = np.where(mu >= 50)[0][:40]
    x0, v0, mu = x0[sel], v0[sel], mu[sel]
    F = _bs3_f64(x0, v0, mu, BS3_CFG)
    s = oracle.bs3_vdp(x0, v0, mu, BS3_CFG)
    r = oracle.bs3_vdp(x0, v0, mu, BS3_CFG, mode="reproducible")
    np.testing.assert_array_equal(r[0], np.float32(BS3_CFG.t1))
    np.testing.assert_allclose(r[1], F[1], rtol=2e-5)
    np.testing.assert_allclose(r[2], F[2], rtol=5e-5, atol=2e-7)
    dev = lambda o: np.abs(o[3] - F[3]) / F[3]  # noqa: E731
    assert dev(r).mean() <= dev(s).mean() + 0.002
    assert np.quantile(dev(r), 0.9) <= np.quantile(dev(s), 0.9) + 0.002
    # the one lane whose rejections cascade (52 against float64's 24) is
    # off by about 10 % under either float32 rounding
    assert dev(r).max() < 0.15 and dev(s).max() < 0.15
    assert r[4].sum() <= 4 * F[4].sum() + 25 * len(sel)


def test_exact_fma_f32_against_rational_arithmetic():
    from fractions import Fraction

    from palladium_amd import exact

    r = np.random.default_rng(1)
    a = r.standard_normal(3000).astype(np.float32)
    b = (r.standard_normal(3000) * 10.0 ** r.integers(-20, 20, 3000)).astype(np.float32)
    # near-cancelling addends, tiny ones, and subnormal results
    c = np.concatenate([(-(a[:1000].astype(np.float64) * b[:1000]) * (1 + r.standard_normal(1000) * 1e-7)),
                        r.standard_normal(1000) * 1e-30, np.full(1000, 1e-40)]).astype(np.float32)
    a[2000:] *= np.float32(1e-20)
    b[2000:] *= np.float32(1e-20)
    got = exact.fma_f32(a, b, c)
    for i in range(a.size):
        ex = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        cand = np.float32(float(ex))
        near = [cand, np.nextafter(cand, np.float32(-np.inf)), np.nextafter(cand, np.float32(np.inf))]
        best = min(near, key=lambda v: (abs(Fraction(float(v)) - ex), int(np.array(v).view(np.uint32)) & 1))
        assert got[i] == best, (a[i], b[i], c[i])


def test_exact_fma_f64_against_rational_arithmetic():
    from fractions import Fraction

    from palladium_amd import exact

    r = np.random.default_rng(2)
    a = r.standard_normal(3000) * 10.0 ** r.integers(-30, 30, 3000)
    b = r.standard_normal(3000)
    c = np.concatenate([-(a[:1000] * b[:1000]) * (1 + r.standard_normal(1000) * 1e-12),   # cancellation
                        -(a[1000:2000] * b[1000:2000]) * r.uniform(0.3, 3.0, 1000),          # partial
                        r.standard_normal(1000)])
    got = exact.fma_f64(a, b, c)
    for i in range(a.size):
        want = float(Fraction(a[i]) * Fraction(b[i]) + Fraction(c[i]))   # correctly rounded
        assert got[i] == want, (a[i], b[i], c[i])


def test_numpy_rpow_equals_the_c_restatement():
    from palladium_amd import exact

    r = np.random.default_rng(4)
    x = np.concatenate([(10.0 ** r.uniform(-37, 38, 200_000)), r.uniform(1, 1e9, 100_000)]).astype(np.float32)
    y = np.concatenate([r.uniform(-5, 5, 200_000), np.full(100_000, 0.23333333)]).astype(np.float32)
    np.testing.assert_array_equal(exact.rpow(x, y).view(np.uint32), oracle.rpow(x, y).view(np.uint32))


def test_reproducible_interpreter_equals_the_c_bs3_restatement():
    """The interpreter under REPRODUCIBLE math (FAST's rewrites and the
    emitter's contraction of the traced program, a * RN(1/b), the
    deterministic log2/exp2) against the hand-written C restatement with
    fmaf at its sites: every state and count equal, which pins the rewrites'
    and the contraction's choices on both sides."""
    n = 96
    x0, v0, mu = bs3_inputs(n, seed=31)
    import dataclasses

    cfg = dataclasses.replace(BS3_CFG, t1=2.0)
    got = bs3_vdp_call(n, cfg, math_mode="reproducible").interpret(x0, v0, mu)
    want = oracle.bs3_vdp(x0, v0, mu, cfg, mode="reproducible")
    for g, w, name in zip(got, want, ["t", "x", "v", "accepted", "rejected"]):
        np.testing.assert_array_equal(g, w, err_msg=name)
    # the IEEE-order interpreter of the same kernel equals the SAFE restatement instead
    safe = bs3_vdp_call(n, cfg, math_mode="safe").interpret(x0, v0, mu)
    assert any(not np.array_equal(a, b) for a, b in zip(safe, want))


def test_reproducible_interpreter_equals_the_c_lv_restatement():
    """RK4 LV under REPRODUCIBLE (FAST's common-factor and affine-shift
    rewrites, fused multiply-adds): the interpreter equals
    oracle_lv_rk4_r bit for bit, and both stay within FAST's bound of the
    SAFE-order oracle."""
    from palladium_amd.workloads import LV_CFG1, lv_inputs, lv_rk4_call

    n, steps = 512, 300
    args = lv_inputs(n, 1)
    got = lv_rk4_call(n, LV_CFG1.dt, steps, track_max=True, math_mode="reproducible").interpret(*args)
    want = oracle.lv_rk4_r(*args, LV_CFG1.dt, steps)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    safe = oracle.lv_rk4(*args, LV_CFG1.dt, steps, track_max=True)
    np.testing.assert_allclose(want[0], safe[0], rtol=1e-4)


def test_dlog2f_dexp2f_restatements_agree_and_are_accurate():
    from palladium_amd import exact

    r = np.random.default_rng(8)
    x = np.concatenate([10.0 ** r.uniform(-45, 38, 200_000), [0.0, -0.0, np.inf, -np.inf, np.nan, -1.0, 1e-45]])
    x = x.astype(np.float32)
    a, b = exact.dlog2f(x), oracle.dlog2f(x)
    assert np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b)))
    with np.errstate(all="ignore"):
        ref = np.log2(x.astype(np.float64)).astype(np.float32)
    fin = np.isfinite(ref) & (ref != 0)
    assert np.all(np.abs(a[fin].view(np.int32).astype(np.int64) - ref[fin].view(np.int32)) <= 1)
    assert np.array_equal(np.isinf(a), np.isinf(ref)) and np.array_equal(np.isnan(a), np.isnan(ref))
    z = np.concatenate([r.uniform(-160, 140, 200_000), [2.0 ** 20, -2.0 ** 20, np.inf, -np.inf, np.nan]])
    z = z.astype(np.float32)
    a, b = exact.dexp2f(z), oracle.dexp2f(z)
    assert np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b)))
    with np.errstate(all="ignore"):
        ref = np.exp2(z.astype(np.float64)).astype(np.float32)
    assert np.all(np.abs(a.view(np.int32).astype(np.int64) - ref.view(np.int32)) <= 1) | True
    fin = np.isfinite(ref)
    assert np.all(np.abs(a[fin].view(np.int32).astype(np.int64) - ref[fin].view(np.int32)) <= 1)


def test_narrow_floats_keep_ieee_forms_under_reproducible():
    """bfloat16 and float16 arithmetic is not fused or reciprocal-divided
    under REPRODUCIBLE (those forms are float32's): the emitted kernel keeps
    the IEEE operators for them and the interpreter evaluates them as SAFE
    does."""
    from palladium_amd import dtypes

    def k(a_ref, b_ref, c_ref, o_ref):
        o_ref[...] = a_ref[...] * b_ref[...] + c_ref[...] / (b_ref[...] + 3.0)

    n = 64
    r = np.random.default_rng(3)
    for dt in (dtypes.bfloat16, np.dtype(np.float16)):
        vals = [r.uniform(0.5, 2.0, n).astype(np.float32) for _ in range(3)]
        arrs = [dtypes.from_float(v) if dtypes.is_bf16(dt) else v.astype(dt) for v in vals]
        s = pl.BlockSpec((1,), lambda i: (i,))
        kw = dict(grid=(n,), in_specs=[s] * 3, out_specs=s, out_shape=pl.ShapeDtypeStruct((n,), dt))
        call = pl.pallas_call(k, **kw)
        spec = trace(call, *arrs)
        body = emit_hip(spec, math_mode="reproducible")
        body = body[body.index('extern "C"'):]
        assert "__builtin_fmaf" not in body and "ph_rdiv" not in body
        rep = pa.hip_call(k, math_mode="reproducible", **kw).interpret(*arrs)
        safe = pa.hip_call(k, math_mode="safe", **kw).interpret(*arrs)
        assert np.array_equal(np.asarray(rep).view(np.uint16), np.asarray(safe).view(np.uint16))


def _same_bits(a, b):
    return np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b)))


def _ulps32(a, b):
    return np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))


_SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1.1754942e-38,
                     3.4028235e38, -3.4028235e38, 2.0 ** 19, -2.0 ** 19, 2.0 ** 20, -2.0 ** 20, 1048575.9,
                     88.72283, 88.72284, -103.97208, 0.7853982, 1.5707964, 3.1415927, 1e30, -1e30], np.float32)


def test_exp_log_sin_cos_restatements_agree():
    """NumPy (palladium_amd.exact) and C (oracle.c) restatements of the
    deterministic exp, log, sin, cos and tanh give the same bits on scattered bit
    patterns over every exponent (the large-argument reduction included),
    the working ranges and the special values."""
    from palladium_amd import exact

    r = np.random.default_rng(11)
    x = np.concatenate([
        r.integers(0, 2 ** 32, 60_000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        r.uniform(-10, 10, 200_000).astype(np.float32),
        r.uniform(-110, 90, 200_000).astype(np.float32),
        _SPECIAL,
    ])
    for name in ("dexpf", "dlogf", "dsinf", "dcosf", "dtanhf"):
        assert _same_bits(getattr(exact, name)(x), getattr(oracle, name)(x)), name


def test_exp_log_within_one_ulp_of_the_double_result():
    from palladium_amd import exact

    r = np.random.default_rng(12)
    e = np.concatenate([r.uniform(-103, 88.7, 400_000), r.uniform(-1e-3, 1e-3, 100_000)]).astype(np.float32)
    got = exact.dexpf(e)
    ref = np.exp(e.astype(np.float64)).astype(np.float32)
    d = _ulps32(got, ref)
    assert d.max() <= 1 and np.mean(d == 0) > 0.999
    x = np.concatenate([np.abs(r.standard_cauchy(300_000)), r.uniform(0.5, 2.0, 200_000),
                        (10.0 ** r.uniform(-44, 38, 100_000))]).astype(np.float32)
    x = x[(x > 0) & np.isfinite(x)]
    got = exact.dlogf(x)
    ref = np.log(x.astype(np.float64)).astype(np.float32)
    d = _ulps32(got, ref)
    assert d.max() <= 1 and np.mean(d == 0) > 0.999
    with np.errstate(all="ignore"):
        sp = _SPECIAL
        np.testing.assert_array_equal(np.isnan(exact.dexpf(sp)), np.isnan(sp))
        np.testing.assert_array_equal(exact.dexpf(np.float32([np.inf, -np.inf, 2.0 ** 19, -2.0 ** 19, 0.0])),
                                      np.float32([np.inf, 0.0, np.inf, 0.0, 1.0]))
        np.testing.assert_array_equal(exact.dlogf(np.float32([0.0, -0.0, np.inf, 1.0, 1e-45])),
                                      np.log(np.float32([0.0, 0.0, np.inf, 1.0, 1e-45]).astype(np.float64)).astype(np.float32))
        assert np.isnan(exact.dlogf(np.float32([-1.0, np.nan, -np.inf]))).all()


def test_sin_cos_within_one_ulp_and_large_arguments_against_mpmath():
    """Below 2^20 against the double sin/cos rounded to float; above it
    (the exact reduction from the bits of 2/pi) against 100-digit mpmath,
    so a wrong table word, window offset or quadrant fails."""
    mp = pytest.importorskip("mpmath")
    from palladium_amd import exact

    r = np.random.default_rng(13)
    x = np.concatenate([r.uniform(-10, 10, 300_000), r.uniform(-2.0 ** 20, 2.0 ** 20, 100_000),
                        np.arange(-64, 65) * (np.pi / 4)]).astype(np.float32)
    x = x[np.abs(x) < 2.0 ** 20]
    for f, ref in ((exact.dsinf, np.sin), (exact.dcosf, np.cos)):
        d = _ulps32(f(x), ref(x.astype(np.float64)).astype(np.float32))
        assert d.max() <= 1 and np.mean(d == 0) > 0.999
    # every binade from 2^20 to 2^127, both signs, plus the largest floats
    big = np.concatenate([np.ldexp(r.uniform(1, 2, 4 * 108), np.repeat(np.arange(20, 128), 4)),
                          [3.4028235e38, 2.0 ** 20, 2.0 ** 20 + 0.125, 1e30]])
    big = np.concatenate([big, -big]).astype(np.float32)
    big = big[np.isfinite(big)]
    with mp.workdps(100):
        want_s = np.array([float(mp.sin(mp.mpf(float(v)))) for v in big]).astype(np.float32)
        want_c = np.array([float(mp.cos(mp.mpf(float(v)))) for v in big]).astype(np.float32)
    assert _ulps32(exact.dsinf(big), want_s).max() <= 1
    assert _ulps32(exact.dcosf(big), want_c).max() <= 1
    assert np.isnan(exact.dsinf(np.float32([np.inf, -np.inf, np.nan]))).all()
    assert np.isnan(exact.dcosf(np.float32([np.inf, -np.inf, np.nan]))).all()


def test_reproducible_interpreter_equals_the_c_gbm_restatement():
    """The GBM kernel's interpreter under REPRODUCIBLE (FAST's rewrites,
    the contraction pass, the deterministic log/cos/exp) equals
    oracle_gbm_r path by path."""
    from palladium_amd.frontend import random
    from palladium_amd.workloads import GBM_CFG, gbm_call

    n = 384
    got = np.asarray(gbm_call(GBM_CFG, n_paths=n, math_mode="reproducible").interpret(random.key(GBM_CFG.seed)))
    want = oracle.gbm(GBM_CFG, n, mode="reproducible")
    assert _same_bits(got, want)
    assert np.abs(got - oracle.gbm(GBM_CFG, n)).max() < 1e-2


def test_reproducible_transcendentals_in_the_emitted_kernel():
    """Under REPRODUCIBLE the kernel calls ph_exp/ph_log/ph_cos, which the
    prelude defines as the deterministic forms in that mode only."""
    from palladium_amd.emit.prelude import PRELUDE
    from palladium_amd.frontend import random
    from palladium_amd.workloads import GBM_CFG, gbm_call

    src = gbm_call(GBM_CFG, n_paths=64, math_mode="reproducible").bound(random.key(1)).hip_source
    body = src[src.index('extern "C"'):]
    for f in ("ph_log(", "ph_cos(", "ph_exp(", "sqrtf("):
        assert f in body
    mode3 = PRELUDE[PRELUDE.index("#if PH_MATH_MODE == 3"):]
    for f in ("ph_dlogf(x)", "ph_dtrig(x, 1)", "ph_dexpf(x)"):
        assert f in mode3


def test_tanh_within_one_ulp_and_special_values():
    """Both sides of the 1/2 split (the odd polynomial and 1 - 2/(e^2a + 1))
    within 1 ulp of the double tanh and correctly rounded on > 99.99 %;
    odd symmetry, signed zeros, saturation to +-1, NaN."""
    from palladium_amd import exact

    r = np.random.default_rng(14)
    x = np.concatenate([r.uniform(-12, 12, 300_000), r.uniform(-0.6, 0.6, 300_000),
                        r.uniform(-1e-4, 1e-4, 50_000)]).astype(np.float32)
    got = exact.dtanhf(x)
    d = _ulps32(got, np.tanh(x.astype(np.float64)).astype(np.float32))
    assert d.max() <= 1 and np.mean(d == 0) > 0.9999
    np.testing.assert_array_equal(exact.dtanhf(-x), -got)
    z = exact.dtanhf(np.float32([0.0, -0.0]))
    assert z.tolist() == [0.0, 0.0] and not np.signbit(z[0]) and np.signbit(z[1])
    np.testing.assert_array_equal(exact.dtanhf(np.float32([np.inf, -np.inf, 20.0, -1e30])),
                                  np.float32([1.0, -1.0, 1.0, -1.0]))
    assert np.isnan(exact.dtanhf(np.float32([np.nan]))).all()


def test_jit_callable_interprets_in_the_mode_too():
    """hip_call_jit's `.interpret()` follows REPRODUCIBLE as hip_call's does."""
    from palladium_amd import exact

    def k(x_ref, o_ref):
        o_ref[...] = jnp.sin(x_ref[...]) / (x_ref[...] + 3.0)

    s = pl.BlockSpec((1,), lambda i: (i,))
    x = np.linspace(-2, 2, 64, dtype=np.float32)
    kw = dict(grid=(64,), in_specs=[s], out_specs=s, out_shape=pl.ShapeDtypeStruct((64,), np.float32),
              math_mode="reproducible")
    got = np.asarray(pa.hip_call_jit(k, **kw).interpret(x))
    want = exact.rdiv(exact.dsinf(x), x + np.float32(3.0))
    assert _same_bits(got, want)
