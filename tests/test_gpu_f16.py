"""float16 on the GPU. Correctly rounded operations (+ - * / compare,
min/max/abs, integer_pow, conversions) are bit-exact with the NumPy
interpreter under SAFE; float32-computed functions (exp, log, sin, sqrt)
differ by at most one float16 ulp (their float32 results can differ in the
last float32 ulp between device and host libm); the cross-lane float16 sum
accumulates in float32 and is held to float16 rounding."""

import numpy as np
import pytest

from f16_cases import arithmetic, inputs, transcendental

pytestmark = pytest.mark.gpu


def test_arithmetic_bit_exact():
    x, y = inputs(1)
    f = arithmetic(math_mode="safe")
    got = f(x, y)
    want = f.interpret(x, y)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)


@pytest.mark.parametrize("mode", ["relaxed", "fast"])
def test_arithmetic_contracted_within_rounding(mode):
    x, y = inputs(2)
    f = arithmetic(math_mode=mode)
    got = f(x, y)
    want = f.interpret(x, y)
    o, w = got[0].astype(np.float64), want[0].astype(np.float64)
    ok = np.isfinite(w)
    # FMA contraction skips one float16 rounding per fused pair, so the
    # difference is a few float16 ulps of the largest term, not of the
    # (possibly cancelled) result.
    xd, yd = x.astype(np.float64), y.astype(np.float64)
    scale = np.abs(xd * yd) + 3 * np.abs(xd) + 3 * np.abs(yd) + np.abs(yd) ** 3 + 1.0
    assert np.all(np.abs(o[ok] - w[ok]) <= 4e-3 * scale[ok])


def test_transcendental_within_one_ulp():
    x, _ = inputs(3)
    f = transcendental(math_mode="safe")
    o, s = f(x)
    wo, _ = f.interpret(x)
    fin = np.isfinite(wo)
    assert np.array_equal(np.isfinite(o), fin)
    ulp = np.spacing(np.abs(wo[fin]).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(o[fin].astype(np.float64) - wo[fin].astype(np.float64)) <= ulp)
    blocks = o.astype(np.float64).reshape(-1, 64)
    ok = np.all(np.isfinite(blocks), axis=1)
    want = blocks[ok].sum(axis=1)
    np.testing.assert_allclose(s[ok].astype(np.float64), want, rtol=1e-3,
                               atol=1e-3 * np.abs(blocks[ok]).sum(axis=1).max())
