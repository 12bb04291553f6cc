"""bfloat16 on the GPU (reference: tests/test_17_robustness.py:143-195).

Under SAFE, operations whose float32 result is correctly rounded (+ - * /
sqrt, compares, min/max/abs, integer_pow, conversions) and the float32-
accumulated per-instance sums and contractions are bit-exact with the NumPy
interpreter. float32-computed library functions (exp, log, sin, tanh) may
differ by one float32 ulp between device and host libm, hence by at most
one bfloat16 ulp after rounding. The cross-lane block sum accumulates in
float32 in butterfly order and is held to bfloat16 rounding."""

import numpy as np
import pytest

from palladium_amd import dtypes

import bf16_cases as cases

pytestmark = pytest.mark.gpu


def _f(a):
    return dtypes.to_float(a) if dtypes.is_bf16(a.dtype) else a


def test_copy_round_trips_every_bit_pattern():
    """All 65,536 bit patterns, NaN payloads and signalling NaNs included,
    cross host -> device -> host unchanged (the reference checks eight)."""
    x = cases.all_bit_patterns()
    got = cases.copy()(x)
    assert dtypes.is_bf16(got.dtype)
    np.testing.assert_array_equal(dtypes.as_bits(got), dtypes.as_bits(x))


def test_reference_affine_kernel_and_pin():
    rng = np.random.default_rng(17)
    x = dtypes.from_float(rng.standard_normal(16).astype(np.float32))
    f = cases.affine(math_mode="safe")
    want = f.interpret(x)
    np.testing.assert_array_equal(dtypes.as_bits(f(x)), dtypes.as_bits(want))
    pinned = f.pin(x)
    np.testing.assert_array_equal(dtypes.as_bits(pinned()), dtypes.as_bits(want))


@pytest.mark.parametrize("mode", ["relaxed", "fast"])
def test_reference_affine_kernel_other_modes(mode):
    # the reference's tolerance for its bf16 kernel (rtol = atol = 2e-2)
    rng = np.random.default_rng(17)
    x = dtypes.from_float(rng.standard_normal(16).astype(np.float32))
    f = cases.affine(math_mode=mode)
    np.testing.assert_allclose(_f(f(x)), _f(f.interpret(x)), rtol=2e-2, atol=2e-2)


def test_arithmetic_bit_exact():
    x, y = cases.inputs(1)
    f = cases.arithmetic(math_mode="safe")
    for g, w in zip(f(x, y), f.interpret(x, y)):
        if dtypes.is_bf16(w.dtype):
            g, w = dtypes.as_bits(g), dtypes.as_bits(w)
        np.testing.assert_array_equal(g, w)


def test_transcendental_within_one_ulp():
    x, _ = cases.inputs(3)
    f = cases.transcendental(math_mode="safe")
    o, s = f(x)
    wo, _ = f.interpret(x)
    o, wo = _f(o).astype(np.float64), _f(wo).astype(np.float64)
    fin = np.isfinite(wo)
    assert np.array_equal(np.isfinite(o), fin)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(wo[fin]), 2.0**-126))) - 7)
    assert np.all(np.abs(o[fin] - wo[fin]) <= ulp)
    blocks = o.reshape(-1, cases.B)
    ok = np.all(np.isfinite(blocks), axis=1)
    want = blocks[ok].sum(axis=1)
    mag = np.abs(blocks[ok]).sum(axis=1)
    assert np.all(np.abs(_f(s)[ok].astype(np.float64) - want) <= 2.0**-8 * mag + 1e-30)


def test_instance_reductions_and_contraction_bit_exact():
    rng = np.random.default_rng(5)
    x = dtypes.from_float(rng.standard_normal(1024).astype(np.float32))
    m = dtypes.from_float(rng.standard_normal((16, 16)).astype(np.float32))
    f = cases.instance_reduce(math_mode="safe")
    for g, w in zip(f(x, m), f.interpret(x, m)):
        np.testing.assert_array_equal(dtypes.as_bits(g), dtypes.as_bits(w))
