"""`dot_general` on the GPU: SAFE bit-exact against the interpreter (same
k-ordered accumulation), FAST within float32 rounding of float64."""

import numpy as np
import pytest

from dot_cases import CASES, numpy_reference

pytestmark = pytest.mark.gpu


def _tuple(x):
    return x if isinstance(x, tuple) else (x,)


@pytest.mark.parametrize("name", sorted(CASES))
def test_safe_bit_exact_vs_interpreter(name):
    f, inputs = CASES[name](np.random.default_rng(9), math_mode="safe")
    got = _tuple(f(*inputs))
    want = _tuple(f.interpret(*inputs))
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)


@pytest.mark.parametrize("name", sorted(CASES))
def test_fast_close_to_float64(name):
    f, inputs = CASES[name](np.random.default_rng(10))
    for g, w in zip(_tuple(f(*inputs)), numpy_reference(name, inputs)):
        if g.dtype.kind == "i":
            np.testing.assert_array_equal(g, w)
        else:
            # |error| <= k * eps * sum|a_k b_k|; 1e-4 covers k <= 96 here.
            np.testing.assert_allclose(g, w, rtol=1e-4, atol=1e-4)
