"""Signed zeros through float min/max, clamp and reductions: the device and
the interpreter agree bit for bit (both order -0 below +0), float32 and
bfloat16."""

import numpy as np
import pytest

from palladium_amd import dtypes

import signed_zero_cases as zc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt", [np.float32, dtypes.bfloat16], ids=["f32", "bf16"])
def test_signed_zero_min_max_bit_exact(dt):
    f = zc.call(dt)
    args = zc.inputs(dt)
    for g, w in zip(f(*args), f.interpret(*args)):
        np.testing.assert_array_equal(np.ascontiguousarray(g).view(np.uint8), np.ascontiguousarray(w).view(np.uint8))


@pytest.mark.parametrize("dt", [np.float32, dtypes.bfloat16], ids=["f32", "bf16"])
def test_round_sign_floor_ceil_bit_exact(dt):
    f = zc.rounding_call(dt)
    x = zc.rounding_inputs(dt)
    for g, w in zip(f(x), f.interpret(x)):
        np.testing.assert_array_equal(np.ascontiguousarray(g).view(np.uint8), np.ascontiguousarray(w).view(np.uint8))
