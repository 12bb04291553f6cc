"""The reference's matmul / reduce / transpose / dtype-matrix cases on the
GPU: against the NumPy closed form (FAST), and bit for bit against the
interpreter under SAFE wherever the op order is fixed (everything except
float sums, whose interpreter order is NumPy's pairwise summation)."""

import numpy as np
import pytest

import palladium_amd as pa
from ref_suite_cases import CASES, check

pytestmark = pytest.mark.gpu

_ORDER_FREE = {"reduce_sum_scalar", "reduce_sum_last", "reduce_sum_first", "reduce_mean", "reduce_mse",
               "reduce_softmax", "dtype_float16_sum"}


@pytest.mark.parametrize("name", sorted(CASES))
def test_fast_matches_closed_form(name):
    kernel, out_shape, args, _ = CASES[name]()
    check(name, pa.hip_call(kernel, out_shape=out_shape)(*args))


@pytest.mark.parametrize("name", sorted(set(CASES) - _ORDER_FREE))
def test_safe_bit_exact_vs_interpreter(name):
    kernel, out_shape, args, _ = CASES[name]()
    f = pa.hip_call(kernel, out_shape=out_shape, math_mode="safe")
    np.testing.assert_array_equal(f(*args), f.interpret(*args))
