"""The reference's matmul / reduce / transpose / dtype-matrix cases on the
GPU: against the NumPy closed form (FAST), bit for bit against the
interpreter under SAFE wherever the device and host compute the same
operations (everything except softmax, whose exp may differ by a float32
ulp between device and host libm), and bit for bit under REPRODUCIBLE for
every case, softmax included (its exp and division are restated there).
Float sums are bit-exact because the interpreter adds in the emitted
order."""

import numpy as np
import pytest

import palladium_amd as pa
from ref_suite_cases import CASES, check

pytestmark = pytest.mark.gpu

_ORDER_FREE = {"reduce_softmax"}


@pytest.mark.parametrize("name", sorted(CASES))
def test_fast_matches_closed_form(name):
    kernel, out_shape, args, _ = CASES[name]()
    check(name, pa.hip_call(kernel, out_shape=out_shape)(*args))


@pytest.mark.parametrize("name", sorted(set(CASES) - _ORDER_FREE))
def test_safe_bit_exact_vs_interpreter(name):
    kernel, out_shape, args, _ = CASES[name]()
    f = pa.hip_call(kernel, out_shape=out_shape, math_mode="safe")
    np.testing.assert_array_equal(f(*args), f.interpret(*args))


@pytest.mark.parametrize("name", sorted(CASES))
def test_reproducible_bit_exact_vs_interpreter(name):
    kernel, out_shape, args, _ = CASES[name]()
    f = pa.hip_call(kernel, out_shape=out_shape, math_mode="reproducible")
    got, want = f(*args), f.interpret(*args)
    for g, w in zip(got if isinstance(got, tuple) else (got,), want if isinstance(want, tuple) else (want,)):
        np.testing.assert_array_equal(g, w)
    check(name, got)


def test_preferred_element_type_accumulates_in_float32_on_device():
    """float16 operands, float32 accumulation: each product 1 + 2^-9 + 2^-20
    is exact only in float32 (reference tests/test_16_diagnostics.py:214-233)."""
    from palladium_amd.frontend import jnp, lax, pl

    def kernel(a_ref, b_ref, o_ref):
        o_ref[...] = lax.dot_general(a_ref[...], b_ref[...], (((1,), (0,)), ((), ())),
                                     preferred_element_type=jnp.float32)

    k = 16
    a = np.full((7, k), 1 + 2**-10, dtype=np.float16)
    b = np.full((k, 8), 1 + 2**-10, dtype=np.float16)
    for mode in ("safe", "fast"):
        got = pa.hip_call(kernel, out_shape=pl.ShapeDtypeStruct((7, 8), np.float32), math_mode=mode)(a, b)
        assert got.dtype == np.float32
        np.testing.assert_allclose(got, np.full((7, 8), k * (1 + 2**-9 + 2**-20)), rtol=0, atol=2**-17)
