"""Differential test of the emitter on integer programs (tests/fuzz_int.py):
GPU against the NumPy interpreter, bit for bit."""

import os

import numpy as np
import pytest

from fuzz_int import make_call, make_inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(int(os.environ.get("PALLADIUM_FUZZ_SEEDS", os.environ.get("PALLADIUM_FUZZ_EXAMPLES", "12")))))
def test_integer_program_bit_exact_vs_interpreter(seed):
    print(f"fuzz_int seed={seed}", flush=True)
    call = make_call(seed, math_mode="safe")
    args = make_inputs(seed)
    for g, w in zip(call(*args), call.interpret(*args)):
        np.testing.assert_array_equal(g, w)
