"""Differential test of the emitter on vector programs (tests/fuzz_vec.py):
per-instance and lane-parallel launches under SAFE math, bit for bit
against the NumPy interpreter."""

import os

import numpy as np
import pytest

from fuzz_vec import make_call, make_inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("lanes", [False, True], ids=["instance", "lanes"])
@pytest.mark.parametrize("seed", range(int(os.environ.get("PALLADIUM_FUZZ_SEEDS", "12"))))
def test_vector_program_bit_exact_vs_interpreter(seed, lanes):
    print(f"fuzz_vec seed={seed} lanes={lanes}", flush=True)
    call = make_call(seed, lanes=lanes, math_mode="safe")
    args = make_inputs(seed)
    got = call(*args)
    want = call.interpret(*args)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
