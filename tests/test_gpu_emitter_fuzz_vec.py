"""Differential test of the emitter on vector programs (tests/fuzz_vec.py):
per-instance and lane-parallel launches under SAFE math, float32 and
bfloat16, bit for bit against the NumPy interpreter."""

import os

import numpy as np
import pytest

from fuzz_vec import make_call, make_inputs

from palladium_amd import dtypes

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("lanes", [False, True], ids=["instance", "lanes"])
@pytest.mark.parametrize("seed", range(int(os.environ.get("PALLADIUM_FUZZ_SEEDS", os.environ.get("PALLADIUM_FUZZ_EXAMPLES", "12")))))
def test_vector_program_bit_exact_vs_interpreter(seed, lanes):
    print(f"fuzz_vec seed={seed} lanes={lanes}", flush=True)
    call = make_call(seed, lanes=lanes, math_mode="safe")
    args = make_inputs(seed)
    got = call(*args)
    want = call.interpret(*args)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)


@pytest.mark.parametrize("dt", [dtypes.bfloat16, np.dtype(np.float16)], ids=["bf16", "f16"])
@pytest.mark.parametrize("lanes", [False, True], ids=["instance", "lanes"])
@pytest.mark.parametrize("seed", range(int(os.environ.get("PALLADIUM_FUZZ_SEEDS", os.environ.get("PALLADIUM_FUZZ_EXAMPLES", "12")))))
def test_vector_program_narrow_float_bit_exact_vs_interpreter(seed, lanes, dt):
    print(f"fuzz_vec {dtypes.name(dt)} seed={seed} lanes={lanes}", flush=True)
    call = make_call(seed, lanes=lanes, dtype=dt, math_mode="safe")
    args = make_inputs(seed, dtype=dt)
    got = call(*args)
    want = call.interpret(*args)
    for g, w in zip(got, want):
        if w.dtype.itemsize == 2:
            g, w = np.ascontiguousarray(g).view(np.uint16), np.ascontiguousarray(w).view(np.uint16)
        np.testing.assert_array_equal(g, w)
