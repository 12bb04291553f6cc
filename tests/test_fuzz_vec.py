"""The vector fuzz programs trace, take the intended lowering and run on
the interpreter (CPU); the GPU comparison is tests/test_gpu_emitter_fuzz_vec.py."""

import numpy as np
import pytest

from fuzz_vec import make_call, make_inputs
from palladium_amd.emit import emit_hip
from palladium_amd.emit.lanes import lane_transform
from palladium_amd.trace import trace


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("lanes", [False, True])
def test_program_traces_and_interprets(seed, lanes):
    call = make_call(seed, rows=128, lanes=lanes)
    args = make_inputs(seed, rows=128)
    spec = trace(call._staged, *args)
    plan = lane_transform(spec)
    assert (plan is not None) == lanes
    assert "ph_" in emit_hip(spec, math_mode="safe")
    o, s, h = call.interpret(*args)
    assert np.all(np.isfinite(o)) and np.all(np.abs(o) <= 50.0)
    assert np.all(s * 8 == np.round(s * 8))  # sums of 1/8-quantised values stay exact


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("lanes", [False, True])
def test_bf16_program_traces_and_interprets(seed, lanes):
    from palladium_amd import dtypes

    call = make_call(seed, rows=128, lanes=lanes, dtype=dtypes.bfloat16)
    args = make_inputs(seed, rows=128, dtype=dtypes.bfloat16)
    spec = trace(call._staged, *args)
    assert (lane_transform(spec) is not None) == lanes
    assert "__bf16" in emit_hip(spec, math_mode="safe")
    o, s, h = call.interpret(*args)
    o = dtypes.to_float(o)
    assert np.all(np.isfinite(o)) and np.all(np.abs(o) <= 50.0)
