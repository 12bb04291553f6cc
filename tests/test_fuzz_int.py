"""The integer fuzz programs (tests/fuzz_int.py) trace, compile for gfx950
and run on the interpreter (CPU); tests/test_gpu_emitter_fuzz_int.py
compares the GPU with the interpreter."""

import numpy as np
import pytest

from fuzz_int import make_call, make_inputs
from palladium_amd.emit import emit_hip
from palladium_amd.trace import trace


@pytest.mark.parametrize("seed", range(8))
def test_program_traces_emits_and_interprets(seed):
    call = make_call(seed, n=64)
    args = make_inputs(seed, n=64)
    src = emit_hip(trace(call._staged, *args), math_mode="safe")
    assert "ph_" in src
    if seed % 2:
        assert "__any(" in src  # the while loop is predicated
    o, u = call.interpret(*args)
    assert o.dtype == np.int32 and u.dtype == np.uint32
