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


def test_float16_program_that_crashed_the_backend_compiles():
    """Seed 72's float16 program aborted LLVM's gfx950 instruction selection
    ("Cannot select: v2f32 = bitcast") when SLP vectorisation met packed
    FP32 being disabled; the compile options now exclude SLP. Compiled in a
    subprocess, since the failure mode is an abort inside hiprtc."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    code = (
        "import sys; sys.path[:0] = [%r, %r]\n"
        "import numpy as np\n"
        "import fuzz_vec\n"
        "from palladium_amd import runtime as rt\n"
        "from palladium_amd.emit import emit_hip\n"
        "from palladium_amd.trace import trace\n"
        "for lanes in (False, True):\n"
        "    call = fuzz_vec.make_call(72, lanes=lanes, dtype=np.float16, math_mode='safe')\n"
        "    spec = trace(call._staged, *fuzz_vec.make_inputs(72, dtype=np.float16))\n"
        "    rt.compile_code_object(emit_hip(spec, math_mode='safe'), spec.name, 'safe')\n"
    ) % (str(root / "tests"), str(root))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
