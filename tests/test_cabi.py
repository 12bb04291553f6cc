"""The C ABI: the library loads, exports every declared symbol, and its
compile path works without a GPU (hiprtc cross-compiles for gfx950)."""

import re
import subprocess
from pathlib import Path

import pytest

from palladium_amd import runtime as rt
from palladium_amd.errors import CompileError

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "palladium_hip.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"\b(ph_[a-z0-9_]+)\s*\(", text))


def test_every_declared_symbol_is_exported():
    lib = rt.library_path()
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (ph_[a-z0-9_]+)$", out, re.M))
    declared = _declared()
    assert len(declared) >= 30
    assert declared <= exported, declared - exported


def test_library_loads_and_reports_version():
    assert rt.lib().ph_version().decode() == "0.1.0"


def test_compile_options_per_math_mode():
    assert rt.compile_options("safe") == "-ffp-contract=off"
    assert "-ffp-contract=fast" in rt.compile_options("relaxed")
    fast = rt.compile_options("fast")
    assert "-ffast-math" in fast and "-fno-finite-math-only" in fast


def test_compile_code_object_on_cpu():
    src = 'extern "C" __global__ void k(float* o) { o[threadIdx.x] = 1.0f; }'
    code = rt.compile_code_object(src, "k", "fast")
    assert code[:4] == b"\x7fELF"


def test_compile_error_carries_log():
    with pytest.raises(CompileError, match="hiprtc compile failed"):
        rt.compile_code_object('extern "C" __global__ void k() { not_c++ }', "k", "safe")


def test_invalid_math_mode_rejected():
    with pytest.raises(ValueError):
        rt.compile_code_object('extern "C" __global__ void k() {}', "k", 7)


def test_packed_fp32_forms_absent_from_code_objects(tmp_path):
    from palladium_amd.workloads import lv_inputs, lv_rk4_call

    call = lv_rk4_call(1024, 0.01, 8)
    from palladium_amd.emit import emit_hip
    from palladium_amd.trace import trace

    src = emit_hip(trace(call._staged, *lv_inputs(1024, 0)))
    code = rt.compile_code_object(src, "lv_rk4", "fast")
    objdump = Path("/opt/rocm/llvm/bin/llvm-objdump")
    if not objdump.exists():
        pytest.skip("llvm-objdump not available")
    p = tmp_path / "lv_rk4.co"
    p.write_bytes(code)
    asm = subprocess.run([str(objdump), "-d", "--mcpu=gfx950", str(p)], capture_output=True, text=True, check=True).stdout
    assert "v_fma" in asm
    assert "v_pk_" not in asm


@pytest.mark.skipif(rt.device_available(), reason="checks the no-device error path")
def test_kernel_load_without_device_fails_loudly():
    k = rt.Kernel('extern "C" __global__ void k(float* o) { o[0] = 1.0f; }', "k")
    with pytest.raises(rt.HipError):
        k.load()


def test_dispatch_entry_points_reject_null_operand_arrays():
    """Argument validation happens before any HIP call (no GPU needed)."""
    import ctypes

    lib = rt.lib()
    src = b'extern "C" __global__ void k(float* o) {}'
    calls = [
        lambda e: lib.ph_dispatch(src, len(src), b"k", 1, 1, 1, 0, 1, 0, None, None, 1, None, None, 0, ctypes.byref(e)),
        lambda e: lib.ph_dispatch_device(src, len(src), b"k", 1, 1, 1, 0, 1, 0, None, None, 0, None, 1, ctypes.byref(e)),
    ]
    for call in calls:
        err = ctypes.c_void_p()
        assert call(err) == 1
        assert b"null operand array" in ctypes.string_at(err.value)
        lib.ph_free_error(err)
