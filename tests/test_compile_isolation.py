"""Opt-in compilation in a helper process (CPU, no GPU needed): a backend
crash becomes a CompileError in the caller, and the next compile works."""

import numpy as np
import pytest

from palladium_amd import compile_worker
from palladium_amd import runtime as rt
from palladium_amd.errors import CompileError

OK_SRC = 'extern "C" __global__ void k(float* o) { o[threadIdx.x] = 1.0f; }'
# An "r" register constraint on an AMDGPU inline asm operand makes LLVM's
# code emitter abort ("LLVM ERROR: Unsupported instruction") rather than
# report an error.
CRASH_SRC = ('extern "C" __global__ void k(float* o) { unsigned int x = threadIdx.x; '
             'asm volatile("" : "+r"(x)); o[threadIdx.x] = (float)x; }')


def test_isolated_compile_matches_in_process():
    assert compile_worker.compile_isolated(OK_SRC, "k", 2)[:4] == b"\x7fELF"
    assert compile_worker.compile_isolated(OK_SRC, "k", 0) == rt.compile_code_object(OK_SRC, "k", 0)


def test_compile_errors_come_back_as_compile_errors():
    with pytest.raises(CompileError, match="hiprtc compile failed"):
        compile_worker.compile_isolated('extern "C" __global__ void k() { not_cpp }', "k", 0)


def test_backend_crash_is_a_compile_error_and_the_next_compile_works():
    with pytest.raises(CompileError, match="compiler process ended"):
        compile_worker.compile_isolated(CRASH_SRC, "k", 2)
    assert compile_worker.compile_isolated(OK_SRC, "k", 2)[:4] == b"\x7fELF"


def test_kernel_load_uses_the_helper_when_enabled(monkeypatch):
    monkeypatch.setenv("PALLADIUM_COMPILE_ISOLATED", "1")
    assert compile_worker.isolation_enabled()
    calls = []
    real = compile_worker.compile_isolated
    monkeypatch.setattr(compile_worker, "compile_isolated", lambda *a, **k: calls.append(a) or real(*a, **k))
    k = rt.Kernel(OK_SRC, "k", "fast")
    if rt.device_available():
        k.load()
        assert calls
    else:
        with pytest.raises(Exception):
            k.load()  # the code object is compiled, then loading needs a device
        assert calls and np.asarray(calls[0][2]) == 2


def test_a_compile_past_the_deadline_is_stopped(monkeypatch):
    monkeypatch.setenv("PALLADIUM_COMPILE_TIMEOUT", "0.0001")
    with pytest.raises(CompileError, match="PALLADIUM_COMPILE_TIMEOUT"):
        compile_worker.compile_isolated(OK_SRC.replace("1.0f", "3.0f"), "k", 0)
    monkeypatch.delenv("PALLADIUM_COMPILE_TIMEOUT")
    assert compile_worker.compile_isolated(OK_SRC, "k", 0)[:4] == b"\x7fELF"
