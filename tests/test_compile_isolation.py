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


def test_a_noisy_child_neither_stalls_nor_corrupts_replies(monkeypatch):
    """200 KB on stderr (more than a pipe holds) and stray bytes written to
    fd 1 before each reply: the compile still succeeds."""
    monkeypatch.setenv("PALLADIUM_COMPILE_WORKER_TEST_NOISE", "200000")
    w = compile_worker._Worker()
    try:
        assert w.compile(OK_SRC, "k", 0, "gfx950") == rt.compile_code_object(OK_SRC, "k", 0)
        assert w.compile(OK_SRC, "k", 2, "gfx950")[:4] == b"\x7fELF"
    finally:
        w._discard(kill=True)


@pytest.mark.parametrize("value", ["abc", "0", "-3", "nan", "inf"])
def test_bad_timeout_values_are_compile_errors(monkeypatch, value):
    monkeypatch.setenv("PALLADIUM_COMPILE_TIMEOUT", value)
    with pytest.raises(CompileError, match="PALLADIUM_COMPILE_TIMEOUT"):
        compile_worker.compile_isolated(OK_SRC, "k", 0)


def test_partial_and_malformed_replies(tmp_path):
    import os
    import struct
    import time

    r, w = os.pipe()
    try:
        os.write(w, struct.pack(">I", 40) + b'{"ok": tr')  # a header cut off mid-way
        with pytest.raises(TimeoutError):
            compile_worker._recv_by(r, time.monotonic() + 0.2)
    finally:
        os.close(r)
        os.close(w)
    r, w = os.pipe()
    try:
        os.write(w, struct.pack(">I", 5) + b"nope!")
        with pytest.raises(compile_worker._ReplyError):
            compile_worker._recv_by(r, time.monotonic() + 1.0)
        os.write(w, struct.pack(">I", 1 << 30))
        with pytest.raises(compile_worker._ReplyError):
            compile_worker._recv_by(r, time.monotonic() + 1.0)
    finally:
        os.close(r)
        os.close(w)
    r, w = os.pipe()
    os.close(w)
    try:
        with pytest.raises(compile_worker._ReplyError):
            compile_worker._recv_by(r, time.monotonic() + 1.0)
    finally:
        os.close(r)
