"""Public API contract on the CPU: explain(), PALLADIUM_EXPLAIN, the error
taxonomy, call-boundary validation, and compile-once under concurrency
(reference: tests/test_16_diagnostics.py, tests/test_17_robustness.py)."""

import threading

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd import DispatchError, EmitError, PalladiumError, TraceError, UnsupportedPrimitiveError
from palladium_amd.frontend import pl

F = np.float32


def _double(n=64, **kw):
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...] * 2.0

    spec = pl.BlockSpec((1,), lambda i: (i,))
    return pa.hip_call(kernel, grid=(n,), in_specs=[spec], out_specs=spec, out_shape=pl.ShapeDtypeStruct((n,), F), **kw)


def test_all_exports_present():
    for name in pa.__all__:
        assert hasattr(pa, name), name


def test_error_hierarchy():
    assert issubclass(TraceError, ValueError) and issubclass(TraceError, PalladiumError)
    assert issubclass(DispatchError, TypeError) and issubclass(DispatchError, PalladiumError)
    assert issubclass(UnsupportedPrimitiveError, EmitError) and issubclass(UnsupportedPrimitiveError, NotImplementedError)


def test_explain_reports_geometry_and_resources():
    diag = _double(1000).explain(np.zeros(1000, F))
    assert diag.grid == (1000,)
    assert diag.threadgroup is None
    assert diag.block == 256 and diag.blocks == 4
    assert diag.hip_lines > 0 and diag.msl_lines == diag.hip_lines
    assert diag.resources.vgprs > 0 and diag.resources.scratch_bytes == 0
    assert f"palladium kernel {diag.name}" in str(diag)


def test_large_gridless_block_compiles_and_hints_at_blockspecs():
    """A 4096-element gridless block (reference tests/test_17_robustness.py:
    202-214 expects such a kernel to either work or name the fix): it
    compiles, long element loops are not force-unrolled, and explain names
    the fix for the scratch it needs."""

    def kernel(x_ref, y_ref, o_ref):
        o_ref[...] = 2.0 * x_ref[...] + y_ref[...]

    call = pa.hip_call(kernel, out_shape=pl.ShapeDtypeStruct((4096,), F))
    x = np.zeros(4096, F)
    src = pa.debug_hip(kernel, x, x, out_shape=pl.ShapeDtypeStruct((4096,), F))
    assert "< 4096" in src and "#pragma unroll" not in src
    diag = call.explain(x, x)
    assert diag.resources.scratch_bytes > 4096
    assert "grid and BlockSpecs" in str(diag)
    assert "hint" not in str(_double(64).explain(np.zeros(64, F)))


def test_explain_explicit_threadgroup():
    diag = _double(128, threadgroup=64).explain(np.zeros(128, F), compile=False)
    assert diag.threadgroup == (64,)
    assert diag.blocks == 2
    assert "threadgroup=(64,)" in str(diag)


def test_explain_env_logs_once_per_compile(monkeypatch, capsys):
    monkeypatch.setenv("PALLADIUM_EXPLAIN", "1")
    call = _double(64)
    x = np.zeros(64, F)
    call.bound(x)
    call.bound(x)
    assert capsys.readouterr().err.count("palladium kernel") == 1


def test_dump_hip_env(monkeypatch, tmp_path):
    monkeypatch.setenv("PALLADIUM_DUMP_HIP", str(tmp_path))
    _double(64).bound(np.zeros(64, F))
    files = list(tmp_path.glob("*.hip"))
    assert len(files) == 1 and "__global__" in files[0].read_text()


def test_dtype_gate_before_tracing():
    with pytest.raises(DispatchError, match="float64"):
        _double(4)(np.zeros(4, np.float64))


def test_arity_shape_dtype_checks():
    call = _double(64)
    x = np.zeros(64, F)
    bound = call.bound(x)
    with pytest.raises(DispatchError, match="kernel takes 1 arrays, got 2"):
        bound(x, x)
    with pytest.raises(DispatchError, match="dtype int32 does not match the traced float32; cast explicitly"):
        bound(np.zeros(64, np.int32))
    with pytest.raises(DispatchError, match=r"expected shape \(64,\), got \(32,\)"):
        bound(np.zeros(32, F))


def test_concurrent_first_calls_compile_once(monkeypatch):
    import palladium_amd

    calls = []
    real_bind = palladium_amd.bind

    def counting_bind(*a, **k):
        calls.append(1)
        return real_bind(*a, **k)

    monkeypatch.setattr(palladium_amd, "bind", counting_bind)
    call = _double(256)
    x = np.zeros(256, F)
    barrier = threading.Barrier(16)
    errors = []

    def worker():
        try:
            barrier.wait()
            call.bound(x)
        except Exception as e:  # pragma: no cover
            errors.append(e)

    ts = [threading.Thread(target=worker) for _ in range(16)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors
    assert len(calls) == 1
    assert len(call.cache) == 1


def test_debug_hip_returns_source():
    src = pa.debug_hip(lambda x_ref, o_ref: None, np.zeros(4, F), out_shape=pl.ShapeDtypeStruct((4,), F))
    assert 'extern "C" __global__' in src


def test_hip_call_jit_rejects_whole_batch_vmap():
    with pytest.raises(ValueError, match="sequential"):
        pa.hip_call_jit(lambda x, o: None, out_shape=pl.ShapeDtypeStruct((1,), F), vmap_method="expand_dims")


def test_hip_call_jit_ffi_attributes():
    call = pa.hip_call_jit(lambda x_ref, o_ref: None, out_shape=pl.ShapeDtypeStruct((4,), F), math_mode="safe")
    attrs = call.ffi_attributes((np.zeros(4, F),))
    assert attrs["function_name"] == "<lambda>" or attrs["function_name"] == "palladium_kernel"
    assert (attrs["grid_x"], attrs["grid_y"], attrs["grid_z"]) == (1, 1, 1)
    assert attrs["block_x"] == 256 and attrs["math_mode"] == 0 and attrs["lanes"] == 1
    assert "__global__" in attrs["hip_source"]


def test_ffi_attributes_carry_lanes_of_a_lane_parallel_kernel():
    from dot_cases import lane_rows

    jit, inputs = lane_rows(np.random.default_rng(0), factory=pa.hip_call_jit)
    attrs = jit.ffi_attributes(inputs)
    # 8 programs of 128 rows: one workgroup of 128 lanes per program.
    assert (attrs["grid_x"], attrs["block_x"], attrs["lanes"]) == (8, 128, 128)


def test_math_mode_values():
    assert pa.MathMode("safe").ordinal == 0 and pa.MathMode.FAST.ordinal == 2
    with pytest.raises(ValueError):
        _double(4, math_mode="turbo")


def test_debug_hip_matches_what_hip_call_compiles():
    """debug_hip applies the math mode's emission (FAST factoring) exactly
    as hip_call does."""

    def kernel(x_ref, y_ref, o_ref):
        x, y = x_ref[...], y_ref[...]
        o_ref[...] = 2.0 * x - (3.0 * x) * y

    x = np.zeros(8, F)
    out = pl.ShapeDtypeStruct((8,), F)
    spec = pa.trace(pl.pallas_call(kernel, out_shape=out), x, x)
    for mode in ("safe", "fast"):
        assert pa.debug_hip(kernel, x, x, out_shape=out, math_mode=mode) == pa.emit_hip(spec, math_mode=mode)
    assert pa.debug_hip(kernel, x, x, out_shape=out) == pa.emit_hip(spec, math_mode="fast")
    assert pa.debug_hip(kernel, x, x, out_shape=out, math_mode="safe") != pa.debug_hip(kernel, x, x, out_shape=out)


def test_hip_call_jit_without_jax_names_the_alternative(monkeypatch):
    import sys

    monkeypatch.setitem(sys.modules, "jax", None)  # import jax -> ImportError
    f = pa.hip_call_jit(lambda x, o: o.__setitem__(Ellipsis, x[...]), out_shape=pl.ShapeDtypeStruct((8,), F))
    with pytest.raises(ImportError, match="hip_call"):
        f(np.zeros(8, F))


def test_explain_reports_lane_parallel_lowering():
    spec = pl.BlockSpec((256,), lambda i: (i,))

    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...] * 2.0

    f = pa.hip_call(kernel, grid=(4,), in_specs=[spec], out_specs=spec, out_shape=pl.ShapeDtypeStruct((1024,), F))
    diag = f.explain(np.zeros(1024, F), compile=False)
    assert diag.lanes == 256 and "lanes/instance=256" in str(diag)
    assert "lanes/instance" not in str(_double(64).explain(np.zeros(64, F), compile=False))
