"""Launch semantics on the GPU (reference: tests/test_dispatch_launch.py,
tests/test_11_ffi.py, tests/test_17_robustness.py)."""

import ctypes
import threading
from pathlib import Path

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd import runtime as rt
from palladium_amd.emit import emit_hip
from palladium_amd.frontend import pl

pytestmark = pytest.mark.gpu

F = np.float32


def _inc(n):
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...] + 1.0

    spec = pl.BlockSpec((1,), lambda i: (i,))
    return pa.hip_call(kernel, grid=(n,), in_specs=[spec], out_specs=spec, out_shape=pl.ShapeDtypeStruct((n,), F))


def test_launch_wait_matches_call(rng):
    f = _inc(256)
    x = rng.standard_normal(256).astype(F)
    np.testing.assert_array_equal(f.launch(x).wait(), f(x))
    np.testing.assert_array_equal(f(x), x + 1.0)


def test_stepping_loop_via_launch(rng):
    f, g = _inc(64), _inc(64)
    x0 = rng.standard_normal(64).astype(F)
    x = x0.copy()
    for _ in range(5):
        x = f(x)
    pending = g.launch(x0)
    for _ in range(4):
        pending = g.launch(pending.wait())
    np.testing.assert_array_equal(pending.wait(), x)


def test_second_launch_before_wait_does_not_corrupt_first(rng):
    n = 1 << 20
    f = _inc(n)
    x0 = rng.standard_normal(n).astype(F)
    x1 = rng.standard_normal(n).astype(F)
    first = f.launch(x0)
    second = f.launch(x1)
    np.testing.assert_array_equal(first.wait(), x0 + 1.0)
    np.testing.assert_array_equal(second.wait(), x1 + 1.0)


def test_pin_redispatches_without_upload(rng):
    f = _inc(128)
    x = rng.standard_normal(128).astype(F)
    call = f.pin(x)
    x[:] = 0  # later mutation is not observed
    a, b = call(), call()
    np.testing.assert_array_equal(a, b)
    assert not np.array_equal(a, np.ones(128, F))


def test_concurrent_launches_on_one_kernel(rng):
    f = _inc(4096)
    xs = [rng.standard_normal(4096).astype(F) for _ in range(8)]
    results = [None] * 8

    def worker(i):
        results[i] = f(xs[i])

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    for x, r in zip(xs, results):
        np.testing.assert_array_equal(r, x + 1.0)


def test_launch_device_with_runtime_buffers(rng):
    f = _inc(1000)
    x = rng.standard_normal(1000).astype(F)
    bound = f.bound(x)
    xb = rt.Buffer.from_numpy(x)
    ob = rt.Buffer.empty((1000,), F)
    bound.launch_device(xb, ob)
    np.testing.assert_array_equal(ob.to_numpy(bound.stream), x + 1.0)
    with pytest.raises(pa.DispatchError):
        bound.launch_device(xb, rt.Buffer.empty((999,), F))


def test_ph_dispatch_c_abi_host_buffers(rng):
    """The FFI-handler entry point: source + name + grid + block + math mode,
    host inputs then outputs, synchronous."""
    n = 777
    f = _inc(n)
    x = rng.standard_normal(n).astype(F)
    spec = pa.trace(f._staged, x)
    src = emit_hip(spec).encode()
    out = np.empty(n, F)
    ins = (ctypes.c_void_p * 1)(x.ctypes.data)
    in_b = (ctypes.c_size_t * 1)(x.nbytes)
    outs = (ctypes.c_void_p * 1)(out.ctypes.data)
    out_b = (ctypes.c_size_t * 1)(out.nbytes)
    err = ctypes.c_void_p()
    rc = rt.lib().ph_dispatch(src, len(src), spec.name.encode(), n, 1, 1, 256, 1, 0, ins, in_b, 1, outs, out_b, 1,
                              ctypes.byref(err))
    assert rc == 0
    np.testing.assert_array_equal(out, x + 1.0)
    rc = rt.lib().ph_dispatch(src, len(src), spec.name.encode(), n, 1, 1, 256, 1, 5, ins, in_b, 1, outs, out_b, 1,
                              ctypes.byref(err))
    assert rc == rt.PH_ERR_INVALID
    assert b"math_mode out of range" in ctypes.cast(err, ctypes.c_char_p).value
    rt.lib().ph_free_error(err)


def test_ph_dispatch_concurrent_callers():
    """XLA:CPU calls the handler from its thread pool: 8 threads dispatch
    through ph_dispatch at once, each with its own inputs and sizes (the
    per-thread staging grows), 20 calls each; every result is its own."""
    sizes = [257, 1000, 4096, 64, 3000, 777, 12345, 511]
    srcs = {}
    for n in set(sizes):
        f = _inc(n)
        spec = pa.trace(f._staged, np.zeros(n, F))
        srcs[n] = (emit_hip(spec).encode(), spec.name.encode())
    errors = []

    def worker(t):
        try:
            r = np.random.default_rng(t)
            for k in range(20):
                n = sizes[(t + k) % len(sizes)]
                src, name = srcs[n]
                x = r.standard_normal(n).astype(F)
                out = np.empty(n, F)
                ins = (ctypes.c_void_p * 1)(x.ctypes.data)
                in_b = (ctypes.c_size_t * 1)(x.nbytes)
                outs = (ctypes.c_void_p * 1)(out.ctypes.data)
                out_b = (ctypes.c_size_t * 1)(out.nbytes)
                err = ctypes.c_void_p()
                rc = rt.lib().ph_dispatch(src, len(src), name, n, 1, 1, 256, 1, 0, ins, in_b, 1, outs, out_b, 1,
                                          ctypes.byref(err))
                if rc != 0 or not np.array_equal(out, x + 1.0):
                    errors.append((t, k, n, rc))
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append((t, repr(e)))

    ts = [threading.Thread(target=worker, args=(t,)) for t in range(8)]
    for th in ts:
        th.start()
    for th in ts:
        th.join(timeout=60)
    assert not any(th.is_alive() for th in ts)
    assert not errors, errors[:5]


def _lane_kernel_attrs(rng):
    """A lane-parallel kernel ((128, 8) @ (8, 4) blocks, one row per lane)
    and the FFI attributes hip_call_jit would bake into the HLO."""
    from dot_cases import lane_rows

    f, inputs = lane_rows(np.random.default_rng(4), math_mode="safe")
    jit, _ = lane_rows(np.random.default_rng(4), factory=pa.hip_call_jit, math_mode="safe")
    attrs = jit.ffi_attributes(inputs)
    assert attrs["lanes"] == 128
    return f, inputs, attrs


def test_ph_dispatch_lane_parallel_kernel(rng):
    f, (a, w), attrs = _lane_kernel_attrs(rng)
    want = f.interpret(a, w)
    out = np.empty_like(want)
    src = attrs["hip_source"].encode()
    ins = (ctypes.c_void_p * 2)(a.ctypes.data, w.ctypes.data)
    in_b = (ctypes.c_size_t * 2)(a.nbytes, w.nbytes)
    outs = (ctypes.c_void_p * 1)(out.ctypes.data)
    out_b = (ctypes.c_size_t * 1)(out.nbytes)
    err = ctypes.c_void_p()
    rc = rt.lib().ph_dispatch(src, len(src), attrs["function_name"].encode(), attrs["grid_x"], attrs["grid_y"],
                              attrs["grid_z"], attrs["block_x"], attrs["lanes"], attrs["math_mode"],
                              ins, in_b, 2, outs, out_b, 1, ctypes.byref(err))
    assert rc == 0, ctypes.cast(err, ctypes.c_char_p).value
    np.testing.assert_array_equal(out, want)


def test_ph_dispatch_device_buffers_on_a_stream(rng):
    """The ROCM-platform handler body: device pointers, the caller's stream,
    no staging and no wait."""
    f, (a, w), attrs = _lane_kernel_attrs(rng)
    want = f.interpret(a, w)
    da, dw = rt.Buffer.from_numpy(a), rt.Buffer.from_numpy(w)
    dout = rt.Buffer.empty(want.shape, want.dtype)
    stream = rt.Stream()
    src = attrs["hip_source"].encode()
    ins = (ctypes.c_void_p * 2)(da.ptr, dw.ptr)
    outs = (ctypes.c_void_p * 1)(dout.ptr)
    err = ctypes.c_void_p()
    rc = rt.lib().ph_dispatch_device(src, len(src), attrs["function_name"].encode(), attrs["grid_x"],
                                     attrs["grid_y"], attrs["grid_z"], attrs["block_x"], attrs["lanes"],
                                     attrs["math_mode"], ctypes.c_void_p(stream.handle), ins, 2, outs, 1,
                                     ctypes.byref(err))
    assert rc == 0, ctypes.cast(err, ctypes.c_char_p).value
    np.testing.assert_array_equal(dout.to_numpy(stream), want)
    rc = rt.lib().ph_dispatch_device(src, len(src), attrs["function_name"].encode(), 0, 1, 1, 256, 1, 0,
                                     ctypes.c_void_p(stream.handle), ins, 2, outs, 1, ctypes.byref(err))
    assert rc == rt.PH_ERR_INVALID
    assert b"grid dims must be positive" in ctypes.cast(err, ctypes.c_char_p).value
    rt.lib().ph_free_error(err)


def test_kernel_cache_compiles_each_source_once():
    before = rt.lib().ph_kernel_cache_size()
    f = _inc(32)
    f(np.zeros(32, F))
    mid = rt.lib().ph_kernel_cache_size()
    k = rt.Kernel(f.cache[next(iter(f.cache))].hip_source, f.cache[next(iter(f.cache))].spec.name, "fast")
    k.load()
    assert rt.lib().ph_kernel_cache_size() == mid >= before + 1


def test_safe_mode_propagates_nan_and_inf():
    def kernel(x_ref, o_ref):
        x = x_ref[...]
        o_ref[...] = x * 0.0 + x / 0.0

    f = pa.hip_call(kernel, out_shape=pl.ShapeDtypeStruct((3,), F), math_mode="safe")
    out = f(np.array([1.0, -1.0, 0.0], F))
    assert np.isnan(out[2]) and np.isinf(out[0]) and out[1] < 0


_TORCH_INTEROP = r"""
import sys
sys.path.insert(0, sys.argv[1])
import torch  # first: palladium_amd then binds to torch's HIP runtime
import numpy as np
import palladium_amd as pa
from palladium_amd.frontend import pl
assert torch.cuda.is_available()
f = pa.hip_call(lambda x_ref, o_ref: o_ref.__setitem__(Ellipsis, x_ref[...] + 1.0),
                grid=(2,), in_specs=[pl.BlockSpec((256,), lambda i: (i,))],
                out_specs=pl.BlockSpec((256,), lambda i: (i,)),
                out_shape=pl.ShapeDtypeStruct((512,), np.float32))
x = torch.arange(512, dtype=torch.float32, device="cuda")
o = torch.empty_like(x)
bound = f.bound(np.zeros(512, np.float32))
torch.cuda.synchronize()
bound.launch_device(x, o)
bound.stream.synchronize()
assert torch.equal(o, x + 1.0)
# bfloat16 tensors wrap as bfloat16 buffers: x * 2 + 1 in bf16, against the
# interpreter on the same values
from palladium_amd import dtypes
g = pa.hip_call(lambda x_ref, o_ref: o_ref.__setitem__(Ellipsis, x_ref[...] * 2.0 + 1.0),
                grid=(2,), in_specs=[pl.BlockSpec((256,), lambda i: (i,))],
                out_specs=pl.BlockSpec((256,), lambda i: (i,)),
                out_shape=pl.ShapeDtypeStruct((512,), dtypes.bfloat16), math_mode="safe")
xb = torch.linspace(-3, 3, 512, device="cuda").to(torch.bfloat16)
ob = torch.empty_like(xb)
host = dtypes.from_float(xb.float().cpu().numpy())
gb = g.bound(host)
torch.cuda.synchronize()
gb.launch_device(xb, ob)
gb.stream.synchronize()
want = dtypes.as_bits(g.interpret(host))
got = ob.cpu().view(torch.int16).numpy().view(np.uint16)
assert np.array_equal(got, want), (got[:8], want[:8])
print("torch interop ok")
"""


def test_torch_device_tensors_zero_copy():
    """torch tensors in HBM passed straight to a kernel. One process holds
    one HIP runtime only when torch is imported before palladium_amd (the
    native library then binds to torch's libamdhip64), so this runs in a
    fresh child process that does exactly that."""
    import importlib.util
    import subprocess
    import sys

    if importlib.util.find_spec("torch") is None:
        pytest.skip("torch is not installed")
    root = str(Path(__file__).resolve().parents[1])
    r = subprocess.run([sys.executable, "-c", _TORCH_INTEROP, root], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "torch interop ok" in r.stdout


def test_isolated_compile_path_runs_kernels(monkeypatch, rng):
    """PALLADIUM_COMPILE_ISOLATED=1: the code object comes from the helper
    process and loads through ph_load_code_object; results equal the
    in-process path's."""
    from palladium_amd.workloads import lv_inputs, lv_rk4_call

    args = lv_inputs(2048, 5)
    want = lv_rk4_call(2048, 0.01, 100, track_max=True, math_mode="safe")(*args)
    monkeypatch.setenv("PALLADIUM_COMPILE_ISOLATED", "1")
    got = lv_rk4_call(2048, 0.01, 100, track_max=True, math_mode="safe")(*args)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)


def test_more_launches_than_buffer_sets_before_any_wait(rng):
    """10 launches (the ring has 4 buffer sets) before the first wait, waited
    in reverse order: a set is only reused after its earlier result has been
    copied out, so every wait returns its own launch's outputs, twice."""
    n = 300
    f = _inc(n)
    xs = [rng.standard_normal(n).astype(F) for _ in range(10)]
    b = f.bound(xs[0])
    pend = [b.launch(x) for x in xs]
    for x, p in reversed(list(zip(xs, pend))):
        np.testing.assert_array_equal(p.wait(), x + 1.0)
        np.testing.assert_array_equal(p.wait(), x + 1.0)


def _two_out(n):
    def kernel(x_ref, a_ref, b_ref):
        x = x_ref[...]
        a_ref[...] = x + 1.0
        b_ref[...] = x * 2.0

    spec = pl.BlockSpec((1,), lambda i: (i,))
    f = pa.hip_call(kernel, grid=(n,), in_specs=[spec], out_specs=(spec, spec),
                    out_shape=(pl.ShapeDtypeStruct((n,), F), pl.ShapeDtypeStruct((n,), F)))
    spec_t = pa.trace(f._staged, np.zeros(n, F))
    return emit_hip(spec_t).encode(), spec_t.name.encode()


def _dispatch_two_out(src, name, x):
    n = x.size
    a, b = np.full(n, np.nan, F), np.full(n, np.nan, F)
    ins = (ctypes.c_void_p * 1)(x.ctypes.data)
    in_b = (ctypes.c_size_t * 1)(x.nbytes)
    outs = (ctypes.c_void_p * 2)(a.ctypes.data, b.ctypes.data)
    out_b = (ctypes.c_size_t * 2)(a.nbytes, b.nbytes)
    err = ctypes.c_void_p()
    rc = rt.lib().ph_dispatch(src, len(src), name, n, 1, 1, 256, 1, 0, ins, in_b, 1, outs, out_b, 2,
                              ctypes.byref(err))
    assert rc == 0, ctypes.cast(err, ctypes.c_char_p).value
    return a, b


def test_ph_dispatch_bounce_then_direct_then_bounce(rng):
    """One thread: outputs of 2 x 16 KB (read back through the pinned
    bounce buffer), then 2 x 1 MB (straight into the caller's memory, the
    staging buffers grow), then 2 x 16 KB again; sizes not multiples of 256."""
    for n in (4099, 262147, 4093):
        src, name = _two_out(n)
        x = rng.standard_normal(n).astype(F)
        a, b = _dispatch_two_out(src, name, x)
        np.testing.assert_array_equal(a, x + 1.0)
        np.testing.assert_array_equal(b, x * 2.0)


def test_ph_dispatch_staging_is_reused_across_threads(rng):
    """Threads that exit hand their staging (stream, device buffers, pinned
    bounce) to the next ones: three waves of 4 threads create at most 4."""
    src, name = _two_out(1000)
    _dispatch_two_out(src, name, np.zeros(1000, F))  # this thread's own
    before = rt.lib().ph_dispatch_staging_count()
    errors = []

    def worker(seed):
        try:
            x = np.random.default_rng(seed).standard_normal(1000).astype(F)
            a, b = _dispatch_two_out(src, name, x)
            if not (np.array_equal(a, x + 1.0) and np.array_equal(b, x * 2.0)):
                errors.append(seed)
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(repr(e))

    for wave in range(3):
        ts = [threading.Thread(target=worker, args=(wave * 4 + t,)) for t in range(4)]
        for th in ts:
            th.start()
        for th in ts:
            th.join(timeout=60)
        assert not any(th.is_alive() for th in ts)
    assert not errors, errors
    assert rt.lib().ph_dispatch_staging_count() - before <= 4
