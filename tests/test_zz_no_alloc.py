"""The allocation-free dispatch (`ph_dispatch_noalloc`) against
`ph_dispatch`, through the C ABI: same kernel handle source, same inputs,
bit-identical outputs, on consecutive calls whose operands shrink (the
shared scratch area keeps the previous call's bytes)."""

import ctypes

import numpy as np
import pytest

import oracle
import palladium_amd as pa
from palladium_amd import runtime as rt
from palladium_amd.frontend import pl
from palladium_amd.workloads import F32, lv_inputs, lv_rk4_kernel

pytestmark = pytest.mark.gpu


def _lv_attrs(n, dt, steps):
    spec = pl.BlockSpec((1,), lambda i: (i,))
    f = pa.hip_call_jit(
        lv_rk4_kernel(dt, steps, track_max=True),
        grid=(n,),
        in_specs=[spec] * 6,
        out_specs=tuple([spec] * 3),
        out_shape=tuple(pl.ShapeDtypeStruct((n,), F32) for _ in range(3)),
        name="lv_rk4_noalloc",
        math_mode="safe",
    )
    args = lv_inputs(n, 1)
    return f.ffi_attributes(args), args


def _arrays(bufs, ctype):
    return (ctype * max(len(bufs), 1))(*bufs)


def _err_text(err):
    msg = ctypes.cast(err, ctypes.c_char_p).value
    rt.lib().ph_free_error(err)
    return msg.decode() if msg else ""


def _get_kernel(attrs):
    src = attrs["hip_source"].encode()
    k = ctypes.c_void_p()
    err = ctypes.c_void_p()
    rc = rt.lib().ph_get_kernel(src, len(src), attrs["function_name"].encode(), attrs["math_mode"],
                                ctypes.byref(k), ctypes.byref(err))
    assert rc == 0, _err_text(err)
    return k


def _dispatch(attrs, args, outs):
    src = attrs["hip_source"].encode()
    err = ctypes.c_void_p()
    rc = rt.lib().ph_dispatch(
        src, len(src), attrs["function_name"].encode(), attrs["grid_x"], attrs["grid_y"], attrs["grid_z"],
        attrs["block_x"], attrs["lanes"], attrs["math_mode"],
        _arrays([a.ctypes.data for a in args], ctypes.c_void_p), _arrays([a.nbytes for a in args], ctypes.c_size_t),
        len(args), _arrays([o.ctypes.data for o in outs], ctypes.c_void_p),
        _arrays([o.nbytes for o in outs], ctypes.c_size_t), len(outs), ctypes.byref(err))
    assert rc == 0, _err_text(err)


def _noalloc(kernel, attrs, args, outs, stream=None):
    err = ctypes.c_void_p()
    rc = rt.lib().ph_dispatch_noalloc(
        kernel, attrs["grid_x"], attrs["grid_y"], attrs["grid_z"], attrs["block_x"], attrs["lanes"],
        ctypes.c_void_p(stream), _arrays([a.ctypes.data for a in args], ctypes.c_void_p),
        _arrays([a.nbytes for a in args], ctypes.c_size_t), len(args),
        _arrays([o.ctypes.data for o in outs], ctypes.c_void_p), _arrays([o.nbytes for o in outs], ctypes.c_size_t),
        len(outs), ctypes.byref(err))
    return rc, (_err_text(err) if rc else "")


def test_scratch_area_size():
    assert rt.lib().ph_noalloc_scratch_bytes() == 64 << 20


@pytest.mark.parametrize("sizes", [(100_000, 3_000), (65_536, 1)])
def test_noalloc_equals_dispatch_on_two_calls(sizes):
    dt, steps = 0.01, 200
    stream = rt.Stream()
    for n in sizes:
        print(f"[noalloc] lv_rk4 SAFE n={n} steps={steps}", flush=True)
        attrs, args = _lv_attrs(n, dt, steps)
        want = [np.empty(n, F32) for _ in range(3)]
        _dispatch(attrs, args, want)
        kernel = _get_kernel(attrs)
        got = [np.full(n, np.nan, F32) for _ in range(3)]
        rc, msg = _noalloc(kernel, attrs, args, got, stream.handle)
        assert rc == 0, msg
        for g, w in zip(got, want):
            np.testing.assert_array_equal(g, w)
        # and both against the oracle, bit for bit under SAFE
        ox, oy, om = oracle.lv_rk4(*args, dt, steps, track_max=True)
        np.testing.assert_array_equal(got[0], ox)
        np.testing.assert_array_equal(got[1], oy)
        np.testing.assert_array_equal(got[2], om)


def test_noalloc_on_the_default_stream():
    attrs, args = _lv_attrs(4096, 0.01, 50)
    want = [np.empty(4096, F32) for _ in range(3)]
    _dispatch(attrs, args, want)
    got = [np.empty(4096, F32) for _ in range(3)]
    rc, msg = _noalloc(_get_kernel(attrs), attrs, args, got, None)
    assert rc == 0, msg
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)


def test_noalloc_lane_parallel_kernel():
    """A lane-parallel kernel ((128, 8) @ (8, 4) blocks, one row per lane),
    then a smaller per-instance kernel on the same scratch area."""
    from dot_cases import lane_rows

    f, inputs = lane_rows(np.random.default_rng(4), math_mode="safe")
    jit, _ = lane_rows(np.random.default_rng(4), factory=pa.hip_call_jit, math_mode="safe")
    attrs = jit.ffi_attributes(inputs)
    assert attrs["lanes"] == 128
    want = f.interpret(*inputs)
    ref = np.empty_like(want)
    _dispatch(attrs, inputs, [ref])
    got = np.empty_like(want)
    rc, msg = _noalloc(_get_kernel(attrs), attrs, inputs, [got])
    assert rc == 0, msg
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(got, want)
    attrs2, args2 = _lv_attrs(64, 0.01, 10)
    want2 = [np.empty(64, F32) for _ in range(3)]
    _dispatch(attrs2, args2, want2)
    got2 = [np.empty(64, F32) for _ in range(3)]
    rc, msg = _noalloc(_get_kernel(attrs2), attrs2, args2, got2)
    assert rc == 0, msg
    for g, w in zip(got2, want2):
        np.testing.assert_array_equal(g, w)


def test_noalloc_rejects_operands_beyond_the_scratch_area():
    attrs, args = _lv_attrs(256, 0.01, 1)
    kernel = _get_kernel(attrs)
    big = np.zeros((64 << 20) // 4 + 1, np.float32)
    outs = [np.empty(256, F32) for _ in range(3)]
    rc, msg = _noalloc(kernel, attrs, (big,) + args[1:], outs)
    assert rc == rt.PH_ERR_INVALID
    assert "scratch area" in msg and "operand 0" in msg
    # operands that fit one by one but not together
    half = np.zeros((40 << 20) // 4, np.float32)
    rc, msg = _noalloc(kernel, attrs, (half, half) + args[2:], outs)
    assert rc == rt.PH_ERR_INVALID and "operand 1" in msg
    rc, msg = _noalloc(None, attrs, args, outs)
    assert rc == rt.PH_ERR_INVALID and "null kernel" in msg


def test_noalloc_from_eight_threads_at_once():
    """Eight threads call the allocation-free entry point on one GPU at once,
    each with its own inputs and stream: the per-GPU lock makes them take
    turns on the shared scratch area, so each result equals ph_dispatch's."""
    import threading

    n, dt, steps = 20_000, 0.01, 100
    attrs, _ = _lv_attrs(n, dt, steps)
    kernel = _get_kernel(attrs)
    cases = []
    for t in range(8):
        args = lv_inputs(n, 100 + t)
        want = [np.empty(n, F32) for _ in range(3)]
        _dispatch(attrs, args, want)
        cases.append((args, want, [np.full(n, np.nan, F32) for _ in range(3)], rt.Stream()))
    print(f"[noalloc] 8 threads, lv_rk4 SAFE n={n} steps={steps}", flush=True)
    barrier = threading.Barrier(8)
    results = [None] * 8

    def run(t):
        args, _, got, stream = cases[t]
        barrier.wait()
        for _ in range(3):
            results[t] = _noalloc(kernel, attrs, args, got, stream.handle)
            if results[t][0]:
                return

    threads = [threading.Thread(target=run, args=(t,)) for t in range(8)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads)
    for t, (args, want, got, _) in enumerate(cases):
        assert results[t][0] == 0, results[t][1]
        for g, w in zip(got, want):
            np.testing.assert_array_equal(g, w)
