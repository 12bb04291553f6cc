"""The GPU parity comparisons can fail: a kernel whose emitted source has
one operation changed (a sign, a stencil neighbour) must disagree with the
oracle where the untouched source agrees bit for bit. Only arithmetic is
altered; every index stays in bounds."""

import numpy as np
import pytest

import oracle
from palladium_amd import runtime as rt
from palladium_amd.emit import emit_hip, launch_geometry
from palladium_amd.trace import trace
from palladium_amd.workloads import GS_CFG, gray_scott_call, gray_scott_initial, lv_inputs, lv_rk4_call

pytestmark = pytest.mark.gpu


def _run(spec, source, host_in, out_shapes):
    geo = launch_geometry(spec)
    k = rt.Kernel(source, spec.name, "safe")
    ins = [rt.Buffer.from_numpy(a) for a in host_in]
    outs = [rt.Buffer.empty(s, np.float32) for s in out_shapes]
    s = rt.Stream()
    k.launch_ptrs(geo.blocks, geo.block, [b.ptr for b in ins + outs], s)
    return [o.to_numpy(s) for o in outs]


def _mutate_once(source, old, new, after='extern "C"'):
    """Replace the first `old` past the marker `after` (the kernel body, not
    the shared prelude)."""
    i = source.index(old, source.index(after))
    return source[:i] + new + source[i + len(old):]


def test_lv_sign_change_is_caught():
    n, dt, steps = 512, 0.01, 100
    args = lv_inputs(n, 0)
    spec = trace(lv_rk4_call(n, dt, steps, math_mode="safe")._staged, *args)
    src = emit_hip(spec, math_mode="safe")
    want = oracle.lv_rk4(*args, dt, steps)
    good = _run(spec, src, args, [(n,), (n,)])
    for g, w in zip(good, want):
        np.testing.assert_array_equal(g, w)
    bad = _run(spec, _mutate_once(src, " - ", " + ", after="for (int _s"), args, [(n,), (n,)])
    assert not np.array_equal(bad[0], want[0])


def test_gray_scott_wrong_neighbour_is_caught():
    size, steps = 64, 1
    u0, v0 = gray_scott_initial(size)
    rng = np.random.default_rng(2)
    u0 = (u0 + rng.random(u0.shape, dtype=np.float32) * 0.1).astype(np.float32)
    spec = trace(gray_scott_call(size=size, math_mode="safe")._staged, u0, v0)
    src = emit_hip(spec, math_mode="safe")
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, steps)
    gu, gv = _run(spec, src, (u0, v0), [(size, size), (size, size)])
    np.testing.assert_array_equal(gu, wu)
    # Read the centre instead of the first neighbour: "(t2) * 64" -> "(_pid0) * 64".
    old = "(int)(t2) * 64"
    assert old in src
    bad_u, _ = _run(spec, _mutate_once(src, old, "(int)(_pid0) * 64"), (u0, v0), [(size, size), (size, size)])
    assert not np.array_equal(bad_u, wu)
