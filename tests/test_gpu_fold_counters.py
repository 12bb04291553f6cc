"""The exact counter fold on the GPU: kernels built with it equal the same
kernels built without it (PALLADIUM_FOLD_COUNTERS=0) bit for bit, under
every math mode, with and without while-loop compaction; under SAFE both
equal the interpreter. Config 2's SAFE counts are checked against the C
oracle in tests/test_gpu_bs3.py."""

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd.frontend import pl
from palladium_amd.trace import trace
from palladium_amd.workloads import bs3_inputs, bs3_vdp_call
from test_fold_counters import _counter_kernel, _random_counter_kernel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mode", ["safe", "fast"])
@pytest.mark.parametrize("compaction", ["1", "0"])
@pytest.mark.parametrize("step,a_cases,b_cases", [(1, (0, 1), (1, 0)), (2, (1, 2), (1, 0))])
def test_folded_counts_equal_unfolded(mode, compaction, step, a_cases, b_cases, monkeypatch):
    n = 4096
    print(f"[fold_counters] mode={mode} compaction={compaction} step={step}", flush=True)
    monkeypatch.setenv("PALLADIUM_WHILE_COMPACTION", compaction)
    x = np.random.default_rng(17).uniform(0.0, 1.0, n).astype(np.float32)
    s = pl.BlockSpec((1,), lambda i: (i,))

    def build():
        return pa.hip_call(_counter_kernel(step, a_cases, b_cases), grid=(n,), in_specs=[s], out_specs=(s, s, s),
                           out_shape=(pl.ShapeDtypeStruct((n,), np.int32),) * 3, math_mode=mode)

    on = build()
    got = on(x)
    monkeypatch.setenv("PALLADIUM_FOLD_COUNTERS", "0")
    off = build()
    assert on.bound(x).hip_source != off.bound(x).hip_source
    want = off(x)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    if mode == "safe":
        for g, w in zip(got, on.interpret(x)):
            np.testing.assert_array_equal(g, w)
    assert np.unique(got[1]).size > 3


def test_bs3_fast_folded_equals_unfolded(monkeypatch):
    n = 4096
    print(f"[fold_counters] bs3 fast n={n}", flush=True)
    args = bs3_inputs(n)
    on = bs3_vdp_call(n, math_mode="fast")
    got = on(*args)
    monkeypatch.setenv("PALLADIUM_FOLD_COUNTERS", "0")
    off = bs3_vdp_call(n, math_mode="fast")
    assert on.bound(*args).hip_source != off.bound(*args).hip_source
    want = off(*args)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(np.asarray(g).view(np.uint32), np.asarray(w).view(np.uint32))


@pytest.mark.parametrize("seed", range(12))
def test_random_counter_loops_equal_the_interpreter(seed, monkeypatch):
    """The fuzz programs of tests/test_fold_counters.py, compiled (SAFE,
    folded where the fold applies): bit-identical to the interpreter."""
    n = 2048
    print(f"[fold_counters] fuzz seed={seed}", flush=True)
    kernel, m = _random_counter_kernel(seed)
    x = np.random.default_rng(seed).uniform(0.0, 1.0, n).astype(np.float32)
    s = pl.BlockSpec((1,), lambda i: (i,))
    f = pa.hip_call(kernel, grid=(n,), in_specs=[s], out_specs=(s,) * m,
                    out_shape=(pl.ShapeDtypeStruct((n,), np.int32),) * m, math_mode="safe")
    for g, w in zip(f(x), f.interpret(x)):
        np.testing.assert_array_equal(g, w)
