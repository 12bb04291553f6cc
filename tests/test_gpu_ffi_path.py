"""hip_call_jit end to end on the GPU with a stand-in for `jax`
(tests/fake_jax.py): FfiCallable builds the attributes and result shapes
exactly as under JAX, and the stand-in's ffi_call dispatches them through
the C ABI's ph_dispatch the way the C++ XLA handler does. Results equal
hip_call's bit for bit (same source, same math mode)."""

import sys

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd import ffi
from palladium_amd.frontend import pl
from palladium_amd.workloads import GS_CFG, gray_scott_initial, gray_scott_kernel, lv_inputs, lv_rk4_kernel

import fake_jax

pytestmark = pytest.mark.gpu
F = np.float32


@pytest.fixture
def jax_standin(monkeypatch):
    mod = fake_jax.make()
    monkeypatch.setitem(sys.modules, "jax", mod)

    def register():
        mod.ffi.register_ffi_target(ffi._TARGET_NAME, mod.ffi.pycapsule(object()), platform="cpu")

    monkeypatch.setattr(ffi, "_register", register)
    return mod


def _both(kernel, **kw):
    return pa.hip_call(kernel, **kw), pa.hip_call_jit(kernel, **kw)


def test_lv_through_the_ffi_path(jax_standin):
    n, dt, steps = 3000, 0.01, 200
    spec = pl.BlockSpec((1,), lambda i: (i,))
    eager, jit = _both(lv_rk4_kernel(dt, steps, True), grid=(n,), in_specs=[spec] * 6, out_specs=(spec,) * 3,
                       out_shape=(pl.ShapeDtypeStruct((n,), F),) * 3, math_mode="safe")
    args = lv_inputs(n, 0)
    for g, w in zip(jit(*args), eager(*args)):
        np.testing.assert_array_equal(g, w)
    target, attrs, vmap = jax_standin.calls[-1]
    assert target == "palladium_hip_dispatch" and vmap is None
    assert (attrs["grid_x"], attrs["grid_y"], attrs["lanes"], attrs["math_mode"]) == (n, 1, 1, 0)


def test_ragged_lane_parallel_blocks_through_the_ffi_path(jax_standin):
    """Config 0's layout: 256-trajectory blocks, ragged tail, lanes = 256."""
    n, dt, steps = 1000, 0.01, 50
    spec = pl.BlockSpec((256,), lambda i: (i,))
    eager, jit = _both(lv_rk4_kernel(dt, steps), grid=(-(-n // 256),), in_specs=[spec] * 6, out_specs=(spec,) * 2,
                       out_shape=(pl.ShapeDtypeStruct((n,), F),) * 2, math_mode="safe")
    args = lv_inputs(n, 3)
    for g, w in zip(jit(*args), eager(*args)):
        np.testing.assert_array_equal(g, w)
    assert jax_standin.calls[-1][1]["lanes"] == 256


def test_two_dimensional_grid_through_the_ffi_path(jax_standin):
    """Gray-Scott on a 2-D grid: grid_x/grid_y attributes, single output
    pair, several calls reusing the cached source."""
    size = 96
    full = pl.BlockSpec((size, size), lambda i, j: (0, 0))
    eager, jit = _both(gray_scott_kernel(GS_CFG, size), grid=(size, size), in_specs=[full, full],
                       out_specs=(full, full), out_shape=(pl.ShapeDtypeStruct((size, size), F),) * 2,
                       math_mode="safe")
    u, v = gray_scott_initial(size)
    eu, ev = u, v
    for _ in range(3):
        u, v = jit(u, v)
        eu, ev = eager(eu, ev)
    np.testing.assert_array_equal(u, eu)
    np.testing.assert_array_equal(v, ev)
    attrs = jax_standin.calls[-1][1]
    assert (attrs["grid_x"], attrs["grid_y"], attrs["grid_z"]) == (size, size, 1)
    assert len(jit._cache) == 1


def test_whole_batch_vmap_is_refused_before_any_dispatch(jax_standin):
    with pytest.raises(ValueError, match="sequential"):
        pa.hip_call_jit(lv_rk4_kernel(0.01, 2), out_shape=pl.ShapeDtypeStruct((8,), F), vmap_method="broadcast_all")
    assert not jax_standin.calls
