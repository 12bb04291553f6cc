"""Loop and carry semantics from the reference's topic tests, on the GPU
under SAFE math against the interpreter bit for bit (and a NumPy closed
form where one exists):
- tests/test_05_loops.py:16-42 (Euler logistic with a scan const),
  70-87 (nested loops), 118-155 (carry swap beside a computed carry),
  157-187 (carry read and alias conflict);
- tests/test_07_preflight.py:108-124 (-inf sentinel running max),
  145-163 (accept/reject inside a loop);
- tests/test_15_control_flow.py:88-107 (while loop rotating its carries),
  in the lane-compacted form and the plain predicated one;
- tests/test_09_indexed_refs.py:91-114 (periodic wraparound indices)."""

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd.frontend import jnp, lax, pl

pytestmark = pytest.mark.gpu
F = np.float32


def _same(f, *args):
    got = f(*args)
    want = f.interpret(*args)
    got, want = (got, want) if isinstance(got, tuple) else ((got,), (want,))
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    return got


def test_euler_logistic_with_a_scan_const(rng):
    dt, steps = 0.01, 100

    def kernel(y0_ref, r_ref, o_ref):
        r = r_ref[...]
        o_ref[...] = lax.fori_loop(0, steps, lambda _, y: y + dt * r * y * (1.0 - y), y0_ref[...])

    f = pa.hip_call(kernel, out_shape=pl.ShapeDtypeStruct((1024,), F), math_mode="safe")
    y0 = rng.uniform(0.1, 0.9, 1024).astype(F)
    r = rng.uniform(0.5, 1.5, 1024).astype(F)
    (got,) = _same(f, y0, r)
    assert np.all(np.abs(got - 1.0) < np.abs(y0 - 1.0))  # flows toward the y = 1 fixed point


def test_nested_loops(rng):
    def kernel(y_ref, o_ref):
        def outer(_, y):
            return lax.fori_loop(0, 10, lambda _, z: z + 0.001 * z, y)

        o_ref[...] = lax.fori_loop(0, 20, outer, y_ref[...])

    f = pa.hip_call(kernel, out_shape=pl.ShapeDtypeStruct((128,), F), math_mode="safe")
    y = rng.uniform(0.5, 1.5, 128).astype(F)
    (got,) = _same(f, y)
    np.testing.assert_allclose(got, y.astype(np.float64) * 1.001 ** 200, rtol=1e-5)


@pytest.mark.parametrize("per_instance", [False, True])
def test_carry_swap_beside_a_computed_carry(per_instance):
    def kernel(a_ref, b_ref, c_ref, ao_ref, bo_ref, co_ref):
        def step(_, c):
            return c[1], c[0], jnp.tanh(c[0] + 0.0 * c[0])

        fa, fb, fc = lax.fori_loop(0, 2, step, (a_ref[...], b_ref[...], c_ref[...]))
        ao_ref[...] = fa
        bo_ref[...] = fb
        co_ref[...] = fc

    n = 16
    shapes = tuple(pl.ShapeDtypeStruct((n,), F) for _ in range(3))
    if per_instance:
        s = pl.BlockSpec((1,), lambda i: (i,))
        f = pa.hip_call(kernel, grid=(n,), in_specs=[s] * 3, out_specs=(s,) * 3, out_shape=shapes, math_mode="safe")
    else:
        f = pa.hip_call(kernel, out_shape=shapes, math_mode="safe")
    a, b, c = np.zeros(n, F), np.ones(n, F), np.zeros(n, F)
    fa, fb, fc = _same(f, a, b, c)
    np.testing.assert_array_equal(fa, a)  # two swaps restore the order
    np.testing.assert_array_equal(fb, b)
    np.testing.assert_array_equal(fc, np.tanh(np.ones(n, F)))


def test_carry_read_and_alias_conflict():
    def kernel(x0_ref, x1_ref, x2_ref, o0_ref, o1_ref, o2_ref):
        def step(_, carry):
            c0, _c1, c2 = carry
            return c2, jnp.tanh(c0 + 0.0 * c0), c0

        f0, f1, f2 = lax.fori_loop(0, 2, step, (x0_ref[...], x1_ref[...], x2_ref[...]))
        o0_ref[...] = f0
        o1_ref[...] = f1
        o2_ref[...] = f2

    f = pa.hip_call(kernel, out_shape=tuple(pl.ShapeDtypeStruct((16,), F) for _ in range(3)), math_mode="safe")
    f0, f1, f2 = _same(f, np.zeros(16, F), np.zeros(16, F), np.ones(16, F))
    np.testing.assert_array_equal(f0, np.zeros(16, F))
    np.testing.assert_array_equal(f1, np.tanh(np.ones(16, F)))
    np.testing.assert_array_equal(f2, np.ones(16, F))


def test_negative_inf_sentinel_running_max(rng):
    def kernel(x_ref, o_ref):
        o_ref[...] = lax.fori_loop(0, 4, lambda i, best: jnp.maximum(best, x_ref[...] - 0.1 * i),
                                   jnp.full((64,), -jnp.inf, F))

    f = pa.hip_call(kernel, out_shape=pl.ShapeDtypeStruct((64,), F), math_mode="safe")
    x = rng.standard_normal(64).astype(F)
    (got,) = _same(f, x)
    np.testing.assert_array_equal(got, x)


def test_accept_reject_inside_a_loop(rng):
    def kernel(y0_ref, r_ref, o_ref):
        r = r_ref[...]

        def step(_, y):
            grown = y + r
            return jnp.where(grown <= 1.0, grown, y)

        o_ref[...] = lax.fori_loop(0, 20, step, y0_ref[...])

    f = pa.hip_call(kernel, out_shape=pl.ShapeDtypeStruct((256,), F), math_mode="safe")
    y0 = rng.uniform(0.0, 0.5, 256).astype(F)
    r = rng.uniform(0.01, 0.2, 256).astype(F)
    (got,) = _same(f, y0, r)
    assert np.all(got <= 1.0)


@pytest.mark.parametrize("n,threadgroup", [(128, None), (2048, None), (2048, 256)])
def test_while_rotating_its_carries(rng, n, threadgroup):
    """Default workgroups emit the loop with lane compaction (at 128
    instances the last workgroup keeps 896 extra lanes); an explicit
    256-lane workgroup gives the plain predicated loop."""
    def kernel(a_ref, o_ref):
        def body(c):
            a, b, k = c
            return b, a + b, k + 1

        a0 = a_ref[0]
        a, b, _ = lax.while_loop(lambda c: c[2] < 5, body, (a0, a0 + 1.0, jnp.int32(0)))
        o_ref[0] = a + b

    s = pl.BlockSpec((1,), lambda i: (i,))
    f = pa.hip_call(kernel, grid=(n,), in_specs=[s], out_specs=s, out_shape=pl.ShapeDtypeStruct((n,), F),
                    math_mode="safe", threadgroup=threadgroup)
    a = rng.standard_normal(n).astype(F)
    assert ("__syncthreads" in f.bound(a).hip_source) == (threadgroup is None)
    (got,) = _same(f, a)
    x, y = a.copy(), a + F(1.0)
    for _ in range(5):
        x, y = y, x + y
    np.testing.assert_array_equal(got, x + y)


def test_periodic_wraparound_indices(rng):
    def kernel(x_ref, o_ref):
        i, j = pl.program_id(0), pl.program_id(1)
        n = 4
        ip = jnp.where(i == n - 1, 0, i + 1)
        im = jnp.where(i != 0, i - 1, n - 1)
        o_ref[i, j] = x_ref[ip, j] + x_ref[im, j]

    blk = pl.BlockSpec((4, 4), lambda i, j: (0, 0))
    f = pa.hip_call(kernel, grid=(4, 4), in_specs=[blk], out_specs=blk, out_shape=pl.ShapeDtypeStruct((4, 4), F),
                    math_mode="safe")
    x = rng.standard_normal((4, 4)).astype(F)
    (got,) = _same(f, x)
    np.testing.assert_array_equal(got, np.roll(x, -1, 0) + np.roll(x, 1, 0))
