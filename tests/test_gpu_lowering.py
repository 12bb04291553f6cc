"""Per-lowering GPU tests, after the reference's tests/test_02..test_15:
each kernel is checked against a NumPy closed form and against the CPU
interpreter (`.interpret`), under SAFE math unless stated."""

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd.frontend import jnp, lax, pl

pytestmark = pytest.mark.gpu

F = np.float32
SDS = pl.ShapeDtypeStruct


def _both(f, *args):
    got = f(*args)
    want = f.interpret(*args)
    if isinstance(got, tuple):
        for g, w in zip(got, want):
            np.testing.assert_array_equal(g, w)
    else:
        np.testing.assert_array_equal(got, want)
    return got


# -- copy / blocks / grids (test_02, test_04) --------------------------------


def test_copy_2d_gridless(rng):
    f = pa.hip_call(lambda x_ref, o_ref: o_ref.__setitem__(Ellipsis, x_ref[...]),
                    out_shape=SDS((3, 5), F), math_mode="safe")
    x = rng.standard_normal((3, 5), dtype=F)
    np.testing.assert_array_equal(_both(f, x), x)


def test_large_gridless_block_runs(rng):
    """4096 elements in one gridless block (reference tests/test_17_robustness.py:
    202-214): one instance walks scratch-resident arrays, results exact."""

    def kernel(x_ref, y_ref, o_ref):
        o_ref[...] = 2.0 * x_ref[...] + y_ref[...]

    f = pa.hip_call(kernel, out_shape=SDS((4096,), F), math_mode="safe")
    x = rng.standard_normal(4096, dtype=F)
    y = rng.standard_normal(4096, dtype=F)
    np.testing.assert_array_equal(_both(f, x, y), F(2.0) * x + y)


def test_blocked_saxpy(rng):
    def kernel(a_ref, x_ref, y_ref, o_ref):
        o_ref[...] = a_ref[0] * x_ref[...] + y_ref[...]

    blk = pl.BlockSpec((8,), lambda i: (i,))
    f = pa.hip_call(kernel, grid=(16,), in_specs=[pl.BlockSpec((1,), lambda i: (0,)), blk, blk],
                    out_specs=blk, out_shape=SDS((128,), F), math_mode="safe")
    a = np.array([1.5], F)
    x, y = rng.standard_normal(128, dtype=F), rng.standard_normal(128, dtype=F)
    np.testing.assert_array_equal(_both(f, a, x, y), (a[0] * x + y).astype(F))


def test_two_d_grid_row_blocks(rng):
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...] * (pl.program_id(0) + 1).astype(jnp.float32) + pl.program_id(1).astype(jnp.float32)

    f = pa.hip_call(kernel, grid=(4, 3), in_specs=[pl.BlockSpec((None, 6), lambda i, j: (i, 0))],
                    out_specs=pl.BlockSpec((None, None, 6), lambda i, j: (i, j, 0)),
                    out_shape=SDS((4, 3, 6), F), math_mode="safe")
    x = rng.standard_normal((4, 6), dtype=F)
    want = x[:, None, :] * np.arange(1, 5, dtype=F)[:, None, None] + np.arange(3, dtype=F)[None, :, None]
    np.testing.assert_array_equal(_both(f, x), want.astype(F))


def test_index_map_arithmetic(rng):
    # Reversed block order: instance i writes block n-1-i.
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...]

    f = pa.hip_call(kernel, grid=(8,), in_specs=[pl.BlockSpec((4,), lambda i: (i,))],
                    out_specs=pl.BlockSpec((4,), lambda i: (7 - i,)), out_shape=SDS((32,), F))
    x = rng.standard_normal(32, dtype=F)
    np.testing.assert_array_equal(_both(f, x), x.reshape(8, 4)[::-1].reshape(-1))


# -- elementwise / preflight (test_03, test_07) --------------------------------


def test_where_abs_the_hard_way(rng):
    f = pa.hip_call(lambda x_ref, o_ref: o_ref.__setitem__(Ellipsis, jnp.where(x_ref[...] > 0.0, x_ref[...], -x_ref[...])),
                    out_shape=SDS((256,), F), math_mode="safe")
    x = rng.standard_normal(256, dtype=F)
    np.testing.assert_array_equal(_both(f, x), np.abs(x))


def test_inf_nan_literals_and_comparisons():
    def kernel(x_ref, o_ref, b_ref):
        x = x_ref[...]
        m = jnp.maximum(x, -jnp.inf)
        o_ref[...] = jnp.where(x > 1e30, jnp.inf, m)
        b_ref[...] = (x != x) | (x >= jnp.inf)

    f = pa.hip_call(kernel, out_shape=(SDS((5,), F), SDS((5,), np.bool_)), math_mode="safe")
    x = np.array([1.0, np.inf, -np.inf, np.nan, 1e31], F)
    o, b = f(x)
    np.testing.assert_array_equal(b, [False, True, False, True, False])
    assert o[1] == np.inf and o[4] == np.inf and o[2] == -np.inf
    assert o[3] == -np.inf  # fmax(NaN, -inf) = -inf: NaN-suppressing like the reference


def test_integer_and_bitwise_ops(rng):
    def kernel(i_ref, u_ref, o_ref, p_ref):
        i, u = i_ref[...], u_ref[...]
        o_ref[...] = (i * 3 + (i // 4) - (i % 7)) ^ (i >> 2)
        p_ref[...] = (u << np.uint32(3)) | (u >> np.uint32(29))

    f = pa.hip_call(kernel, out_shape=(SDS((64,), np.int32), SDS((64,), np.uint32)), math_mode="safe")
    i = rng.integers(-1000, 1000, 64).astype(np.int32)
    u = rng.integers(0, 2**32, 64, dtype=np.uint64).astype(np.uint32)
    o, p = _both(f, i, u)
    np.testing.assert_array_equal(p, ((u << np.uint32(3)) | (u >> np.uint32(29))))


def test_transcendentals_within_ulps(rng):
    def kernel(x_ref, o_ref):
        x = x_ref[...]
        o_ref[...] = jnp.exp(x) + jnp.log(x + 3.0) + jnp.sin(x) * jnp.cos(x) + jnp.tanh(x) + jnp.sqrt(x + 3.0)

    f = pa.hip_call(kernel, out_shape=SDS((512,), F), math_mode="safe")
    x = rng.uniform(-2, 2, 512).astype(F)
    np.testing.assert_allclose(f(x), f.interpret(x), rtol=2e-6, atol=2e-6)


# -- loops (test_05) ---------------------------------------------------------


def test_fori_loop_carry_permutation():
    def kernel(o_ref):
        a, b, c = lax.fori_loop(0, 7, lambda i, c: (c[1], c[2], c[0] + 1.0), (1.0, 2.0, 3.0))
        o_ref[0] = a * 100.0 + b * 10.0 + c

    f = pa.hip_call(kernel, out_shape=SDS((1,), F), math_mode="safe")
    a, b, c = 1.0, 2.0, 3.0
    for _ in range(7):
        a, b, c = b, c, a + 1.0
    np.testing.assert_array_equal(_both(f), [a * 100 + b * 10 + c])


def test_loop_index_and_traced_bounds():
    def kernel(n_ref, o_ref):
        s = lax.fori_loop(0, 10, lambda i, s: s + i.astype(jnp.float32), 0.0)
        t = lax.fori_loop(0, n_ref[0], lambda i, t: t + 2 * i, 0)
        o_ref[0] = s + t.astype(jnp.float32)

    f = pa.hip_call(kernel, out_shape=SDS((1,), F), math_mode="safe")
    np.testing.assert_array_equal(_both(f, np.array([5], np.int32)), [45.0 + 20.0])


def test_vector_carries_in_scan():
    def kernel(x_ref, o_ref):
        def body(c, _):
            return c * 0.5 + jnp.sum(c) * 0.01, None

        v, _ = lax.scan(body, x_ref[...], None, length=6)
        o_ref[...] = v

    f = pa.hip_call(kernel, out_shape=SDS((8,), F), math_mode="safe")
    x = np.arange(8, dtype=F)
    _both(f, x)


# -- indexed refs (test_09) --------------------------------------------------


def test_dynamic_row_index(rng):
    def kernel(x_ref, o_ref):
        i = pl.program_id(0)
        o_ref[0, :] = x_ref[i, :]

    f = pa.hip_call(kernel, grid=(3,), in_specs=[pl.BlockSpec((3, 4), lambda i: (0, 0))],
                    out_specs=pl.BlockSpec((1, 4), lambda i: (i, 0)), out_shape=SDS((3, 4), F))
    x = rng.standard_normal((3, 4), dtype=F)
    np.testing.assert_array_equal(_both(f, x), x)


def test_dslice_window(rng):
    def kernel(x_ref, o_ref):
        i = pl.program_id(0)
        o_ref[...] = x_ref[pl.ds(i * 2, 4)]

    f = pa.hip_call(kernel, grid=(5,), in_specs=[pl.BlockSpec((14,), lambda i: (0,))],
                    out_specs=pl.BlockSpec((4,), lambda i: (i,)), out_shape=SDS((20,), F))
    x = rng.standard_normal(14, dtype=F)
    want = np.concatenate([x[2 * i : 2 * i + 4] for i in range(5)])
    np.testing.assert_array_equal(_both(f, x), want)


def test_fully_scalar_indexed_stencil(rng):
    def kernel(x_ref, o_ref):
        i, j = pl.program_id(0), pl.program_id(1)
        n = 4
        jl = jnp.where(j > 0, j - 1, 0)
        jr = jnp.where(j < n - 1, j + 1, n - 1)
        left = jnp.where(j > 0, x_ref[i, jl], 0.0)
        right = jnp.where(j < n - 1, x_ref[i, jr], 0.0)
        o_ref[i, j] = 2.0 * x_ref[i, j] - left - right

    full = pl.BlockSpec((4, 4), lambda i, j: (0, 0))
    f = pa.hip_call(kernel, grid=(4, 4), in_specs=[full], out_specs=full, out_shape=SDS((4, 4), F), math_mode="safe")
    x = rng.standard_normal((4, 4), dtype=F)
    xp = np.pad(x, ((0, 0), (1, 1)))
    np.testing.assert_array_equal(_both(f, x), (2.0 * x - xp[:, :-2] - xp[:, 2:]).astype(F))


# -- reductions (test_13) ------------------------------------------------------


def test_reductions_over_axes(rng):
    def kernel(x_ref, s_ref, m_ref, n_ref):
        x = x_ref[...]
        s_ref[...] = jnp.sum(x, axis=1)
        m_ref[...] = jnp.max(x, axis=0)
        n_ref[0] = jnp.min(x)

    f = pa.hip_call(kernel, out_shape=(SDS((3,), F), SDS((5,), F), SDS((1,), F)), math_mode="safe")
    x = rng.standard_normal((3, 5), dtype=F)
    s, m, n = _both(f, x)
    np.testing.assert_array_equal(m, x.max(axis=0))
    assert n[0] == x.min()


def test_running_max_sentinel(rng):
    def kernel(x_ref, o_ref):
        m = lax.fori_loop(0, 16, lambda i, m: jnp.maximum(m, x_ref[i]), -jnp.inf)
        o_ref[0] = m

    f = pa.hip_call(kernel, out_shape=SDS((1,), F), math_mode="safe")
    x = rng.standard_normal(16, dtype=F)
    assert _both(f, x)[0] == x.max()


# -- control flow (test_15) ----------------------------------------------------


def test_cond_per_instance(rng):
    def kernel(x_ref, o_ref):
        x = x_ref[...]
        o_ref[...] = lax.cond(pl.program_id(0) % 2 == 0, lambda v: v * 2.0, lambda v: v - 1.0, x)

    blk = pl.BlockSpec((1,), lambda i: (i,))
    f = pa.hip_call(kernel, grid=(64,), in_specs=[blk], out_specs=blk, out_shape=SDS((64,), F), math_mode="safe")
    x = rng.standard_normal(64, dtype=F)
    want = np.where(np.arange(64) % 2 == 0, x * 2.0, x - 1.0).astype(F)
    np.testing.assert_array_equal(_both(f, x), want)


def test_switch_clamps_index():
    def kernel(i_ref, o_ref):
        o_ref[0] = lax.switch(i_ref[0], [lambda: 1.0, lambda: 2.0, lambda: 3.0])

    f = pa.hip_call(kernel, grid=(5,), in_specs=[pl.BlockSpec((1,), lambda i: (i,))],
                    out_specs=pl.BlockSpec((1,), lambda i: (i,)), out_shape=SDS((5,), F))
    np.testing.assert_array_equal(_both(f, np.array([-3, 0, 1, 2, 9], np.int32)), [1, 1, 2, 3, 3])


def test_divergent_while_per_lane():
    def kernel(o_ref):
        i = pl.program_id(0)
        n, acc = lax.while_loop(lambda c: c[0] < i % 37, lambda c: (c[0] + 1, c[1] * 1.1), (0, 1.0))
        o_ref[0] = acc + n.astype(jnp.float32)

    f = pa.hip_call(kernel, grid=(300,), out_specs=pl.BlockSpec((1,), lambda i: (i,)),
                    out_shape=SDS((300,), F), math_mode="safe")
    _both(f)
