"""The NumPy interpreter (`.interpret`) against the C oracle (CPU)."""

import numpy as np

import oracle
from palladium_amd.frontend import jnp, lax, pl, random
from palladium_amd.workloads import (
    GS_CFG,
    GBMConfig,
    gbm_call,
    gray_scott_call,
    gray_scott_initial,
    lv_inputs,
    lv_rk4_call,
)


def test_lv_interpret_is_bit_exact_with_oracle():
    args = lv_inputs(3000, 0)
    got = lv_rk4_call(3000, 0.01, 200, track_max=True).interpret(*args)
    want = oracle.lv_rk4(*args, 0.01, 200, track_max=True)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)


def test_gray_scott_interpret_is_bit_exact_with_oracle():
    u0, v0 = gray_scott_initial(40)
    call = gray_scott_call(size=40)
    u, v = u0, v0
    for _ in range(5):
        u, v = call.interpret(u, v)
    wu, wv = oracle.gray_scott(u0, v0, GS_CFG, 5)
    np.testing.assert_array_equal(u, wu)
    np.testing.assert_array_equal(v, wv)


def test_gbm_interpret_bits_path_matches_oracle():
    cfg = GBMConfig(n_steps=8)
    got = gbm_call(cfg, n_paths=512).interpret(random.key(cfg.seed))
    want = oracle.gbm(cfg, 512)
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=1e-4)


def test_random_bits_uniform_fold_in_interpret():
    def kernel(k_ref, bits_ref, fold_ref, u_ref):
        key = random.wrap_key_data(k_ref[...])
        bits_ref[...] = random.bits(key, (16,))
        fold_ref[...] = random.key_data(random.fold_in(key, 17))
        u_ref[...] = random.uniform(key, (16,))

    call = pl.pallas_call(kernel, out_shape=(pl.ShapeDtypeStruct((16,), np.uint32), pl.ShapeDtypeStruct((2,), np.uint32),
                                             pl.ShapeDtypeStruct((16,), np.float32)), interpret=True)
    key = random.key(1234)
    bits, folded, u = call(key)
    np.testing.assert_array_equal(bits, oracle.random_bits(key, 16))
    np.testing.assert_array_equal(folded, oracle.fold_in(key, 17))
    np.testing.assert_array_equal(u, np.array([oracle.bits_to_uniform(b) for b in bits], np.float32))


def test_while_masks_finished_instances():
    # Instance i loops i times; its store happens once, after its own loop.
    def kernel(o_ref):
        i = pl.program_id(0)
        n, acc = lax.while_loop(lambda c: c[0] < i, lambda c: (c[0] + 1, c[1] * 2.0), (0, 1.0))
        o_ref[0] = acc + n.astype(jnp.float32)

    call = pl.pallas_call(kernel, grid=(6,), out_specs=pl.BlockSpec((1,), lambda i: (i,)),
                          out_shape=pl.ShapeDtypeStruct((6,), np.float32), interpret=True)
    np.testing.assert_array_equal(call(), np.array([2.0 ** i + i for i in range(6)], np.float32))


def test_cond_and_switch_per_instance():
    def kernel(o_ref):
        i = pl.program_id(0)
        o_ref[0] = lax.switch(i, [lambda: 10.0, lambda: 20.0, lambda: 30.0]) + lax.cond(i > 1, lambda: 1.0, lambda: 2.0)

    call = pl.pallas_call(kernel, grid=(5,), out_specs=pl.BlockSpec((1,), lambda i: (i,)),
                          out_shape=pl.ShapeDtypeStruct((5,), np.float32), interpret=True)
    np.testing.assert_array_equal(call(), np.array([12, 22, 31, 31, 31], np.float32))


def test_indexed_refs_and_blocks_2d():
    def kernel(x_ref, o_ref):
        i = pl.program_id(0)
        row = x_ref[i, :]
        o_ref[...] = row * 2.0 + x_ref[0, 1]

    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    call = pl.pallas_call(kernel, grid=(3,), in_specs=[pl.BlockSpec((3, 4), lambda i: (0, 0))],
                          out_specs=pl.BlockSpec((None, 4), lambda i: (i, 0)),
                          out_shape=pl.ShapeDtypeStruct((3, 4), np.float32), interpret=True)
    np.testing.assert_array_equal(call(x), x * 2.0 + 1.0)


def test_min_max_order_negative_zero_below_positive_zero():
    """Float min/max, clamp and the max/min reductions order -0 below +0,
    as gfx950's v_min_f32/v_max_f32 do for fminf/fmaxf (NumPy's own
    fmin/fmax return the second operand on equal inputs)."""
    import signed_zero_cases as zc
    from palladium_amd import dtypes

    for dt in (np.float32, dtypes.bfloat16):
        got = zc.call(dt).interpret(*zc.inputs(dt))
        for g, w in zip(got, zc.expected()):
            g = dtypes.to_float(g) if dtypes.is_bf16(g.dtype) else g
            np.testing.assert_array_equal(np.signbit(g), np.signbit(w))
            np.testing.assert_array_equal(g, w)


def test_round_sign_floor_ceil_edge_values():
    """roundf (away), rintf (even), sign with signed zeros and NaN kept,
    floorf/ceilf: zeros, halves, 0.49999997, odd integers past 2^23, inf."""
    import signed_zero_cases as zc

    got = zc.rounding_call().interpret(zc.rounding_inputs())
    for g, w in zip(got, zc.rounding_expected()):
        np.testing.assert_array_equal(g, w)
        np.testing.assert_array_equal(np.signbit(g), np.signbit(w))
