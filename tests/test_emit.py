"""Emitter unit tests (CPU): source shape, hiprtc compilation of every rule,
and the error taxonomy."""

import numpy as np
import pytest

from palladium_amd import runtime as rt
from palladium_amd.emit import emit_hip, rule
from palladium_amd.errors import EmitError, UnsupportedPrimitiveError
from palladium_amd.frontend import jnp, lax, pl, random
from palladium_amd.interpret import interpret_call
from palladium_amd.trace import trace


def _spec(kernel, out_shape, *args, **kw):
    return trace(pl.pallas_call(kernel, out_shape=out_shape, **kw), *args)


def _compile(spec, mode="fast"):
    src = emit_hip(spec)
    return src, rt.compile_code_object(src, spec.name, mode)


F = np.float32


def test_scalar_values_are_registers_not_arrays():
    s1 = pl.BlockSpec((1,), lambda i: (i,))

    def k(x_ref, o_ref):
        x = x_ref[...]
        o_ref[...] = lax.fori_loop(0, 10, lambda i, v: v * 1.5 + 1.0, x)

    src, _ = _compile(_spec(k, pl.ShapeDtypeStruct((64,), F), np.zeros(64, F), grid=(64,), in_specs=[s1], out_specs=s1))
    body = src.split("__launch_bounds__")[1]
    assert "[1]" not in body
    assert "float t" in body


def test_all_elementwise_rules_compile():
    def k(x_ref, y_ref, i_ref, o_ref, oi_ref, ob_ref):
        x, y, i = x_ref[...], y_ref[...], i_ref[...]
        f = [x + y, x - y, x * y, x / y, jnp.minimum(x, y), jnp.maximum(x, y), x ** y, -x, jnp.abs(x),
             jnp.exp(x), jnp.log(x), jnp.sin(x), jnp.cos(x), jnp.sqrt(x), jnp.tanh(x), x ** 3, x ** -2,
             jnp.clamp(0.1, x, 0.9), jnp.where(x < y, x, y), jnp.floor(x), jnp.rsqrt(x), jnp.exp2(x),
             jnp.sign(x), jnp.remainder(x, y), i.astype(jnp.float32)]
        acc = f[0]
        for v in f[1:]:
            acc = acc + v
        o_ref[...] = acc
        u = i.astype(jnp.uint32)
        ii = [i + 1, i * 3, i // 2, i % 5, jnp.minimum(i, 4), i >> 1, i << 2, ~i, i & 7, i | 8, i ^ 3,
              (u >> np.uint32(3)).astype(jnp.int32), lax.bitcast_convert_type(x, jnp.int32)]
        acc_i = ii[0]
        for v in ii[1:]:
            acc_i = acc_i + v
        oi_ref[...] = acc_i
        ob_ref[...] = jnp.logical_and(x <= y, jnp.logical_not(x == y)) | (x >= y) ^ (x != y) | (x > y)

    args = (np.ones(8, F), np.ones(8, F), np.ones(8, np.int32))
    outs = (pl.ShapeDtypeStruct((8,), F), pl.ShapeDtypeStruct((8,), np.int32), pl.ShapeDtypeStruct((8,), np.bool_))
    spec = _spec(k, outs, *args)
    for mode in ("safe", "relaxed", "fast"):
        _compile(spec, mode)


def test_control_flow_and_reductions_compile():
    def k(x_ref, o_ref, m_ref):
        x = x_ref[...]

        def body(c):
            i, v = c
            v = lax.cond(jnp.sum(v) > 1.0, lambda v: v * 0.5, lambda v: v + 1.0, v)
            return i + 1, v

        _, v = lax.while_loop(lambda c: c[0] < 10, body, (0, x))
        v = lax.switch(jnp.argmax if False else 1, [lambda v: v, lambda v: v * 2.0, lambda v: v * 3.0], v)
        o_ref[...] = v
        m_ref[0] = jnp.max(v) + jnp.min(v) + jnp.any(v > 0).astype(jnp.float32) + jnp.all(v > 0).astype(jnp.float32)

    spec = _spec(k, (pl.ShapeDtypeStruct((4,), F), pl.ShapeDtypeStruct((1,), F)), np.ones(4, F))
    src, _ = _compile(spec)
    assert "while (true)" in src


def test_traced_switch_index_compiles():
    def k(x_ref, i_ref, o_ref):
        o_ref[...] = lax.switch(i_ref[0], [lambda v: v, lambda v: v * 2.0, lambda v: -v], x_ref[...])

    spec = _spec(k, pl.ShapeDtypeStruct((4,), F), np.ones(4, F), np.zeros(1, np.int32))
    src, _ = _compile(spec)
    assert "else if" in src


def test_random_rules_compile():
    def k(k_ref, o_ref, f_ref):
        key = random.wrap_key_data(k_ref[...])
        o_ref[...] = random.bits(random.fold_in(key, pl.program_id(0)), (4,))
        f_ref[...] = random.key_data(key)

    spec = _spec(k, (pl.ShapeDtypeStruct((16,), np.uint32), pl.ShapeDtypeStruct((2,), np.uint32)), np.zeros(2, np.uint32),
                 grid=(4,), in_specs=[pl.BlockSpec((2,), lambda i: (0,))],
                 out_specs=(pl.BlockSpec((4,), lambda i: (i,)), pl.BlockSpec((2,), lambda i: (0,))))
    _compile(spec)


def test_noncontiguous_block_rejected():
    call = pl.pallas_call(lambda x, o: None, grid=(2, 2), in_specs=[pl.BlockSpec((4, 4), lambda i, j: (i, j))],
                          out_specs=pl.BlockSpec((4, 4), lambda i, j: (i, j)), out_shape=pl.ShapeDtypeStruct((8, 8), F))
    with pytest.raises(EmitError, match="not contiguous"):
        emit_hip(trace(call, np.zeros((8, 8), F)))


def test_unknown_primitive_raises_and_rule_extends():
    from palladium_amd.frontend.jnp import _stage

    def k(x_ref, o_ref):
        x = x_ref[...]
        o_ref[...] = _stage("my_cube", [x], x.shape, x.dtype)

    spec = _spec(k, pl.ShapeDtypeStruct((1,), F), np.ones(1, F))
    with pytest.raises(UnsupportedPrimitiveError, match="my_cube"):
        emit_hip(spec)

    from palladium_amd.emit import RULES, declare

    @rule("my_cube")
    def _cube(env, cursor, eqn):
        a = env.val(eqn.invars[0])
        declare(env, cursor, eqn.outvars[0], init=f"({a.at('0')} * {a.at('0')} * {a.at('0')})")

    try:
        src = emit_hip(spec)
        assert "* " in src
        rt.compile_code_object(src, spec.name, "fast")
    finally:
        RULES.pop("my_cube", None)


def test_store_into_input_ref_rejected():
    def k(x_ref, o_ref):
        x_ref[...] = o_ref[...]

    spec = _spec(k, pl.ShapeDtypeStruct((1,), F), np.ones(1, F))
    with pytest.raises(EmitError, match="input ref"):
        emit_hip(spec)


def test_block_size_validation():
    spec = _spec(lambda x, o: None, pl.ShapeDtypeStruct((1,), F), np.ones(1, F))
    with pytest.raises(EmitError, match="multiple of 64"):
        emit_hip(spec, block=100)
    assert "__launch_bounds__(512)" in emit_hip(spec, block=512)


def test_ragged_tail_of_independent_rows_is_lowered_masked():
    """Config 0's layout: N = 100,000 in blocks of 256, grid ceil(N/256)."""
    from palladium_amd.emit.lanes import lane_transform
    from palladium_amd.interpret import check_block_bounds

    blk = pl.BlockSpec((256,), lambda i: (i,))

    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...] * 2.0

    call = pl.pallas_call(kernel, grid=(391,), in_specs=[blk], out_specs=blk,
                          out_shape=pl.ShapeDtypeStruct((100_000,), F))
    spec = trace(call, np.zeros(100_000, F))
    check_block_bounds(spec)
    assert lane_transform(spec).rows == 100_000
    src = emit_hip(spec)
    assert "const bool _live = _pid0 * 256 + _lane < 100000;" in src
    assert "if (_live) {" in src
    x = np.arange(100_000, dtype=F)
    np.testing.assert_array_equal(interpret_call(call, x), x * 2)


def test_ragged_blocks_rejected_when_rows_interact():
    """A reduction across the block would see the tail: not lowered."""
    from palladium_amd.interpret import check_block_bounds

    blk = pl.BlockSpec((256,), lambda i: (i,))

    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...] - jnp.max(x_ref[...])

    call = pl.pallas_call(kernel, grid=(391,), in_specs=[blk], out_specs=blk,
                          out_shape=pl.ShapeDtypeStruct((100_000,), F))
    spec = trace(call, np.zeros(100_000, F))
    with pytest.raises(EmitError, match="past the array extent"):
        check_block_bounds(spec)


def test_xcd_remap_is_a_bijection():
    from palladium_amd.emit.core import NUM_XCDS

    for nb in (16, 17, 391, 3907, 65536):
        per, rem = divmod(nb, NUM_XCDS)
        seen = set()
        for b in range(nb):
            xcd, slot = b % NUM_XCDS, b // NUM_XCDS
            blk = xcd * (per + 1) + slot if xcd < rem else rem * (per + 1) + (xcd - rem) * per + slot
            seen.add(blk)
        assert seen == set(range(nb))


def test_two_d_tile_order_is_a_bijection():
    from palladium_amd.emit.core import _tile2d

    for grid, block in (((64, 128), 256), ((4096, 4096), 256), ((8, 64), 512)):
        tile = _tile2d(grid, block)
        assert tile is not None
        ti, tj = tile
        tiles_j = grid[1] // tj
        nblk = grid[0] * grid[1] // block
        if nblk > 4096:
            continue
        seen = set()
        for blk in range(nblk):
            tw, th = blk % tiles_j, blk // tiles_j
            for t in range(block):
                seen.add((th * ti + t // tj, tw * tj + t % tj))
        assert seen == {(i, j) for i in range(grid[0]) for j in range(grid[1])}


def test_two_d_tile_only_when_it_divides():
    from palladium_amd.emit.core import _tile2d

    assert _tile2d((3, 128), 256) is None  # rows not a multiple of 4
    assert _tile2d((8, 100), 256) is None  # cols not a multiple of 64
    assert _tile2d((8,), 256) is None


def test_two_d_threadgroup_sets_the_instance_tile():
    """A 2-D threadgroup (x, y) tiles a 2-D grid with x instances of
    program_id(0) by y of program_id(1) per workgroup, as Metal's
    threadsPerThreadgroup does for the reference; one that does not divide
    the grid keeps the row-major order. The workgroup size is x * y."""
    import palladium_amd as pa
    from palladium_amd.dispatch import _block_of, _tile_of

    def k(x_ref, o_ref):
        i, j = pl.program_id(0), pl.program_id(1)
        o_ref[i, j] = x_ref[i, j] * 2.0 + (i * 64 + j).astype(jnp.float32)

    n = 64
    x = np.arange(n * n, dtype=np.float32).reshape(n, n)
    full = pl.BlockSpec((n, n), lambda i, j: (0, 0))
    kw = dict(grid=(n, n), in_specs=[full], out_specs=full, out_shape=pl.ShapeDtypeStruct((n, n), np.float32))
    assert _tile_of((16, 16)) == (16, 16) and _tile_of((256,)) is None and _tile_of((8, 8, 4)) is None
    assert _block_of((16, 16)) == 256
    src = pa.debug_hip(k, x, threadgroup=(16, 16), **kw)
    assert "threadIdx.x / 16u" in src and "threadIdx.x % 16u" in src
    default = pa.debug_hip(k, x, **kw)
    assert "threadIdx.x / 64u" in default
    ragged = pa.debug_hip(k, x, threadgroup=(48, 4), **kw)   # 48 does not divide 64
    assert "threadIdx.x / 4u" not in ragged


def test_empty_grid_is_a_clear_error_and_interprets_to_empty():
    """A grid with no program instances cannot launch: emission names the
    grid instead of handing the runtime a zero-block launch, while the
    interpreter returns the empty result."""
    import palladium_amd as pa
    from palladium_amd.errors import EmitError

    def k(x_ref, o_ref):
        o_ref[...] = x_ref[...] * 2.0

    s = pl.BlockSpec((1,), lambda i: (i,))
    x = np.zeros(0, np.float32)
    f = pa.hip_call(k, grid=(0,), in_specs=[s], out_specs=s, out_shape=pl.ShapeDtypeStruct((0,), np.float32))
    assert np.asarray(f.interpret(x)).shape == (0,)
    with pytest.raises(EmitError, match="no program instances"):
        f.explain(x, compile=False)
