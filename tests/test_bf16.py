"""bfloat16 on the CPU: the host conversions, the frontend's promotion
rules, the interpreter's float32-then-round semantics, and emission
(reference: tests/test_17_robustness.py:143-195; `src/palladium/
dispatch.py:47-61` ships bf16 bytes as uint16)."""

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd import DispatchError, TraceError, dtypes
from palladium_amd.frontend import jnp, pl

import bf16_cases as cases

BF = dtypes.bfloat16


def _nearest_bf16(f: np.ndarray) -> np.ndarray:
    """Brute force, independent of the bit trick under test: of the two
    bfloat16 neighbours of each finite float32, the one nearer in float64
    (ties: even last mantissa bit); returns bit patterns."""
    u = f.view(np.uint32).astype(np.uint64)
    lo = (u & 0xFFFF0000).astype(np.uint32)
    hi = (lo.astype(np.uint64) + 0x10000).astype(np.uint32)
    lo_v = lo.view(np.float32).astype(np.float64)
    hi_v = hi.view(np.float32).astype(np.float64)
    x = f.astype(np.float64)
    # Past the largest finite bf16 the upper neighbour is infinity; IEEE
    # rounding measures the distance to it as to 2^128 (the next value the
    # exponent range would hold).
    hi_v = np.where(np.isinf(hi_v), np.sign(hi_v) * 2.0**128, hi_v)
    with np.errstate(invalid="ignore", over="ignore"):
        dlo, dhi = np.abs(x - lo_v), np.abs(hi_v - x)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (((lo >> 16) & 1) == 1))
    return np.where(pick_hi, hi >> 16, lo >> 16).astype(np.uint16)


def test_rounding_matches_brute_force_nearest():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 400_000, dtype=np.uint64).astype(np.uint32)
    # exact ties, ties one ulp either side, and the overflow boundary
    ties = (rng.integers(0, 2**16, 2000, dtype=np.uint32) << 16) | 0x8000
    edges = np.array([0x7F7F7FFF, 0x7F7F8000, 0x7F7FFFFF, 0xFF7F8000, 0x00008000, 0x80008001,
                      0x3F80_8000, 0x3F81_8000, 0x0000_7FFF], np.uint32)
    bits = np.concatenate([bits, ties, ties + 1, ties - 1, edges])
    f = bits.view(np.float32)
    f = f[np.isfinite(f)]
    np.testing.assert_array_equal(dtypes.bits_from_f32(f), _nearest_bf16(f))


def test_known_values():
    # 1.0, pi, 1/3, the largest finite value and the smallest subnormal
    got = dtypes.bits_from_f32(np.array([1.0, np.pi, 1 / 3, 3.3895314e38, 9.18355e-41], np.float32))
    np.testing.assert_array_equal(got, [0x3F80, 0x4049, 0x3EAB, 0x7F7F, 0x0001])
    # max finite + half an ulp and beyond -> inf
    assert dtypes.bits_from_f32(np.array([3.4e38], np.float32))[0] == 0x7F80


def test_every_pattern_round_trips_and_nans_stay_nan():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = dtypes.f32_from_bits(bits)
    back = dtypes.bits_from_f32(f)
    nan = np.isnan(f)
    np.testing.assert_array_equal(back[~nan], bits[~nan])
    assert np.all(np.isnan(dtypes.f32_from_bits(back[nan])))
    # a quiet NaN keeps its payload and sign
    assert dtypes.bits_from_f32(dtypes.f32_from_bits(np.array([0x7FC1, 0xFFC3], np.uint16))).tolist() == [0x7FC1, 0xFFC3]


def test_array_helpers_and_scalar_constructor():
    x = dtypes.from_float([1.0, 2.5, -3.0])
    assert dtypes.is_bf16(x.dtype) and x.dtype.itemsize == 2
    np.testing.assert_array_equal(dtypes.to_float(x), [1.0, 2.5, -3.0])
    s = jnp.bfloat16(1.3)
    assert dtypes.is_bf16(np.asarray(s).dtype)
    assert dtypes.scalar_f32(s) == 1.296875
    assert dtypes.name(BF) == "bfloat16" and dtypes.kind(BF) == "f"
    assert not dtypes.is_bf16(np.uint16) and not dtypes.is_bf16(np.float16)
    with pytest.raises(TypeError):
        dtypes.to_float(np.zeros(2, np.uint16))


def _out_dtype(fn, *avals):
    def kernel(*refs):
        refs[-1][...] = fn(*[r[...] for r in refs[:-1]]).astype(jnp.float32)

    seen = {}

    def probe(*refs):
        seen["dt"] = fn(*[r[...] for r in refs[:-1]]).dtype
        kernel(*refs)

    specs = [pl.BlockSpec((4,), lambda i: (i,))] * (len(avals) + 1)
    pa.debug_hip(probe, *[np.zeros(4, a) for a in avals], grid=(1,), in_specs=specs[:-1], out_specs=specs[-1],
                 out_shape=pl.ShapeDtypeStruct((4,), np.float32))
    return dtypes.name(seen["dt"])


def test_promotion_rules_follow_jax():
    assert _out_dtype(lambda a: a * 2.0, BF) == "bfloat16"  # weak float keeps bf16
    assert _out_dtype(lambda a: a + 1, BF) == "bfloat16"  # weak int keeps bf16
    assert _out_dtype(lambda a, b: a + b, BF, np.float32) == "float32"
    assert _out_dtype(lambda a, b: a + b, BF, np.float16) == "float32"
    assert _out_dtype(lambda a, b: a + b, BF, np.int32) == "bfloat16"
    assert _out_dtype(lambda a: a + jnp.bfloat16(1.0), BF) == "bfloat16"
    assert _out_dtype(lambda a: a.astype(jnp.bfloat16), np.float32) == "bfloat16"


def test_interpreter_affine_is_float32_then_round():
    x = dtypes.from_float(np.linspace(-3, 3, 16, dtype=np.float32))
    got = cases.affine().interpret(x)
    assert dtypes.is_bf16(got.dtype)
    xf = dtypes.to_float(x)
    want = dtypes.round_f32(dtypes.round_f32(xf * np.float32(2.0)) + np.float32(1.0))
    np.testing.assert_array_equal(dtypes.to_float(got), want)


def test_interpreter_reductions_accumulate_in_float32_in_order():
    # 1 + 15 * 2^-8: every running float32 sum is exact and the total is a
    # tie between 1 + 7 * 2^-7 and 1 + 8 * 2^-7, so float32 accumulation
    # rounds it to 1.0625; accumulating in bfloat16 would round each
    # 1 + 2^-8 back to 1.0 (a tie to even) and return 1.0.
    row = np.array([1.0] + [2.0**-8] * 15, np.float32)
    x = dtypes.from_float(np.tile(row, 64))
    m = dtypes.from_float(np.eye(16, dtype=np.float32))
    s, mx, d = cases.instance_reduce(math_mode="safe").interpret(x, m)
    np.testing.assert_array_equal(dtypes.to_float(s), np.full(64, 1.0625, np.float32))
    np.testing.assert_array_equal(dtypes.to_float(mx), np.ones(64, np.float32))
    np.testing.assert_array_equal(dtypes.to_float(d), dtypes.to_float(x))  # identity contraction


def test_emitted_source_widens_and_accumulates_in_float():
    x = dtypes.from_float(np.zeros(1024, np.float32))
    m = dtypes.from_float(np.zeros((16, 16), np.float32))

    def kernel(x_ref, m_ref, s_ref, mx_ref, d_ref):
        xx = x_ref[...]
        s_ref[...] = jnp.sum(xx, keepdims=True)
        mx_ref[...] = jnp.max(xx, keepdims=True)
        d_ref[...] = jnp.dot(m_ref[...], xx)

    row = pl.BlockSpec((16,), lambda i: (i,))
    one = pl.BlockSpec((1,), lambda i: (i,))
    src = pa.debug_hip(kernel, x, m, grid=(64,), in_specs=[row, pl.BlockSpec((16, 16), lambda i: (0, 0))],
                       out_specs=(one, one, row),
                       out_shape=(pl.ShapeDtypeStruct((64,), BF),) * 2 + (pl.ShapeDtypeStruct((1024,), BF),))
    assert "const __bf16* __restrict__ arg0_base" in src
    assert "float _acc" in src and "((__bf16)_acc" in src


def test_dispatch_messages_name_bfloat16():
    f = cases.affine()
    with pytest.raises(DispatchError, match="dtype float32 does not match the traced bfloat16"):
        f.bound(dtypes.from_float(np.zeros(16, np.float32)))._check_args((np.zeros(16, np.float32),))
    with pytest.raises(TraceError, match="bfloat16"):
        jnp_kernel_dtype_error()


def jnp_kernel_dtype_error():
    def kernel(x_ref, o_ref):
        o_ref[...] = x_ref[...].astype(np.float64)

    pa.debug_hip(kernel, np.zeros(4, np.float32), out_shape=pl.ShapeDtypeStruct((4,), np.float32))


@pytest.mark.parametrize("make", [cases.arithmetic, cases.transcendental, cases.instance_reduce, cases.copy])
def test_kernels_compile_for_gfx950(make):
    x, y = cases.inputs(0)
    f = make(math_mode="safe")
    args = {cases.arithmetic: (x, y), cases.transcendental: (x,),
            cases.instance_reduce: (x[:1024], dtypes.from_float(np.zeros((16, 16), np.float32))),
            cases.copy: (cases.all_bit_patterns(),)}[make]
    diag = f.explain(*args)
    assert diag.resources is not None and diag.resources.vgpr_spills == 0
