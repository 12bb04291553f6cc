"""The interpreter's semantics on special values (CPU): integer division
and remainder defined for every input as XLA defines them, saturating
float->int conversion with NaN -> 0, shifts with out-of-range amounts,
wrapping int32 arithmetic. The GPU is compared against the interpreter on
the same grid in tests/test_gpu_edge_values.py."""

import numpy as np

import edge_cases as ec

INT_MIN, INT_MAX = -(2**31), 2**31 - 1


def _run_int():
    a, b = ec.int_pairs()
    n, (a, b) = ec.pad64(a, b)
    names, call = ec.int_call(a.size)
    return a[:n], b[:n], {k: np.asarray(v)[:n] for k, v in zip(names, call.interpret(a, b))}


def test_integer_division_and_remainder_defined_everywhere():
    a, b, out = _run_int()
    a64, b64 = a.astype(np.int64), b.astype(np.int64)
    for i in range(a.size):
        x, y = int(a64[i]), int(b64[i])
        if y == 0:
            q, r = -1, x
        elif x == INT_MIN and y == -1:
            q, r = INT_MIN, 0
        else:
            q = abs(x) // abs(y) * (1 if (x >= 0) == (y > 0) else -1)
            r = x - q * y
        assert out["div"][i] == q and out["rem"][i] == r, (x, y, out["div"][i], out["rem"][i])
        ux, uy = x & 0xFFFFFFFF, y & 0xFFFFFFFF
        assert out["u32_div"][i] == (0xFFFFFFFF if uy == 0 else ux // uy)
        assert out["u32_rem"][i] == (ux if uy == 0 else ux % uy)


def test_int32_arithmetic_wraps_and_shifts_saturate():
    a, b, out = _run_int()
    a64, b64 = a.astype(np.int64), b.astype(np.int64)
    wrap = lambda v: ((v + 2**31) % 2**32) - 2**31  # noqa: E731
    np.testing.assert_array_equal(out["add"], wrap(a64 + b64))
    np.testing.assert_array_equal(out["mul"], wrap(a64 * b64))
    np.testing.assert_array_equal(out["neg"], wrap(-a64))
    np.testing.assert_array_equal(out["abs"], wrap(np.abs(a64)))
    amount = b64 & 0xFFFFFFFF  # shift amounts are read as unsigned
    ua = a64 & 0xFFFFFFFF
    np.testing.assert_array_equal(out["shl"], np.where(amount < 32, wrap(ua << np.minimum(amount, 31)), 0))
    np.testing.assert_array_equal(out["shr_logical"], np.where(amount < 32, wrap(ua >> np.minimum(amount, 31)), 0))
    np.testing.assert_array_equal(out["shr_arith"], a64 >> np.minimum(amount, 31))


def test_float_to_int_saturates_and_sends_nan_to_zero():
    x, y = ec.float_pairs()
    n, (x, y) = ec.pad64(x, y)
    names, call = ec.float_call(x.size)
    out = dict(zip(names, call.interpret(x, y)))
    xs = x[:n].astype(np.float64)
    want_i = np.where(np.isnan(xs), 0, np.clip(np.trunc(np.nan_to_num(xs, posinf=3e38, neginf=-3e38)), INT_MIN, INT_MAX))
    want_u = np.where(np.isnan(xs), 0, np.clip(np.trunc(np.nan_to_num(xs, posinf=3e38, neginf=-3e38)), 0, 2**32 - 1))
    np.testing.assert_array_equal(out["to_i32"][:n], want_i.astype(np.int32))
    np.testing.assert_array_equal(out["to_u32"][:n], want_u.astype(np.uint32))
    np.testing.assert_array_equal(out["bits"][:n], x[:n].view(np.int32))
