"""Differential test of the emitter: seeded random kernels run on the GPU
under SAFE math against the NumPy interpreter (`.interpret`) (and, with
powers and transcendentals added, under REPRODUCIBLE). Under SAFE only IEEE
operations are generated (+ - * / fmin fmax abs neg select), so results
must agree bit for bit. Programs mix expression trees, fori_loops with
permuted carries, switch and bounded while loops (after the reference's
tests/test_fuzz_emitter.py grammar; seeds per test from PALLADIUM_FUZZ_SEEDS
or the reference's PALLADIUM_FUZZ_EXAMPLES, 12 by default). The same programs
run in bfloat16, where each operation is evaluated in float32 and rounded
to bfloat16 on both sides."""

import os

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd import dtypes
from palladium_amd.frontend import jnp, lax, pl

pytestmark = pytest.mark.gpu

F = np.float32


def _expr(rng, leaves, depth, powers=False, transc=False):
    if depth == 0 or rng.random() < 0.25:
        return leaves[rng.integers(len(leaves))] if rng.random() < 0.85 else float(np.float32(rng.uniform(-2, 2)))
    op = rng.integers(16 if transc else (11 if powers else 9))
    a = _expr(rng, leaves, depth - 1, powers, transc)
    b = _expr(rng, leaves, depth - 1, powers, transc)
    if op == 11:
        return jnp.exp(jnp.clip(a, -20.0, 20.0)) * 0.25
    if op == 12:
        return jnp.log(jnp.abs(a) + 0.25)
    if op == 13:
        return jnp.sin(a * b)
    if op == 14:
        return jnp.cos(a) * b
    if op == 15:
        return jnp.tanh(a - b)
    if op == 9:
        return (jnp.abs(a) + 0.5) ** jnp.clip(b, -3.0, 3.0)
    if op == 10:
        return a * b + a * 0.75 - b * b
    if op == 0:
        return a + b
    if op == 1:
        return a - b
    if op == 2:
        return a * b * 0.5
    if op == 3:
        return a / (jnp.abs(b) + 1.0)
    if op == 4:
        return jnp.minimum(a, b)
    if op == 5:
        return jnp.maximum(a, b)
    if op == 6:
        return -jnp.abs(a)
    if op == 7:
        return jnp.where(a < b, a, b * 0.25)
    return jnp.clip(a, -4.0, 4.0)


def _tame(v, dt=F):
    v = jnp.clip(v, -100.0, 100.0)
    return jnp.broadcast_to(v if v.dtype == dt else v.astype(dt), (1,))


def _make_kernel(seed, powers=False, transc=False):
    def kernel(x_ref, y_ref, o_ref, p_ref):
        rng = np.random.default_rng(seed)
        x, y = x_ref[...], y_ref[...]
        dt = x.dtype
        v = _tame(_expr(rng, [x, y], 4, powers, transc), dt)

        def body(i, c):
            a, b, c3 = c
            r = np.random.default_rng(seed + 1)
            na = _tame(_expr(r, [a, b, c3], 3, powers, transc), dt)
            return (b, c3, na) if seed % 2 else (na, a, b)  # permuted carries

        a, b, c = lax.fori_loop(0, 5 + seed % 7, body, (v, x, y))
        k = lax.switch(pl.program_id(0) % 3, [lambda t: t * 2.0, lambda t: t - 1.0, lambda t: jnp.abs(t)], a)
        # an integer carry hashed with division and remainder whose divisor
        # passes through zero (n - 2 at n = 2): defined, so still predicated
        n, w, h = lax.while_loop(lambda s: jnp.logical_and(s[0] < 3 + pl.program_id(0) % 4, s[1] < 50.0),
                                 lambda s: (s[0] + 1, s[1] * 1.5 + 1.0,
                                            (s[2] * 7 + s[0]) // (s[0] - 2) + lax.rem(s[2], s[0] - 2)),
                                 (0, jnp.abs(b), pl.program_id(0) * 13 + 5))
        o_ref[...] = _tame(k + c * 0.5, dt)
        p_ref[...] = w + n.astype(x.dtype) + (h % 16).astype(x.dtype) * 0.0625

    return kernel


@pytest.mark.parametrize("seed", range(int(os.environ.get("PALLADIUM_FUZZ_SEEDS", os.environ.get("PALLADIUM_FUZZ_EXAMPLES", "12")))))
def test_random_program_bit_exact_vs_interpreter(seed):
    n = 300
    rng = np.random.default_rng(100 + seed)
    x = rng.uniform(-3, 3, n).astype(F)
    y = rng.uniform(-3, 3, n).astype(F)
    spec = pl.BlockSpec((1,), lambda i: (i,))
    call = pa.hip_call(_make_kernel(seed), grid=(n,), in_specs=[spec, spec], out_specs=(spec, spec),
                       out_shape=(pl.ShapeDtypeStruct((n,), F),) * 2, math_mode="safe")
    got = call(x, y)
    want = call.interpret(x, y)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)


@pytest.mark.parametrize("dt", [dtypes.bfloat16, np.dtype(np.float16)], ids=["bf16", "f16"])
@pytest.mark.parametrize("seed", range(int(os.environ.get("PALLADIUM_FUZZ_SEEDS", os.environ.get("PALLADIUM_FUZZ_EXAMPLES", "12")))))
def test_random_program_narrow_float_bit_exact_vs_interpreter(seed, dt):
    n = 300
    rng = np.random.default_rng(200 + seed)
    x, y = rng.uniform(-3, 3, n).astype(F), rng.uniform(-3, 3, n).astype(F)
    x, y = (dtypes.from_float(x), dtypes.from_float(y)) if dtypes.is_bf16(dt) else (x.astype(dt), y.astype(dt))
    spec = pl.BlockSpec((1,), lambda i: (i,))
    call = pa.hip_call(_make_kernel(seed), grid=(n,), in_specs=[spec, spec], out_specs=(spec, spec),
                       out_shape=(pl.ShapeDtypeStruct((n,), dt),) * 2, math_mode="safe")
    got = call(x, y)
    want = call.interpret(x, y)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(np.ascontiguousarray(g).view(np.uint16), np.ascontiguousarray(w).view(np.uint16))


@pytest.mark.parametrize("seed", range(int(os.environ.get("PALLADIUM_FUZZ_SEEDS", os.environ.get("PALLADIUM_FUZZ_EXAMPLES", "12")))))
def test_random_program_reproducible_bit_exact_vs_interpreter(seed):
    """The same grammar plus powers, sums of products, exp, log, sin, cos
    and tanh, under REPRODUCIBLE math: the emitter fuses single-use products
    into fused multiply-adds, divides by the correctly rounded reciprocal
    and takes the deterministic pow and transcendentals; the interpreter
    does the same in NumPy (`palladium_amd.exact`), so every result agrees
    bit for bit."""
    n = 300
    rng = np.random.default_rng(300 + seed)
    x = rng.uniform(-3, 3, n).astype(F)
    y = rng.uniform(-3, 3, n).astype(F)
    spec = pl.BlockSpec((1,), lambda i: (i,))
    call = pa.hip_call(_make_kernel(seed, powers=True, transc=True), grid=(n,), in_specs=[spec, spec],
                       out_specs=(spec, spec), out_shape=(pl.ShapeDtypeStruct((n,), F),) * 2, math_mode="reproducible")
    src = call.bound(x, y).hip_source
    assert "__builtin_fmaf" in src[src.index('extern "C"'):]
    got = call(x, y)
    want = call.interpret(x, y)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
