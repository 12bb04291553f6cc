"""Seeded random integer kernels for the differential emitter tests.

Expression trees over int32 and uint32 values mix wrapping arithmetic,
truncating division and remainder (divisors include zero and -1 against
INT_MIN), bitwise operations, shifts by arbitrary amounts (negative and
>= 32 included), min/max, selects, abs/neg and round trips through float32
with saturating conversion. Every operation is defined for every input
(XLA's definitions), so device and interpreter must agree bit for bit.
Half of the programs iterate a data-dependent while loop, which the emitter
predicates.
"""

import numpy as np

import palladium_amd as pa
from palladium_amd.frontend import jnp, lax, pl

I32, U32 = np.int32, np.uint32
SPECIALS = np.array([0, 1, -1, 2, -2, 31, 32, 33, -32, 2**31 - 1, -2**31, -2**31 + 1, 65535, 12345], np.int64)


def _expr(rng, leaves, depth):
    if depth == 0 or rng.random() < 0.2:
        if rng.random() < 0.8:
            return leaves[rng.integers(len(leaves))]
        return int(SPECIALS[rng.integers(len(SPECIALS))]) if rng.random() < 0.5 else int(rng.integers(-50, 50))
    op = rng.integers(16)
    a = _expr(rng, leaves, depth - 1)
    b = _expr(rng, leaves, depth - 1)
    a = a if not isinstance(a, int) else jnp.asarray(np.int32(a))
    if op == 0:
        return a + b
    if op == 1:
        return a - b
    if op == 2:
        return a * b
    if op == 3:
        return lax.div(a, b)
    if op == 4:
        return lax.rem(a, b)
    if op == 5:
        return a & b
    if op == 6:
        return a | b
    if op == 7:
        return a ^ b
    if op == 8:
        return lax.shift_left(a, b)
    if op == 9:
        return lax.shift_right_arithmetic(a, b)
    if op == 10:
        return lax.shift_right_logical(a, b)
    if op == 11:
        return jnp.where(a < b, jnp.maximum(a, b), jnp.minimum(a, b))
    if op == 12:
        return -jnp.abs(a)
    if op == 13:  # unsigned division (divisor made odd, so nonzero), back to int32
        return lax.div(a.astype(jnp.uint32), jnp.asarray(b).astype(jnp.uint32) | 1).astype(jnp.int32)
    if op == 14:  # through float32: scaled, then a saturating conversion back
        return (a.astype(jnp.float32) * 3.5).astype(jnp.int32)
    return ~a


def make_kernel(seed):
    def kernel(a_ref, b_ref, o_ref, u_ref):
        rng = np.random.default_rng(seed)
        a, b = a_ref[...], b_ref[...]
        v = jnp.broadcast_to(jnp.asarray(_expr(rng, [a, b], 4)).astype(jnp.int32), a.shape)
        if seed % 2:
            def body(s):
                i, x = s
                r = np.random.default_rng(seed + 7)
                return i + 1, jnp.broadcast_to(jnp.asarray(_expr(r, [x, i, a], 3)).astype(jnp.int32), x.shape)

            a0 = a_ref[0]
            _, v = lax.while_loop(lambda s: jnp.logical_and(s[0] < 2 + (a0 & 3), s[0] < 6), body, (0, v))
        o_ref[...] = v
        u_ref[...] = v.astype(jnp.uint32) >> (b.astype(jnp.uint32) & 7)

    return kernel


def make_call(seed, n=256, **kw):
    spec = pl.BlockSpec((1,), lambda i: (i,))
    return pa.hip_call(make_kernel(seed), grid=(n,), in_specs=[spec, spec], out_specs=(spec, spec),
                       out_shape=(pl.ShapeDtypeStruct((n,), I32), pl.ShapeDtypeStruct((n,), U32)), **kw)


def make_inputs(seed, n=256):
    rng = np.random.default_rng(5000 + seed)
    pick = rng.random(n) < 0.4
    a = np.where(pick, SPECIALS[rng.integers(len(SPECIALS), size=n)], rng.integers(-2**31, 2**31, n))
    b = np.where(rng.random(n) < 0.4, SPECIALS[rng.integers(len(SPECIALS), size=n)], rng.integers(-100, 100, n))
    return a.astype(np.int64).astype(I32), b.astype(np.int64).astype(I32)
