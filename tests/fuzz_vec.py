"""Seeded random vector kernels for the differential emitter tests.

Each program works on (rows, 4) float32 blocks plus an int32 column, in one
of two launch shapes: one program instance per row (`(1, 4)` blocks) or
64 rows per instance, which the emitter runs lane-parallel (one row per
lane). The grammar mixes element-wise trees with broadcasting, row
reductions (max/min exact in any order; sums over values quantised to
1/8 so that they are exact too), small dot products with a constant
matrix, a `cond` on a data-dependent row predicate, `iota`, integer
hashing (multiply wrap, xor, shifts), a fori_loop and a lockstep
while_loop over `jnp.any` of the rows, so every result is
exactly determined and the GPU must match the interpreter bit for bit
under SAFE math. The same programs run with bfloat16 blocks (each
operation evaluated in float32 and rounded; the quantised sums and dot
products are exact in float32 before their one rounding, so the lane-
parallel butterfly order cannot change them either).
"""

import numpy as np

import palladium_amd as pa
from palladium_amd import dtypes
from palladium_amd.frontend import jnp, lax, pl

F = np.float32
W = 4


def _expr(rng, leaves, depth):
    if depth == 0 or rng.random() < 0.2:
        if rng.random() < 0.85:
            return leaves[rng.integers(len(leaves))]
        return float(np.float32(rng.uniform(-2, 2)))
    op = rng.integers(10)
    a = _expr(rng, leaves, depth - 1)
    b = _expr(rng, leaves, depth - 1)
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
        return jnp.where(a < b, a, b * 0.25)
    if op == 7:
        return jnp.clip(a, -3.0, 3.0)
    if op == 8:
        return -jnp.abs(a)
    return a * 0.75 - b


def _tame(v, shape=None, dt=None):
    v = jnp.clip(v, -50.0, 50.0)
    if dt is not None and v.dtype != dt:  # a lone literal leaf traces as a strong float32
        v = v.astype(dt)
    return v if shape is None else jnp.broadcast_to(v, shape)


def _quant(v):
    return jnp.floor(_tame(v) * 8.0) * 0.125


def make_kernel(seed, lanes=False):
    def kernel(x_ref, y_ref, k_ref, o_ref, s_ref, h_ref):
        rng = np.random.default_rng(seed)
        x, y = x_ref[...], y_ref[...]  # (R, 4)
        dt = x.dtype
        k = k_ref[...]  # (R, 1) int32
        col = lax.broadcasted_iota(jnp.int32, x.shape, 1).astype(dt)
        v = _tame(_expr(rng, [x, y, col * 0.5], 4), x.shape, dt)
        rmax = jnp.broadcast_to(jnp.max(v, axis=1).reshape(v.shape[0], 1), v.shape)
        rmin = jnp.broadcast_to(jnp.min(v, axis=1).reshape(v.shape[0], 1), v.shape)
        v = _tame(_expr(rng, [v, rmax, rmin, x], 3), x.shape, dt)
        # A constant 4x4 matrix with small dyadic entries.
        wi = lax.broadcasted_iota(jnp.int32, (W, W), 0) * 3 + lax.broadcasted_iota(jnp.int32, (W, W), 1)
        wm = ((wi * (seed % 5 + 1)) % 5 - 2).astype(dt) * 0.5
        d = jnp.dot(_quant(v), wm)
        if seed % 3 == 0 and not lanes:
            d = jnp.dot(wm, _quant(v).T).T  # transposes that move the row dim
        elif seed % 3 == 0:
            d = lax.dot_general(_quant(v), wm, (((1,), (1,)), ((), ())))  # v @ wm.T
        q = jnp.sum(_quant(d), axis=1).reshape(v.shape[0], 1)
        pred = jnp.max(q) > 0.0  # a predicate per program instance
        out = lax.cond(pred, lambda t: t * 0.5 + 1.0, lambda t: jnp.abs(t) - 2.0, d)

        def body(i, c):
            return _tame(c * 0.5 + jnp.minimum(c, x) - i.astype(dt) * 0.25, dt=dt)

        out = lax.fori_loop(0, 2 + seed % 4, body, out)

        # lockstep while (examples/02's pattern): iterate until no row of the
        # instance is below a threshold; across lanes this is a cross-lane
        # reduction in the loop condition
        def wcond(s):
            return jnp.logical_and(s[0] < 5, jnp.any(s[1] < 4.0 - (seed % 3)))

        def wbody(s):
            return s[0] + 1, _tame(jnp.abs(s[1]) * 0.75 + 1.25, dt=dt)

        out = lax.while_loop(wcond, wbody, (0, out))[1]
        o_ref[...] = out
        s_ref[...] = q
        h = k * 1103515245 + 12345
        h = h ^ lax.shift_right_logical(h, 7)
        h = h ^ (h << 3)
        h_ref[...] = h + (jnp.sum(q) > 3.0).astype(jnp.int32)

    return kernel


def make_call(seed, rows=512, lanes=False, dtype=F, **kw):
    r = 64 if lanes else 1
    blk = pl.BlockSpec((r, W), lambda i: (i, 0))
    col = pl.BlockSpec((r, 1), lambda i: (i, 0))
    return pa.hip_call(make_kernel(seed, lanes), grid=(rows // r,), in_specs=[blk, blk, col],
                       out_specs=(blk, col, col),
                       out_shape=(pl.ShapeDtypeStruct((rows, W), dtype), pl.ShapeDtypeStruct((rows, 1), dtype),
                                  pl.ShapeDtypeStruct((rows, 1), np.int32)), **kw)


def make_inputs(seed, rows=512, dtype=F):
    rng = np.random.default_rng(1000 + seed)
    x = rng.uniform(-3, 3, (rows, W)).astype(F)
    y = rng.uniform(-3, 3, (rows, W)).astype(F)
    k = rng.integers(-(2**31), 2**31 - 1, (rows, 1)).astype(np.int32)
    if dtypes.is_bf16(dtype):
        x, y = dtypes.from_float(x), dtypes.from_float(y)
    elif np.dtype(dtype) != F:
        x, y = x.astype(dtype), y.astype(dtype)
    return x, y, k
