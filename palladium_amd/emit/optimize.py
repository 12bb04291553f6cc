"""FAST-math jaxpr rewrites applied before emission.

Under FAST the backend may reassociate float arithmetic (the reference's
FAST contract, `src/palladium/__init__.py:203-209`). One rewrite pays off on
the ODE right-hand sides this backend is built for: factoring a common
multiplicand out of a sum or difference of products,

    a*x - (b*x)*y   ->   x * (a - b*y)        (one multiply and one FMA)
    (c*x)*y - d*y   ->   y * (c*x - d)

which removes one operation per term pair and leaves the rest in FMA form.
The compiler finds this for some terms on its own but not across the RK4
stages; doing it on the jaxpr makes the kernel ~6 % shorter. Only
single-use product chains are rewritten (no value is recomputed), and only
equal-shaped float operands (no broadcasting).

A second rewrite shortens power-law step-size controllers (the PI
controller of `tests/test_08_adaptive.py:76-122`,
`factor = safety * (1/err)**c1 * prev**c2`), whose chain of reciprocal,
two branchy `pow` calls and multiplies lies on the serial path from one
adaptive attempt to the next:

    pow(x, c)              ->  exp2(c * log2(x))      (c a non-integer literal)
    log2(1 / y)            ->  -log2(y)
    exp2(a) * exp2(b)      ->  exp2(a + b)            (single-use exp2 values)
    k * exp2(a)            ->  exp2(log2(k) + a)      (k a positive literal)

so the controller costs one hardware log2 on the chain, FMAs and one
hardware exp2. For a non-integer exponent `pow(x, c)` and `exp2(c*log2 x)`
agree on every special operand (finite negative x gives NaN, +-0 gives 0
or inf, +inf gives inf or 0, NaN propagates) except x = -inf, where pow
gives +inf or +0 and log2 NaN: a base not provably non-negative from its
producer (max with a non-negative operand, abs, exp, sqrt, sums, products
and quotients of such values, selects among them, and while-loop carries
that start and stay so) has -inf read as +inf first, which also keeps
`log2(1/y) = -log2(y)` exact at y = -0 and y = -inf. The results differ by the rounding of the log and exp,
within FAST's approximate-transcendental contract.
"""

from __future__ import annotations

import os
from typing import Any

import numpy as np

from palladium_amd.ir import ClosedJaxpr, Jaxpr, JaxprEqn, Literal, ShapedArray, Var, primitive

__all__ = ["carry_logs", "contract_products", "drop_dead_code", "drop_redundant_clamps", "factor_common_products", "fast_rewrites", "funnel_shifts",
           "power_laws_to_exp2", "reuse_affine_shifts", "share_pow_logs", "fold_counters"]


def _same(a: Any, b: Any) -> bool:
    if isinstance(a, Literal) and isinstance(b, Literal):
        return a.val == b.val and a.aval.dtype == b.aval.dtype
    return a is b


def _rewrite_sub(v: Any, fn: Any = None) -> Any:
    fn = fn or factor_common_products
    if isinstance(v, ClosedJaxpr):
        return ClosedJaxpr(fn(v.jaxpr), v.consts)
    if isinstance(v, Jaxpr):
        return fn(v)
    if isinstance(v, tuple) and v and all(isinstance(b, ClosedJaxpr) for b in v):
        return tuple(ClosedJaxpr(fn(b.jaxpr), b.consts) for b in v)
    return v


def fast_rewrites(jaxpr: Jaxpr) -> Jaxpr:
    """Every FAST-only rewrite, in order."""
    j = factor_common_products(carry_logs(power_laws_to_exp2(drop_redundant_clamps(jaxpr))))
    return j if os.environ.get("PALLADIUM_AFFINE_SHIFTS") == "0" else reuse_affine_shifts(j)


def _lower_bound(v: Any, producer: dict) -> float | None:
    """A float32 lower bound of `v` that holds bit for bit, from the ops
    that made it: JAX's uniform construction (bits >> 9 | 0x3F800000,
    bitcast: [1, 2)), then subtraction, addition of literals and
    multiplication by a positive literal (round-to-nearest is monotonic,
    so applying the op to the bound bounds the result)."""
    e = producer.get(v)
    if e is None:
        return None
    name = e.primitive.name
    if name == "bitcast_convert_type" and np.dtype(v.aval.dtype) == np.float32:
        o = producer.get(e.invars[0])
        if o is not None and o.primitive.name == "or":
            a, b = o.invars
            if isinstance(a, Literal):
                a, b = b, a
            sh = producer.get(a)
            if (isinstance(b, Literal) and int(b.val) == 0x3F800000 and sh is not None
                    and sh.primitive.name == "shift_right_logical" and isinstance(sh.invars[1], Literal)
                    and int(sh.invars[1].val) >= 9):
                return 1.0
        return None
    if name in ("sub", "add", "mul") and isinstance(e.invars[1], Literal) and isinstance(e.invars[0], Var):
        lb = _lower_bound(e.invars[0], producer)
        c = _f32_literal(e.invars[1])
        if lb is None or c is None:
            return None
        with np.errstate(all="ignore"):
            if name == "sub":
                return float(np.float32(lb) - np.float32(c))
            if name == "add":
                return float(np.float32(lb) + np.float32(c))
            if c > 0:
                return float(np.float32(lb) * np.float32(c))
    return None


def drop_redundant_clamps(jaxpr: Jaxpr) -> Jaxpr:
    """`max(c, x)` with x provably >= c is x: the clamp `jax.random.uniform`
    stages after mapping random bits onto [minval, maxval) can never act,
    and the compiler cannot see it from the bit manipulation."""
    producer = {ov: e for e in jaxpr.eqns for ov in e.outvars}
    subst: dict[Any, Any] = {}
    new_eqns: list[JaxprEqn] = []
    for e in jaxpr.eqns:
        params = {k: _rewrite_sub(v, drop_redundant_clamps) for k, v in e.params.items()}
        invars = [subst.get(a, a) if isinstance(a, Var) else a for a in e.invars]
        e = JaxprEqn(invars, e.outvars, e.primitive, params)
        if e.primitive.name == "max" and len(e.outvars) == 1:
            a, b = e.invars
            if isinstance(a, Var) and isinstance(b, Literal):
                a, b = b, a
            c = _f32_literal(a)
            if (c is not None and isinstance(b, Var) and np.dtype(b.aval.dtype) == np.float32
                    and tuple(b.aval.shape) == tuple(e.outvars[0].aval.shape)):
                lb = _lower_bound(b, producer)
                if lb is not None and lb >= c:
                    subst[e.outvars[0]] = b
                    continue
        new_eqns.append(e)
    outvars = [subst.get(o, o) if isinstance(o, Var) else o for o in jaxpr.outvars]
    return Jaxpr(jaxpr.constvars, jaxpr.invars, outvars, new_eqns)


def _use_counts(jaxpr: Jaxpr) -> dict[Any, int]:
    uses: dict[Any, int] = {}
    for e in jaxpr.eqns:
        for a in e.invars:
            if isinstance(a, Var):
                uses[a] = uses.get(a, 0) + 1
    for o in jaxpr.outvars:
        if isinstance(o, Var):
            uses[o] = uses.get(o, 0) + 2
    return uses


def _f32_literal(v: Any) -> float | None:
    if isinstance(v, Literal) and np.dtype(v.aval.dtype) == np.float32 and not v.aval.shape:
        x = float(np.float32(v.val))
        return x if np.isfinite(x) else None
    return None


def _non_negative(v: Any, producer: dict, known: frozenset = frozenset()) -> bool:
    """Whether `v` is provably >= 0 or NaN (never -inf) from the ops that
    made it; `known` holds variables already proven so (loop carries)."""
    if isinstance(v, Literal):
        x = _f32_literal(v)
        return x is not None and x >= 0
    if v in known:
        return True
    e = producer.get(v)
    if e is None:
        return False
    name = e.primitive.name
    if name in ("abs", "exp", "exp2", "sqrt"):
        return True
    if name == "max":
        return any(_non_negative(a, producer, known) for a in e.invars)
    if name in ("add", "mul", "div", "min", "broadcast_in_dim", "reshape", "squeeze"):
        return all(_non_negative(a, producer, known) for a in e.invars)
    if name == "select_n":
        return all(_non_negative(a, producer, known) for a in e.invars[1:])
    return False


def _nonneg_carries(e: JaxprEqn, producer: dict, known: frozenset) -> tuple[frozenset, set]:
    """Body invars of a `while` that are provably >= 0 or NaN on every
    iteration: operands non-negative outside, and carries whose initial
    value is and whose update keeps them so (largest fixed point)."""
    cn, bn = int(e.params["cond_nconsts"]), int(e.params["body_nconsts"])
    body = getattr(e.params["body_jaxpr"], "jaxpr", e.params["body_jaxpr"])
    consts, carries = e.invars[cn:cn + bn], e.invars[cn + bn:]
    bconsts, bcarries = body.invars[:bn], body.invars[bn:]
    base = {bv for bv, ov in zip(bconsts, consts) if _non_negative(ov, producer, known)}
    cand = {k for k, iv in enumerate(carries) if _non_negative(iv, producer, known)}
    bprod = {ov: x for x in body.eqns for ov in x.outvars}
    while True:
        assumed = frozenset(base | {bcarries[k] for k in cand})
        keep = {k for k in cand if _non_negative(body.outvars[k], bprod, assumed)}
        if keep == cand:
            return assumed, cand
        cand = keep


def power_laws_to_exp2(jaxpr: Jaxpr, known: frozenset = frozenset()) -> Jaxpr:
    """Rewrite float32 `pow` by non-integer literal exponents, and products
    of the results, into `exp2` of a linear combination of `log2`s.
    `known`: variables proven >= 0 or NaN by the caller (while carries)."""
    uses = _use_counts(jaxpr)
    producer = {ov: e for e in jaxpr.eqns for ov in e.outvars}
    exp2_arg: dict[Any, Any] = {}      # outvar of an exp2 made here -> its operand
    exp2_eqn: dict[Any, JaxprEqn] = {}
    new_eqns: list[JaxprEqn] = []

    def lit(x: float) -> Literal:
        return Literal(np.float32(x), ShapedArray((), np.float32, weak_type=True))


    def f32(v: Any) -> bool:
        return np.dtype(getattr(v.aval, "dtype", np.float64)) == np.float32

    for e in jaxpr.eqns:
        if e.primitive.name == "while":
            inner, idx = _nonneg_carries(e, producer, known)
            known = known | {e.outvars[k] for k in idx}   # the loop's results stay so
            params = dict(e.params)
            params["body_jaxpr"] = _rewrite_sub(e.params["body_jaxpr"], lambda j: power_laws_to_exp2(j, inner))
            params["cond_jaxpr"] = _rewrite_sub(e.params["cond_jaxpr"], power_laws_to_exp2)
        else:
            params = {k: _rewrite_sub(v, power_laws_to_exp2) for k, v in e.params.items()}
        e = JaxprEqn(e.invars, e.outvars, e.primitive, params)
        name = e.primitive.name
        out = e.outvars[0] if len(e.outvars) == 1 else None
        if name == "pow" and out is not None and f32(out) and isinstance(e.invars[0], Var):
            c = _f32_literal(e.invars[1])
            x = e.invars[0]
            if c is not None and c != int(c) and tuple(x.aval.shape) == tuple(out.aval.shape):
                aval = ShapedArray(out.aval.shape, np.float32)
                src = producer.get(x)
                if (src is not None and src.primitive.name == "div" and _f32_literal(src.invars[0]) == 1.0
                        and isinstance(src.invars[1], Var)
                        and tuple(src.invars[1].aval.shape) == tuple(out.aval.shape)):
                    x, c = src.invars[1], -c      # log2(1/y) = -log2(y)
                if not _non_negative(x, producer, known):
                    # pow(-inf, c) is +inf or +0, log2(-inf) is NaN: read -inf as +inf
                    is_ninf, xs = Var(ShapedArray(out.aval.shape, np.bool_)), Var(aval)
                    new_eqns.append(JaxprEqn([x, lit(-np.inf)], [is_ninf], primitive("eq"), {}))
                    new_eqns.append(JaxprEqn([is_ninf, x, lit(np.inf)], [xs], primitive("select_n"), {}))
                    x = xs
                lg, m = Var(aval), Var(aval)
                new_eqns.append(JaxprEqn([x], [lg], primitive("log2"), {}))
                new_eqns.append(JaxprEqn([lit(c), lg], [m], primitive("mul"), {}))
                ex = JaxprEqn([m], [out], primitive("exp2"), {})
                new_eqns.append(ex)
                exp2_arg[out], exp2_eqn[out] = m, ex
                continue
        if name == "mul" and out is not None and f32(out):
            a, b = e.invars
            shape = tuple(out.aval.shape)

            def single_exp2(v: Any) -> bool:
                return (isinstance(v, Var) and v in exp2_arg and uses.get(v, 0) == 1
                        and tuple(v.aval.shape) == shape)

            terms = None
            if single_exp2(a) and single_exp2(b):
                terms = (exp2_arg[a], exp2_arg[b], (a, b))
            else:
                for k, v in ((a, b), (b, a)):
                    kv = _f32_literal(k)
                    if kv is not None and kv > 0 and single_exp2(v):
                        terms = (lit(float(np.log2(np.float64(kv)))), exp2_arg[v], (v,))
                        break
            if terms is not None:
                p, q, gone = terms
                dead = {id(exp2_eqn[g]) for g in gone}
                new_eqns = [x for x in new_eqns if id(x) not in dead]
                aval = ShapedArray(shape, np.float32)
                ssum = Var(aval)
                new_eqns.append(JaxprEqn([p, q], [ssum], primitive("add"), {}))
                ex = JaxprEqn([ssum], [out], primitive("exp2"), {})
                new_eqns.append(ex)
                exp2_arg[out], exp2_eqn[out] = ssum, ex
                continue
        new_eqns.append(e)
    return Jaxpr(jaxpr.constvars, jaxpr.invars, jaxpr.outvars, new_eqns)


def factor_common_products(jaxpr: Jaxpr) -> Jaxpr:
    """Return a new jaxpr with `p*f ± q*f` rewritten to `f*(p ± q)`."""
    uses: dict[Any, int] = {}
    for e in jaxpr.eqns:
        for a in e.invars:
            if isinstance(a, Var):
                uses[a] = uses.get(a, 0) + 1
    for o in jaxpr.outvars:
        if isinstance(o, Var):
            uses[o] = uses.get(o, 0) + 2
    producer = {ov: e for e in jaxpr.eqns for ov in e.outvars}

    def is_float(v: Any) -> bool:
        return getattr(v.aval, "dtype", None) is not None and v.aval.dtype.kind == "f"

    def factors(t: Any, shape: tuple, dead: list) -> list[Any]:
        e = producer.get(t) if isinstance(t, Var) else None
        if (e is not None and e.primitive.name == "mul" and uses.get(t, 0) == 1
                and all(isinstance(x, Literal) or tuple(x.aval.shape) == shape for x in e.invars)):
            dead.append(e)
            return factors(e.invars[0], shape, dead) + factors(e.invars[1], shape, dead)
        return [t]

    new_eqns: list[JaxprEqn] = []
    for e in jaxpr.eqns:
        params = {k: _rewrite_sub(v) for k, v in e.params.items()}
        e = JaxprEqn(e.invars, e.outvars, e.primitive, params)
        name = e.primitive.name
        out = e.outvars[0] if e.outvars else None
        if name in ("add", "sub") and out is not None and is_float(out):
            shape = tuple(out.aval.shape)
            p, q = e.invars
            if all(isinstance(x, Var) and tuple(x.aval.shape) == shape for x in (p, q)):
                dp: list = []
                dq: list = []
                fp = factors(p, shape, dp)
                fq = factors(q, shape, dq)
                common = None
                if len(fp) > 1 and len(fq) > 1:
                    for f in fp:
                        if any(_same(f, g) for g in fq):
                            common = f
                            break
                if common is not None:
                    rp = list(fp)
                    rp.pop(next(i for i, f in enumerate(rp) if _same(f, common)))
                    rq = list(fq)
                    rq.pop(next(i for i, f in enumerate(rq) if _same(f, common)))
                    aval = ShapedArray(shape, out.aval.dtype)
                    staged: list[JaxprEqn] = []

                    def product(terms: list[Any]) -> Any:
                        acc = terms[0]
                        for t in terms[1:]:
                            v = Var(aval)
                            staged.append(JaxprEqn([acc, t], [v], primitive("mul"), {}))
                            acc = v
                        return acc

                    a = product(rp)
                    b = product(rq)
                    inner = Var(aval)
                    staged.append(JaxprEqn([a, b], [inner], primitive(name), {}))
                    staged.append(JaxprEqn([common, inner], [out], primitive("mul"), {}))
                    # The product eqns feeding this one were emitted earlier in
                    # `new_eqns`; drop them now that nothing reads them.
                    dead_outs = {d.outvars[0] for d in dp + dq}
                    new_eqns = [x for x in new_eqns if not (x.outvars and x.outvars[0] in dead_outs)]
                    new_eqns.extend(staged)
                    continue
        new_eqns.append(e)
    return Jaxpr(jaxpr.constvars, jaxpr.invars, jaxpr.outvars, new_eqns)


def _closed_like(orig: Any, jaxpr: Jaxpr) -> Any:
    return ClosedJaxpr(jaxpr, orig.consts) if isinstance(orig, ClosedJaxpr) else jaxpr


def share_pow_logs(jaxpr: Jaxpr) -> Jaxpr:
    """SAFE rewrite, exact: `pow(x, y)` is `pow_with_log(x, y, pow_log(x))`
    bit for bit (the deterministic power splits into the double log2 of its
    base and the rest), so a while loop whose body takes the power of a
    carry `c` and of a value `v`, and updates the carry as
    `c' = select_n(p, c, v)` (either case order), can carry `pow_log(c)`
    beside `c`: the body uses the carried log for `c`'s powers, computes
    `pow_log(v)` once for all of `v`'s powers, and selects the next log as
    it selects the next carry. A power-law step-size controller
    (`tests/test_08_adaptive.py:76-122` of the reference:
    `factor = safety * inv_err**c1 * prev**c2`, `prev = where(accept,
    inv_err, prev)`) then computes one log per attempt instead of two."""
    new_eqns: list[JaxprEqn] = []
    for e in jaxpr.eqns:
        params = {k: _rewrite_sub(v, share_pow_logs) for k, v in e.params.items()}
        e = JaxprEqn(e.invars, e.outvars, e.primitive, params)
        if e.primitive.name == "while":
            pre, e = _share_while(e)
            new_eqns += pre
        new_eqns.append(e)
    return Jaxpr(jaxpr.constvars, jaxpr.invars, jaxpr.outvars, new_eqns)


def _f64(shape: tuple) -> ShapedArray:
    return ShapedArray(shape, np.float64)


def _share_while(e: JaxprEqn) -> tuple[list[JaxprEqn], JaxprEqn]:
    cn, bn = int(e.params["cond_nconsts"]), int(e.params["body_nconsts"])
    body = getattr(e.params["body_jaxpr"], "jaxpr", e.params["body_jaxpr"])
    cond = getattr(e.params["cond_jaxpr"], "jaxpr", e.params["cond_jaxpr"])
    carries = body.invars[bn:]
    producer = {ov: x for x in body.eqns for ov in x.outvars}

    def f32_scalarish(v: Any) -> bool:
        return isinstance(v, Var) and np.dtype(v.aval.dtype) == np.float32

    bases = {x.invars[0] for x in body.eqns if x.primitive.name == "pow" and f32_scalarish(x.invars[0])}
    found = []  # (carry index, carry var, other case, select eqn)
    for k, c in enumerate(carries):
        if c not in bases:
            continue
        sel = producer.get(body.outvars[k])
        if sel is None or sel.primitive.name != "select_n" or len(sel.invars) != 3:
            continue
        if np.dtype(sel.invars[0].aval.dtype) != np.bool_:
            continue
        cases = sel.invars[1:]
        others = [v for v in cases if v is not c]
        if len(others) != 1 or sum(v is c for v in cases) != 1:
            continue
        v = others[0]
        if v not in bases or tuple(v.aval.shape) != tuple(c.aval.shape):
            continue
        found.append((k, c, v, sel))
    if not found:
        return [], e
    log_of: dict[Any, Any] = {}
    new_in = []
    for k, c, _, _ in found:
        log_of[c] = Var(_f64(tuple(c.aval.shape)))
        new_in.append(log_of[c])
    wanted = {v for _, _, v, _ in found}
    eqns: list[JaxprEqn] = []
    for x in body.eqns:
        if x.primitive.name == "pow" and x.invars[0] in (set(log_of) | wanted):
            b = x.invars[0]
            if b not in log_of:  # first power of v: its log, once
                log_of[b] = Var(_f64(tuple(b.aval.shape)))
                eqns.append(JaxprEqn([b], [log_of[b]], primitive("pow_log"), {}))
            eqns.append(JaxprEqn([b, x.invars[1], log_of[b]], x.outvars, primitive("pow_with_log"), {}))
            continue
        eqns.append(x)
    new_out = []
    for k, c, v, sel in found:
        nxt = Var(_f64(tuple(c.aval.shape)))
        cases = [log_of[c] if u is c else log_of[v] for u in sel.invars[1:]]
        eqns.append(JaxprEqn([sel.invars[0], *cases], [nxt], primitive("select_n"), {}))
        new_out.append(nxt)
    new_body = Jaxpr(body.constvars, body.invars + new_in, body.outvars + new_out, eqns)
    new_cond = Jaxpr(cond.constvars, cond.invars + [Var(_f64(tuple(c.aval.shape))) for _, c, _, _ in found],
                     cond.outvars, cond.eqns)
    pre, inits = [], []
    for k, c, _, _ in found:
        init = e.invars[cn + bn + k]
        lv = Var(_f64(tuple(c.aval.shape)))
        pre.append(JaxprEqn([init], [lv], primitive("pow_log"), {}))
        inits.append(lv)
    params = dict(e.params)
    params["body_jaxpr"] = _closed_like(e.params["body_jaxpr"], new_body)
    params["cond_jaxpr"] = _closed_like(e.params["cond_jaxpr"], new_cond)
    outs = e.outvars + [Var(_f64(tuple(c.aval.shape))) for _, c, _, _ in found]
    return pre, JaxprEqn(e.invars + inits, outs, e.primitive, params)


def carry_logs(jaxpr: Jaxpr) -> Jaxpr:
    """FAST: a while-loop carry `c` that the body reads only through
    `log2(c)` and updates only as `c' = select_n(p, c, v)` (either case
    order), and that neither the condition nor the code after the loop
    reads, is replaced by its log2: the body uses the carried log, the
    update selects `log2(v)` (for `v = 1 / y`, `-log2(y)`, reusing a log2 of
    y the body already takes), and the initial value's log is taken once
    before the loop. After `power_laws_to_exp2`, the PI controller's
    `prev_inv_err` (`tests/test_08_adaptive.py:76-122` of the reference) is
    such a carry: the attempt then computes neither the reciprocal of the
    error nor the log of `prev`. Results differ from the unrewritten loop
    by the rounding of log2(1 / y) against -log2(y), within FAST's contract."""
    used_after: set = set()
    for e in jaxpr.eqns:
        used_after.update(v for v in e.invars if isinstance(v, Var))
    used_after.update(v for v in jaxpr.outvars if isinstance(v, Var))
    new_eqns: list[JaxprEqn] = []
    for e in jaxpr.eqns:
        params = {k: _rewrite_sub(v, carry_logs) for k, v in e.params.items()}
        e = JaxprEqn(e.invars, e.outvars, e.primitive, params)
        if e.primitive.name == "while":
            pre, e = _carry_logs_while(e, used_after)
            new_eqns += pre
        new_eqns.append(e)
    return Jaxpr(jaxpr.constvars, jaxpr.invars, jaxpr.outvars, new_eqns)


def _carry_logs_while(e: JaxprEqn, used_after: set) -> tuple[list[JaxprEqn], JaxprEqn]:
    cn, bn = int(e.params["cond_nconsts"]), int(e.params["body_nconsts"])
    body = getattr(e.params["body_jaxpr"], "jaxpr", e.params["body_jaxpr"])
    cond = getattr(e.params["cond_jaxpr"], "jaxpr", e.params["cond_jaxpr"])
    carries = body.invars[bn:]
    producer = {ov: x for x in body.eqns for ov in x.outvars}
    readers: dict[Any, list] = {}
    for x in body.eqns:
        for v in x.invars:
            if isinstance(v, Var):
                readers.setdefault(v, []).append(x)
    out_pos: dict[Any, list] = {}
    for k, v in enumerate(body.outvars):
        out_pos.setdefault(v, []).append(k)
    cond_used = {v for x in cond.eqns for v in x.invars} | set(cond.outvars)

    def f32(v: Any) -> bool:
        return isinstance(v, Var) and np.dtype(v.aval.dtype) == np.float32

    plans = []
    for k, c in enumerate(carries):
        if not f32(c) or cond.invars[cn + k] in cond_used or e.outvars[k] in used_after:
            continue
        sel = producer.get(body.outvars[k])
        if sel is None or sel.primitive.name != "select_n" or len(sel.invars) != 3:
            continue
        cases = sel.invars[1:]
        if sum(u is c for u in cases) != 1 or out_pos.get(body.outvars[k]) != [k]:
            continue
        (v,) = [u for u in cases if u is not c]
        if c in out_pos:  # returned as some carry's next value: read as a value
            continue
        rs = readers.get(c, [])
        logs = [x for x in rs if x.primitive.name == "log2"]
        if not logs or len(logs) + 1 != len(rs) or sel not in rs or readers.get(body.outvars[k], []):
            continue
        # log2(v): an existing log2 of v, or -log2(y) for v = 1 / y with log2(y) taken
        lv = next((x.outvars[0] for x in readers.get(v, []) if x.primitive.name == "log2"), None)
        neg_of = None
        if lv is None:
            d = producer.get(v)
            if (d is not None and d.primitive.name == "div" and _f32_literal(d.invars[0]) == 1.0
                    and isinstance(d.invars[1], Var)):
                neg_of = next((x.outvars[0] for x in readers.get(d.invars[1], []) if x.primitive.name == "log2"),
                              None)
            if neg_of is None:
                continue
        plans.append((k, c, v, sel, logs, lv, neg_of))
    if not plans:
        return [], e
    subst: dict[Any, Any] = {}
    new_in = list(body.invars)
    extra: list[JaxprEqn] = []
    new_out = list(body.outvars)
    drop = set()
    for k, c, v, sel, logs, lv, neg_of in plans:
        lc = Var(ShapedArray(c.aval.shape, np.float32))
        new_in[bn + k] = lc
        for x in logs:
            subst[x.outvars[0]] = lc
            drop.add(id(x))
        if lv is None:
            lv = Var(ShapedArray(c.aval.shape, np.float32))
            extra.append(JaxprEqn([neg_of], [lv], primitive("neg"), {}))
        nxt = Var(ShapedArray(c.aval.shape, np.float32))
        cases = [lc if u is c else lv for u in sel.invars[1:]]
        extra.append(JaxprEqn([sel.invars[0], *cases], [nxt], primitive("select_n"), {}))
        new_out[k] = nxt
        drop.add(id(sel))

    def sub(v: Any) -> Any:
        return subst.get(v, v) if isinstance(v, Var) else v

    eqns = [JaxprEqn([sub(v) for v in x.invars], x.outvars, x.primitive, x.params)
            for x in body.eqns if id(x) not in drop] + extra
    new_body = Jaxpr(body.constvars, new_in, [sub(v) for v in new_out], eqns)
    new_cond_in = list(cond.invars)
    for k, *_ in plans:
        new_cond_in[cn + k] = Var(ShapedArray(cond.invars[cn + k].aval.shape, np.float32))
    new_cond = Jaxpr(cond.constvars, new_cond_in, cond.outvars, cond.eqns)
    pre, inits = [], list(e.invars)
    for k, c, *_ in plans:
        lv0 = Var(ShapedArray(c.aval.shape, np.float32))
        pre.append(JaxprEqn([e.invars[cn + bn + k]], [lv0], primitive("log2"), {}))
        inits[cn + bn + k] = lv0
    params = dict(e.params)
    params["body_jaxpr"] = _closed_like(e.params["body_jaxpr"], new_body)
    params["cond_jaxpr"] = _closed_like(e.params["cond_jaxpr"], new_cond)
    outs = list(e.outvars)
    for k, *_ in plans:
        outs[k] = Var(ShapedArray(outs[k].aval.shape, np.float32))  # no longer the carry's value
    return pre, JaxprEqn(inits, outs, e.primitive, params)


def funnel_shifts(jaxpr: Jaxpr) -> Jaxpr:
    """Exact, every math mode: `or(shift_right_logical(x, n), C)` for a
    32-bit integer literal C whose low 32 - n bits are zero is
    `alignbit(C >> (32 - n), x, n)`, the low word of the 64-bit pair
    (C >> (32 - n), x) shifted right by n: one `v_alignbit_b32` where the
    compiler emits a shift and an or. `jax.random.uniform`'s float
    construction `bits >> 9 | 0x3F800000` (the reference's staged ops,
    `tests/test_10_random_bits.py:42-54`) is this form."""
    producer = {ov: e for e in jaxpr.eqns for ov in e.outvars}

    def const(v: Any) -> int | None:
        """The integer value of a scalar literal, or of a broadcast of one."""
        for _ in range(4):
            if isinstance(v, Literal):
                return int(np.asarray(v.val).astype(np.int64)) if np.ndim(v.val) == 0 else None
            e = producer.get(v) if isinstance(v, Var) else None
            if e is None or e.primitive.name != "broadcast_in_dim":
                return None
            v = e.invars[0]
        return None

    new_eqns: list[JaxprEqn] = []
    for e in jaxpr.eqns:
        params = {k: _rewrite_sub(v, funnel_shifts) for k, v in e.params.items()}
        e = JaxprEqn(e.invars, e.outvars, e.primitive, params)
        if e.primitive.name == "or" and len(e.invars) == 2:
            out = e.outvars[0]
            dt = np.dtype(out.aval.dtype)
            for sv, cv in (e.invars, e.invars[::-1]):
                sh = producer.get(sv) if isinstance(sv, Var) else None
                cval = const(cv)
                if (dt not in (np.uint32, np.int32) or cval is None or sh is None
                        or sh.primitive.name != "shift_right_logical" or const(sh.invars[1]) is None):
                    continue
                n = const(sh.invars[1])
                c = cval & 0xFFFFFFFF
                x = sh.invars[0]
                if not (0 < n < 32) or c & ((1 << (32 - n)) - 1) or np.dtype(x.aval.dtype) != dt \
                        or tuple(x.aval.shape) != tuple(out.aval.shape):
                    continue
                hi = Literal(np.uint32(c >> (32 - n)), ShapedArray((), np.uint32))
                amt = Literal(np.uint32(n), ShapedArray((), np.uint32))
                if dt == np.uint32:
                    new_eqns.append(JaxprEqn([hi, x, amt], [out], primitive("alignbit"), {}))
                else:
                    xu, ru = Var(ShapedArray(x.aval.shape, np.uint32)), Var(ShapedArray(x.aval.shape, np.uint32))
                    new_eqns.append(JaxprEqn([x], [xu], primitive("bitcast_convert_type"), {"new_dtype": np.dtype(np.uint32)}))
                    new_eqns.append(JaxprEqn([hi, xu, amt], [ru], primitive("alignbit"), {}))
                    new_eqns.append(JaxprEqn([ru], [out], primitive("bitcast_convert_type"), {"new_dtype": dt}))
                break
            else:
                new_eqns.append(e)
            continue
        new_eqns.append(e)
    return Jaxpr(jaxpr.constvars, jaxpr.invars, jaxpr.outvars, new_eqns)


def reuse_affine_shifts(jaxpr: Jaxpr) -> Jaxpr:
    """FAST: a Runge-Kutta stage evaluates the right-hand side at a shifted
    state, `y + h k`; where the same expression was already evaluated at
    the unshifted state, the shift can be added to that value instead:

        a - b (y + h k)   ->   (a - b y) - (b h) k      (a - b y computed before)
        c (x + h k) - d   ->   (c x - d) + (c h) k      (c x - d computed before)

    for a literal h. The instruction count stays (the shifted state is still
    needed elsewhere, and `b h` is loop-invariant when b is), but the new
    value no longer waits for the shifted state: one dependent operation
    fewer per stage on a latency-bound integrator (the LV right-hand side
    `x (a - b y)`, `y (c x - d)` of the reference's
    `examples/01_ode_ensembles.py:72-91`). Rounding differs from the traced
    order, within FAST's reassociation contract."""
    producer = {ov: e for e in jaxpr.eqns for ov in e.outvars}
    f32 = np.dtype(np.float32)

    def is_f32(v: Any) -> bool:
        return np.dtype(getattr(v.aval, "dtype", np.float64)) == f32

    def same(a: Any, b: Any) -> bool:
        return _same(a, b)

    def prod_of(v: Any) -> tuple | None:
        e = producer.get(v) if isinstance(v, Var) else None
        return tuple(e.invars) if e is not None and e.primitive.name == "mul" else None

    def shift_of(v: Any) -> tuple | None:
        """(y, h, k) for v = y + h k (either order, h a literal)."""
        e = producer.get(v) if isinstance(v, Var) else None
        if e is None or e.primitive.name != "add":
            return None
        for y, m in (e.invars, e.invars[::-1]):
            hk = prod_of(m)
            if hk is None:
                continue
            for h, k in (hk, hk[::-1]):
                if _f32_literal(h) is not None and isinstance(k, Var):
                    return y, h, k
        return None

    def _aval_of(v: Any, out: Any) -> Any:
        return v.aval if isinstance(v, Var) else ShapedArray((), np.float32)

    def fits(v: Any, k: Any, out: Any) -> bool:
        """v * h * k has out's shape with no broadcast of a variable."""
        return (k.aval.shape == out.aval.shape
                and (_f32_literal(v) is not None or (isinstance(v, Var) and v.aval.shape == out.aval.shape)))

    seen_sub: list[JaxprEqn] = []   # earlier subs, in order
    bypassed: set = set()           # products the rewritten subs no longer read
    new_eqns: list[JaxprEqn] = []
    for e in jaxpr.eqns:
        params = {k: _rewrite_sub(v, reuse_affine_shifts) for k, v in e.params.items()}
        e = JaxprEqn(e.invars, e.outvars, e.primitive, params)
        out = e.outvars[0] if len(e.outvars) == 1 else None
        done = False
        if e.primitive.name == "sub" and out is not None and is_f32(out):
            lhs, rhs = e.invars
            # a - b (y + h k), with a - b y earlier
            bv = prod_of(rhs)
            for b, v in ((bv, bv[::-1]) if bv else ()):
                sh = shift_of(v)
                if done or sh is None:
                    continue
                y, h, k = sh
                if not fits(b, k, out):
                    continue
                for s0 in seen_sub:
                    p0 = prod_of(s0.invars[1])
                    if (same(s0.invars[0], lhs) and p0 is not None
                            and ((same(p0[0], b) and same(p0[1], y)) or (same(p0[0], y) and same(p0[1], b)))):
                        bh, t = Var(_aval_of(b, out)), Var(out.aval)
                        new_eqns.append(JaxprEqn([b, h], [bh], primitive("mul"), {}))
                        new_eqns.append(JaxprEqn([bh, k], [t], primitive("mul"), {}))
                        new_eqns.append(JaxprEqn([s0.outvars[0], t], [out], primitive("sub"), {}))
                        bypassed.add(rhs)
                        done = True
                        break
            # c (x + h k) - d, with c x - d earlier
            cv = prod_of(lhs)
            for c, v in ((cv, cv[::-1]) if (cv and not done) else ()):
                sh = shift_of(v)
                if done or sh is None:
                    continue
                x, h, k = sh
                if not fits(c, k, out):
                    continue
                for s0 in seen_sub:
                    q0 = prod_of(s0.invars[0])
                    if (same(s0.invars[1], rhs) and q0 is not None
                            and ((same(q0[0], c) and same(q0[1], x)) or (same(q0[0], x) and same(q0[1], c)))):
                        ch, t = Var(_aval_of(c, out)), Var(out.aval)
                        new_eqns.append(JaxprEqn([c, h], [ch], primitive("mul"), {}))
                        new_eqns.append(JaxprEqn([ch, k], [t], primitive("mul"), {}))
                        new_eqns.append(JaxprEqn([s0.outvars[0], t], [out], primitive("add"), {}))
                        bypassed.add(lhs)
                        done = True
                        break
        if done:
            continue
        if e.primitive.name == "sub" and out is not None:
            seen_sub.append(e)
        new_eqns.append(e)
    used = {v for e in new_eqns for v in e.invars if isinstance(v, Var)} | set(jaxpr.outvars)
    new_eqns = [e for e in new_eqns if not (e.outvars[0] in bypassed and e.outvars[0] not in used)]
    return Jaxpr(jaxpr.constvars, jaxpr.invars, jaxpr.outvars, new_eqns)



def fold_counters(jaxpr: Jaxpr) -> Jaxpr:
    """Exact, every math mode: in a while loop with integer carries

        a' = a + select_n(p, a0, a1)     b' = b + select_n(p, b0, b1)     n' = n + s

    for literals with a0 + b0 == a1 + b1 == s (an adaptive solver's
    accepted and rejected counts beside its attempt count,
    `examples/02_adaptive_lockstep.py:85-140` and
    `tests/test_08_adaptive.py:33-142` of the reference), a + b - n never
    changes, so b need not be carried: it leaves the loop, and after it

        b_final = b_init + (n_final - n_init) - (a_final - a_init)

    in the same wrapping integer arithmetic. The loop loses b's add and
    select; the condition and the rest of the body must not read b."""
    new_eqns: list[JaxprEqn] = []
    for e in jaxpr.eqns:
        params = {k: _rewrite_sub(v, fold_counters) for k, v in e.params.items()}
        e = JaxprEqn(e.invars, e.outvars, e.primitive, params)
        if e.primitive.name == "while":
            e, post = _fold_counters_while(e)
            new_eqns.append(e)
            new_eqns.extend(post)
            continue
        new_eqns.append(e)
    return Jaxpr(jaxpr.constvars, jaxpr.invars, jaxpr.outvars, new_eqns)


def _fold_counters_while(e: JaxprEqn) -> tuple[JaxprEqn, list[JaxprEqn]]:
    cn, bn = int(e.params["cond_nconsts"]), int(e.params["body_nconsts"])
    body = getattr(e.params["body_jaxpr"], "jaxpr", e.params["body_jaxpr"])
    cond = getattr(e.params["cond_jaxpr"], "jaxpr", e.params["cond_jaxpr"])
    carries = body.invars[bn:]
    producer = {ov: x for x in body.eqns for ov in x.outvars}
    readers: dict[Any, list] = {}
    for x in body.eqns:
        for v in x.invars:
            if isinstance(v, Var):
                readers.setdefault(v, []).append(x)
    cond_used = {v for x in cond.eqns for v in x.invars} | set(cond.outvars)

    def lit(v: Any) -> int | None:
        for _ in range(4):
            if isinstance(v, Literal):
                return int(np.asarray(v.val).astype(np.int64)) if np.ndim(v.val) == 0 else None
            x = producer.get(v) if isinstance(v, Var) else None
            if x is None or x.primitive.name != "broadcast_in_dim":
                return None
            v = x.invars[0]
        return None

    def increment(k: int) -> Any:
        """The added operand of carry k's update `c + X`, or None."""
        c, out = carries[k], body.outvars[k]
        x = producer.get(out) if isinstance(out, Var) else None
        if x is None or x.primitive.name != "add" or len(x.invars) != 2:
            return None
        if x.invars[0] is c:
            return x.invars[1]
        return x.invars[0] if x.invars[1] is c else None

    def is_int(v: Any) -> bool:
        return np.issubdtype(np.dtype(v.aval.dtype), np.integer)

    steps, selects = {}, {}
    for k, c in enumerate(carries):
        if not is_int(c) or body.outvars.count(body.outvars[k]) != 1:
            continue
        inc = increment(k)
        if inc is None:
            continue
        s = lit(inc)
        if s is not None:
            steps[k] = s
            continue
        x = producer.get(inc) if isinstance(inc, Var) else None
        if x is not None and x.primitive.name == "select_n" and len(x.invars) == 3:
            cases = [lit(v) for v in x.invars[1:]]
            if None not in cases:
                selects[k] = (x.invars[0], cases[0], cases[1])
    plan = None
    # Drop, of a pair, the count that moves when p is false (a rejection
    # count): the one kept then steps under `p`, the mask the loop's other
    # selects already use, not under `!p`.
    order = sorted(selects, key=lambda j: not (selects[j][1] != 0 and selects[j][2] == 0))
    for j in order:
        pj, b0, b1 = selects[j]
        cj = carries[j]
        if (cond.invars[cn + j] in cond_used or readers.get(cj, []) != [producer[body.outvars[j]]]
                or cj in body.outvars):
            continue
        for i, (pi, a0, a1) in selects.items():
            if i == j or pi is not pj or a0 + b0 != a1 + b1:
                continue
            n = next((n for n, s in steps.items() if s == a0 + b0 and n not in (i, j)
                      and carries[n].aval.dtype == cj.aval.dtype == carries[i].aval.dtype
                      and carries[n].aval.shape == cj.aval.shape == carries[i].aval.shape), None)
            if n is not None:
                plan = (i, j, n)
                break
        if plan:
            break
    if plan is None:
        return e, []
    i, j, n = plan
    # b leaves the loop: its update (and the select feeding only it) goes,
    # and so does its slot in the body's, the condition's and the loop's
    # operands and results; after the loop its initial value is still the
    # loop operand's, so
    #     b_final = b_init + (n_final - n_init) - (a_final - a_init).
    upd = producer[body.outvars[j]]
    dead = {id(upd)}
    sel = producer.get(upd.invars[0] if upd.invars[1] is carries[j] else upd.invars[1])
    if sel is not None and len(readers.get(sel.outvars[0], [])) == 1 and sel.outvars[0] not in body.outvars:
        dead.add(id(sel))
    new_body = Jaxpr(body.constvars, body.invars[:bn + j] + body.invars[bn + j + 1:],
                     body.outvars[:j] + body.outvars[j + 1:], [x for x in body.eqns if id(x) not in dead])
    new_cond = Jaxpr(cond.constvars, cond.invars[:cn + j] + cond.invars[cn + j + 1:], cond.outvars, cond.eqns)
    params = dict(e.params)
    params["body_jaxpr"] = _closed_like(e.params["body_jaxpr"], new_body)
    params["cond_jaxpr"] = _closed_like(e.params["cond_jaxpr"], new_cond)
    init = e.invars[cn + bn:]
    b_final = e.outvars[j]
    aval = b_final.aval
    dn, da, d = Var(aval), Var(aval), Var(aval)
    post = [JaxprEqn([e.outvars[n], init[n]], [dn], primitive("sub"), {}),
            JaxprEqn([e.outvars[i], init[i]], [da], primitive("sub"), {}),
            JaxprEqn([dn, da], [d], primitive("sub"), {}),
            JaxprEqn([init[j], d], [b_final], primitive("add"), {})]
    k = cn + bn + j
    outs = e.outvars[:j] + e.outvars[j + 1:]
    return JaxprEqn(e.invars[:k] + e.invars[k + 1:], outs, e.primitive, params), post


def _product_operands(e: JaxprEqn) -> tuple[Any, Any] | None:
    """(a, b) when `e` computes a * b: a mul, or integer_pow with y = 2."""
    if e.primitive.name == "mul" and len(e.invars) == 2:
        return e.invars[0], e.invars[1]
    if e.primitive.name == "integer_pow" and int(e.params.get("y", 0)) == 2:
        return e.invars[0], e.invars[0]
    return None


def contract_products(jaxpr: Jaxpr) -> Jaxpr:
    """REPRODUCIBLE: fuse a float32 product into the add or subtract that is
    its only use,

        a*b + c  ->  fma(a, b, c)        c + a*b  ->  fma(a, b, c)
        a*b - c  ->  fma(a, b, -c)       c - a*b  ->  fma(-a, b, c)

    with `x**2` read as x*x. When both operands of the add are such
    products, the one computed later in the program is fused (it is the one
    the sum waits for), so a chain `(p1 + p2) + p3` becomes
    fma(p3, fma(p2, p1)). The sites are a function of the program alone,
    and each fma is correctly rounded, so a host restatement that writes
    C `fmaf` at the same sites reproduces the device bit for bit. Negation
    is exact, so the signs are carried as parameters `neg_ab`, `neg_c`."""
    producer = {ov: e for e in jaxpr.eqns for ov in e.outvars}
    order = {id(e): k for k, e in enumerate(jaxpr.eqns)}
    uses = _use_counts(jaxpr)
    f32 = np.dtype(np.float32)

    def is_f32(v: Any) -> bool:
        return np.dtype(getattr(v.aval, "dtype", np.float64)) == f32

    fused: set = set()
    new_eqns: list[JaxprEqn] = []
    for e in jaxpr.eqns:
        params = {k: _rewrite_sub(v, contract_products) for k, v in e.params.items()}
        e = JaxprEqn(e.invars, e.outvars, e.primitive, params)
        name = e.primitive.name
        out = e.outvars[0] if len(e.outvars) == 1 else None
        if name in ("add", "sub") and out is not None and is_f32(out) and len(e.invars) == 2:
            best = None
            for side, v in enumerate(e.invars):
                pe = producer.get(v) if isinstance(v, Var) else None
                if pe is None or uses.get(v, 0) != 1 or v in fused:
                    continue
                ab = _product_operands(pe)
                if ab is None or not is_f32(v) or tuple(v.aval.shape) != tuple(out.aval.shape):
                    continue
                if best is None or order[id(pe)] > best[0]:
                    best = (order[id(pe)], side, v, ab)
            if best is not None:
                _, side, v, (a, b) = best
                other = e.invars[1 - side]
                neg_ab = name == "sub" and side == 1
                neg_c = name == "sub" and side == 0
                fused.add(v)
                new_eqns.append(JaxprEqn([a, b, other], [out], primitive("fma"),
                                         {"neg_ab": neg_ab, "neg_c": neg_c}))
                continue
        new_eqns.append(e)
    new_eqns = [e for e in new_eqns if not (len(e.outvars) == 1 and e.outvars[0] in fused)]
    return Jaxpr(jaxpr.constvars, jaxpr.invars, jaxpr.outvars, new_eqns)


# Primitives with no effect beyond their results (stores, lane collectives,
# loops, calls and user-registered rules are not listed, so they stay).
_PURE = frozenset((
    "add sub mul div rem min max pow neg abs sign exp exp2 log log2 log1p expm1 sin cos tan tanh sqrt "
    "rsqrt floor ceil round logistic atan2 lt le gt ge eq ne and or xor not shift_right_logical "
    "shift_right_arithmetic shift_left clamp select_n integer_pow convert_element_type "
    "bitcast_convert_type fma pow_log pow_with_log get broadcast_in_dim reshape squeeze expand_dims "
    "transpose program_id num_programs random_wrap random_unwrap random_fold_in random_bits "
    "threefry2x32 iota lane_index"
).split())


def drop_dead_code(jaxpr: Jaxpr) -> Jaxpr:
    """Every mode: remove the equations of side-effect-free primitives whose
    results nothing reads (at their own level: a loop body's results are
    its carries), in nested jaxprs too. Rewrites leave such equations
    behind (a reciprocal the carried log replaced, say), and the emitted
    C++ cannot always lose them itself: a helper holding a volatile asm
    (the wavefront-uniform slow-path tests) is never removed by the
    compiler. Removing an unread pure value changes no result."""
    eqns = [JaxprEqn(e.invars, e.outvars, e.primitive,
                     {k: _rewrite_sub(v, drop_dead_code) for k, v in e.params.items()}) for e in jaxpr.eqns]
    live = {v for v in jaxpr.outvars if isinstance(v, Var)}
    kept: list[JaxprEqn] = []
    for e in reversed(eqns):
        if e.primitive.name in _PURE and e.outvars and not any(o in live for o in e.outvars):
            continue
        kept.append(e)
        live.update(a for a in e.invars if isinstance(a, Var))
    return Jaxpr(jaxpr.constvars, jaxpr.invars, jaxpr.outvars, kept[::-1])
