"""`jax.lax`-shaped control flow and primitives for the frontend.

Staging layout follows JAX's, which is what the reference lowering rules
consume:
- `fori_loop` with static bounds stages `scan` (consts first, then the
  loop index carry, then user carries; `src/palladium/emit/rules.py:679-714`);
- `while_loop` stages `while` with `cond_nconsts`/`body_nconsts`
  (`rules.py:812-844`);
- `cond`/`switch` stage `cond` over a clamped int32 index
  (`rules.py:847-878`).
"""

from __future__ import annotations

from typing import Any, Callable, Sequence

import numpy as np

from palladium_amd.dtypes import name as _dtype_name
from palladium_amd.errors import TraceError
from palladium_amd.frontend import jnp
from palladium_amd.frontend.core import (
    BOOL,
    I32,
    Builder,
    Tracer,
    building,
    closed,
    current_builder,
    default_dtype,
    literal,
)
from palladium_amd.ir import ClosedJaxpr, Jaxpr, ShapedArray

# Re-exports with lax names.
add = jnp.add
sub = jnp.subtract
mul = jnp.multiply
max = jnp.maximum  # noqa: A001
min = jnp.minimum  # noqa: A001
neg = jnp.negative
abs = jnp.abs  # noqa: A001
exp = jnp.exp
log = jnp.log
sin = jnp.sin
cos = jnp.cos
sqrt = jnp.sqrt
rsqrt = jnp.rsqrt
tanh = jnp.tanh
pow = jnp.power  # noqa: A001
integer_pow = jnp.integer_pow
select_n = jnp.select_n
clamp = jnp.clamp
convert_element_type = jnp.convert_element_type
bitcast_convert_type = jnp.bitcast_convert_type
broadcast_in_dim = jnp.broadcast_in_dim
reshape = jnp.reshape
bitwise_and = jnp.bitwise_and
bitwise_or = jnp.bitwise_or
bitwise_xor = jnp.bitwise_xor
bitwise_not = jnp.invert
shift_left = jnp.left_shift
lt = jnp.less
le = jnp.less_equal
gt = jnp.greater
ge = jnp.greater_equal
eq = jnp.equal
ne = jnp.not_equal


broadcasted_iota = jnp.broadcasted_iota
dot_general = jnp.dot_general
transpose = jnp.transpose


def dot(lhs: Any, rhs: Any, precision: Any = None, preferred_element_type: Any = None) -> Tracer:
    return jnp.dot(lhs, rhs, precision=precision, preferred_element_type=preferred_element_type)


def div(a: Any, b: Any) -> Tracer:
    """lax.div: dtype-preserving; integers truncate toward zero (x / 0 and
    INT_MIN / -1 are defined as XLA defines them), floats divide."""
    return jnp._nary("div", a, b)


def rem(a: Any, b: Any) -> Tracer:
    """lax.rem: remainder with the dividend's sign (C fmod for floats)."""
    return jnp._nary("rem", a, b)


def round(x: Any, rounding_method: int = 0) -> Tracer:  # noqa: A001
    """lax.round: 0 = away from zero (default), 1 = to nearest even."""
    return jnp._unary("round", x, True, rounding_method=int(rounding_method))


def iota(dtype: Any, size: int) -> Tracer:
    return jnp.broadcasted_iota(dtype, (int(size),), 0)


def shift_right_logical(a: Any, b: Any) -> Tracer:
    return jnp._nary("shift_right_logical", a, b)


def shift_right_arithmetic(a: Any, b: Any) -> Tracer:
    return jnp._nary("shift_right_arithmetic", a, b)


# ---------------------------------------------------------------------------
# pytrees (tuples / lists / dicts / leaves)


def _flatten(tree: Any) -> tuple[list[Any], Any]:
    if isinstance(tree, (tuple, list)):
        leaves: list[Any] = []
        subs = []
        for t in tree:
            lv, st = _flatten(t)
            leaves += lv
            subs.append((len(lv), st))
        return leaves, (type(tree), subs)
    if isinstance(tree, dict):
        keys = sorted(tree)
        lv, st = _flatten([tree[k] for k in keys])
        return lv, (dict, keys, st)
    return [tree], None


def _unflatten(struct: Any, leaves: list[Any]) -> Any:
    if struct is None:
        return leaves[0]
    if struct[0] is dict:
        _, keys, st = struct
        vals = _unflatten(st, leaves)
        return dict(zip(keys, vals))
    typ, subs = struct
    out = []
    pos = 0
    for n, st in subs:
        out.append(_unflatten(st, leaves[pos : pos + n]))
        pos += n
    return typ(out) if typ is not tuple else tuple(out)


def _to_tracer(x: Any) -> Tracer:
    if isinstance(x, Tracer):
        return x
    if isinstance(x, np.ndarray) and x.ndim > 0:
        raise TraceError("loop carries must be traced values or Python scalars")
    return jnp.full((), x, dtype=None if not isinstance(x, np.generic) else x.dtype)


def _avals(leaves: list[Tracer]) -> list[ShapedArray]:
    return [t.aval for t in leaves]


def _trace_fn(fn: Callable, in_avals: list[ShapedArray], struct: Any, prefix: list[Any] = ()) -> tuple[Builder, list[Any]]:
    parent = current_builder()
    b = Builder(parent)
    with building(b):
        args = [b.arg(a) for a in in_avals]
        tree = _unflatten(struct, args)
        out = fn(*prefix, tree) if prefix else fn(tree)
    return b, out


def _match_carry(outs: list[Any], avals: list[ShapedArray], what: str) -> tuple[list[ShapedArray], bool]:
    """New carry avals if only weak types differ; raises on real mismatch."""
    new = []
    changed = False
    for o, a in zip(outs, avals, strict=True):
        oa = o.aval if isinstance(o, Tracer) else ShapedArray((), default_dtype(o), True)
        if oa.shape != a.shape:
            raise TraceError(f"{what}: carry shape changed from {a.shape} to {oa.shape}")
        if oa.dtype != a.dtype:
            if a.weak_type:
                new.append(ShapedArray(a.shape, oa.dtype, oa.weak_type))
                changed = True
                continue
            if oa.weak_type:
                new.append(a)
                continue
            raise TraceError(f"{what}: carry dtype changed from {_dtype_name(a.dtype)} to {_dtype_name(oa.dtype)}")
        if a.weak_type and not oa.weak_type:
            new.append(ShapedArray(a.shape, a.dtype, False))
            changed = True
            continue
        new.append(a)
    return new, changed


def _coerce_out(b: Builder, outs: list[Any], avals: list[ShapedArray]) -> list[Any]:
    fixed = []
    with building(b):
        for o, a in zip(outs, avals, strict=True):
            if not isinstance(o, Tracer) or o.dtype != a.dtype:
                o = jnp.convert_element_type(o, a.dtype, weak_type=a.weak_type) if isinstance(o, Tracer) else jnp.full(a.shape, o, a.dtype)
            fixed.append(o)
    return fixed


def _coerce_init(leaves: list[Tracer], avals: list[ShapedArray]) -> list[Tracer]:
    return [
        t if t.dtype == a.dtype and t.weak_type == a.weak_type else jnp.convert_element_type(t, a.dtype, weak_type=a.weak_type)
        for t, a in zip(leaves, avals, strict=True)
    ]


# ---------------------------------------------------------------------------
# loops


def fori_loop(lower: Any, upper: Any, body_fun: Callable, init_val: Any, *, unroll: int | bool | None = None) -> Any:
    """`lax.fori_loop`. Static bounds stage `scan` over `(i, *carry)`;
    traced bounds stage `while` over `(i, upper, *carry)`."""
    leaves, struct = _flatten(init_val)
    leaves = [_to_tracer(x) for x in leaves]
    if isinstance(lower, Tracer) or isinstance(upper, Tracer):
        lo = lower if isinstance(lower, Tracer) else jnp.full((), int(lower), I32)
        hi = upper if isinstance(upper, Tracer) else jnp.full((), int(upper), I32)

        def body_flat(c):
            i, u, *rest = c
            new = body_fun(i, _unflatten(struct, rest))
            nl, _ = _flatten(new)
            return (i + 1, u, *nl)

        out = while_loop(lambda c: c[0] < c[1], body_flat, (lo, hi, *leaves))
        return _unflatten(struct, list(out[2:]))

    lower, upper = int(lower), int(upper)
    length = upper - lower if upper > lower else 0
    idx_aval = ShapedArray((), I32, False)
    avals = _avals(leaves)
    for _ in range(3):
        parent = current_builder()
        b = Builder(parent)
        with building(b):
            i = b.arg(idx_aval)
            args = [b.arg(a) for a in avals]
            new = body_fun(i, _unflatten(struct, args))
            new_leaves, new_struct = _flatten(new)
            if len(new_leaves) != len(args):
                raise TraceError("fori_loop: body must return the carry structure it was given")
            i_next = i + 1
        new_avals, changed = _match_carry(new_leaves, avals, "fori_loop")
        if not changed:
            break
        avals = new_avals
    else:
        raise TraceError("fori_loop: carry types did not converge")
    new_leaves = _coerce_out(b, new_leaves, avals)
    body = closed(b, [i_next, *new_leaves])
    consts = b.captured_outer()
    init = _coerce_init(leaves, avals)
    out_avals = [idx_aval, *avals]
    start = literal(lower, I32, weak=False)
    params = dict(
        reverse=False,
        length=length,
        jaxpr=body,
        num_consts=len(consts),
        num_carry=len(out_avals),
        linear=tuple([False] * (len(consts) + len(out_avals))),
        unroll=int(unroll) if unroll not in (None, False, True) else (1 if not unroll else length),
        _split_transpose=False,
    )
    outs = current_builder().add("scan", [*consts, start, *init], out_avals, **params)
    return _unflatten(struct, outs[1:])


def scan(f: Callable, init: Any, xs: Any = None, length: int | None = None, reverse: bool = False, unroll: int = 1) -> tuple[Any, Any]:
    """`lax.scan`, staged as JAX stages it: consts, carries, then scanned
    xs as invars; carries then stacked ys as outvars. The emitter lowers
    the pure-carry form (`xs=None`, no ys) and rejects the others with the
    reference's messages (`src/palladium/emit/rules.py:717-738`)."""
    if reverse:
        raise TraceError("no reverse-mode scan support, use lax.fori_loop")
    x_leaves, x_struct = _flatten(xs) if xs is not None else ([], None)
    x_leaves = [_to_tracer(x) for x in x_leaves]
    if x_leaves:
        n = x_leaves[0].shape[0] if x_leaves[0].shape else None
        if n is None or any(not x.shape or x.shape[0] != n for x in x_leaves):
            raise TraceError("lax.scan xs must share a leading dim")
        if length is not None and int(length) != n:
            raise TraceError(f"lax.scan length={length} disagrees with xs leading dim {n}")
        length = n
    if length is None:
        raise TraceError("lax.scan without xs needs length=")
    leaves, struct = _flatten(init)
    leaves = [_to_tracer(x) for x in leaves]
    avals = _avals(leaves)
    x_avals = [ShapedArray(tuple(x.shape[1:]), x.dtype, x.weak_type) for x in x_leaves]
    for _ in range(3):
        b = Builder(current_builder())
        with building(b):
            args = [b.arg(a) for a in avals]
            xargs = [b.arg(a) for a in x_avals]
            res = f(_unflatten(struct, args), _unflatten(x_struct, xargs) if x_leaves else None)
            if not (isinstance(res, tuple) and len(res) == 2):
                raise TraceError("scan body must return (carry, y)")
            carry, y = res
            new_leaves, _ = _flatten(carry)
            y_leaves, y_struct = _flatten(y) if y is not None else ([], None)
            y_leaves = [_to_tracer(v) for v in y_leaves]
        avals2, changed = _match_carry(new_leaves, avals, "scan")
        if not changed:
            break
        avals = avals2
    new_leaves = _coerce_out(b, new_leaves, avals)
    body = closed(b, new_leaves + y_leaves)
    # closed() puts captured consts first; the scanned xs follow the carries
    consts = b.captured_outer()
    params = dict(
        reverse=False, length=int(length), jaxpr=body, num_consts=len(consts), num_carry=len(avals),
        linear=tuple([False] * (len(consts) + len(avals) + len(x_leaves))), unroll=int(unroll),
        _split_transpose=False,
    )
    y_avals = [ShapedArray((int(length),) + tuple(v.shape), v.dtype, False) for v in y_leaves]
    outs = current_builder().add("scan", [*consts, *_coerce_init(leaves, avals), *x_leaves], avals + y_avals, **params)
    ys = _unflatten(y_struct, outs[len(avals):]) if y_leaves else None
    return _unflatten(struct, outs[: len(avals)]), ys


def while_loop(cond_fun: Callable, body_fun: Callable, init_val: Any) -> Any:
    """`lax.while_loop`: data-dependent trip count per program instance."""
    leaves, struct = _flatten(init_val)
    leaves = [_to_tracer(x) for x in leaves]
    avals = _avals(leaves)
    for _ in range(3):
        bb = Builder(current_builder())
        with building(bb):
            args = [bb.arg(a) for a in avals]
            new = body_fun(_unflatten(struct, args))
            new_leaves, _ = _flatten(new)
            if len(new_leaves) != len(args):
                raise TraceError("while_loop: body must return the carry structure it was given")
        avals2, changed = _match_carry(new_leaves, avals, "while_loop")
        if not changed:
            break
        avals = avals2
    new_leaves = _coerce_out(bb, new_leaves, avals)
    body = closed(bb, new_leaves)
    body_consts = bb.captured_outer()

    cb = Builder(current_builder())
    with building(cb):
        cargs = [cb.arg(a) for a in avals]
        pred = cond_fun(_unflatten(struct, cargs))
        if not isinstance(pred, Tracer):
            pred = jnp.full((), bool(pred), BOOL)
        if pred.dtype != BOOL or pred.shape not in ((), (1,)):
            raise TraceError(f"while_loop: cond_fun must return a scalar bool, got {pred.aval.str_short()}")
    cond = closed(cb, [pred])
    cond_consts = cb.captured_outer()
    params = dict(cond_jaxpr=cond, body_jaxpr=body, cond_nconsts=len(cond_consts), body_nconsts=len(body_consts))
    outs = current_builder().add(
        "while", [*cond_consts, *body_consts, *_coerce_init(leaves, avals)], avals, **params
    )
    return _unflatten(struct, outs)


# ---------------------------------------------------------------------------
# conditionals


def _stage_branches(index: Tracer, branches: Sequence[Callable], operands: tuple) -> Any:
    op_leaves, op_struct = _flatten(list(operands))
    op_leaves = [_to_tracer(x) for x in op_leaves]
    op_avals = _avals(op_leaves)
    parent = current_builder()
    traced = []
    for fn in branches:
        b = Builder(parent)
        with building(b):
            args = [b.arg(a) for a in op_avals]
            out = fn(*_unflatten(op_struct, args))
            out_leaves, out_struct = _flatten(out)
            out_leaves = [o if isinstance(o, Tracer) else jnp.full((), o) for o in out_leaves]
        traced.append((b, out_leaves, out_struct))
    ref_avals = [o.aval for o in traced[0][1]]
    for b, outs, _ in traced[1:]:
        if [(o.shape, o.dtype) for o in outs] != [(a.shape, a.dtype) for a in ref_avals]:
            raise TraceError("cond/switch branches must return the same structure, shapes and dtypes")
    # Union of captured outer values, in first-seen order.
    union: dict[int, Tracer] = {}
    for b, _, _ in traced:
        for t in b.captured_outer():
            union.setdefault(id(t.var), t)
    cap_list = list(union.values())
    closed_branches = []
    for b, outs, _ in traced:
        outvars = [b.atom(o) for o in outs]
        own = {id(t.var): v for t, v in b.captures.values()}
        cap_vars = [own.get(id(t.var)) or b.new_var(t.aval) for t in cap_list]
        closed_branches.append(ClosedJaxpr(Jaxpr([], cap_vars + b.invars, outvars, b.eqns), []))
    out_avals = [ShapedArray(a.shape, a.dtype, False) for a in ref_avals]
    outs = parent.add("cond", [index, *cap_list, *op_leaves], out_avals, branches=tuple(closed_branches))
    return _unflatten(traced[0][2], outs)


def cond(pred: Any, true_fun: Callable, false_fun: Callable, *operands: Any) -> Any:
    """`lax.cond`: branch 0 is the false branch, as JAX stages it."""
    if not isinstance(pred, Tracer):
        return (true_fun if pred else false_fun)(*operands)
    if pred.shape not in ((),):
        raise TraceError("lax.cond predicate must be a scalar")
    index = jnp.convert_element_type(pred, I32)
    return _stage_branches(index, [false_fun, true_fun], operands)


def switch(index: Any, branches: Sequence[Callable], *operands: Any) -> Any:
    """`lax.switch`: the index clamps into `[0, len(branches) - 1]`."""
    if not isinstance(index, Tracer):
        i = int(np.clip(int(index), 0, len(branches) - 1))
        return branches[i](*operands)
    index = jnp.convert_element_type(index, I32)
    index = jnp.clamp(0, index, len(branches) - 1)
    return _stage_branches(index, list(branches), operands)
