"""`jax.numpy`-shaped array ops for kernels traced by the frontend.

Each function stages the same primitive(s) that `jax.numpy` stages for
the corresponding call inside a Pallas kernel, so a kernel body written
against `jax.numpy` traces to the same equation sequence (and therefore
the same float op order) here. Primitive names are JAX's
(`src/palladium/emit/core.py:568-601` lists the elementwise subset the
reference lowers).
"""

from __future__ import annotations

import builtins
import math
from typing import Any, Sequence

import numpy as np

from palladium_amd.errors import TraceError
from palladium_amd.frontend.core import (
    BOOL,
    F32,
    I32,
    U32,
    Tracer,
    check_dtype,
    current_builder,
    default_dtype,
    literal,
)
from palladium_amd.dtypes import bfloat16_type as _bfloat16_type
from palladium_amd.dtypes import kind as _kind
from palladium_amd.ir import KeyAval, Literal, ShapedArray

float32 = np.float32
float16 = np.float16
bfloat16 = _bfloat16_type
int32 = np.int32
uint32 = np.uint32
bool_ = np.bool_
pi = math.pi
e = math.e
inf = math.inf
nan = math.nan

# ---------------------------------------------------------------------------
# operand normalisation


def _is_tracer(x: Any) -> bool:
    return isinstance(x, Tracer)


def _weak(x: Any) -> bool:
    if isinstance(x, Tracer):
        return x.weak_type
    return not isinstance(x, (np.generic, np.ndarray))


def _dtype_of(x: Any) -> np.dtype:
    return x.dtype if isinstance(x, Tracer) else default_dtype(x)


def _shape_of(x: Any) -> tuple[int, ...]:
    return x.shape if isinstance(x, Tracer) else ()


def _broadcast_shapes(*shapes: tuple[int, ...]) -> tuple[int, ...]:
    try:
        return tuple(np.broadcast_shapes(*shapes))
    except ValueError:
        raise TraceError(f"incompatible shapes for broadcasting: {shapes}") from None


def _result_dtype(args: Sequence[Any]) -> np.dtype:
    strong = [_dtype_of(a) for a in args if not _weak(a)]
    weak = [_dtype_of(a) for a in args if _weak(a)]
    kinds = "biuf"
    if strong:
        dt = strong[0]
        for d in strong[1:]:
            if d != dt:
                if _kind(d) == "f" and _kind(dt) == "f":
                    dt = F32  # float16 with float32
                elif _kind(d) == "f" or _kind(dt) == "f":
                    dt = d if _kind(d) == "f" else dt
                elif {d, dt} <= {I32, U32, BOOL}:
                    dt = I32 if BOOL in (d, dt) and U32 not in (d, dt) else (U32 if U32 in (d, dt) and BOOL in (d, dt) else I32)
                else:
                    raise TraceError(f"cannot mix dtypes {dt} and {d}; cast explicitly")
        # A weak float meeting a strong int promotes to float (JAX semantics).
        if _kind(dt) in "iub" and builtins.any(_kind(w) == "f" for w in weak):
            return F32
        if dt == BOOL and builtins.any(_kind(w) in "iu" for w in weak):
            return I32
        return dt
    best = builtins.max(weak, key=lambda d: kinds.index(_kind(d)))
    return {"f": F32, "i": I32, "u": U32, "b": BOOL}[_kind(best)]


def _as_operand(x: Any, dtype: np.dtype, shape: tuple[int, ...]) -> Any:
    """Tracer (converted/broadcast as needed) or scalar Literal."""
    if isinstance(x, Tracer):
        if x.dtype != dtype:
            x = convert_element_type(x, dtype, weak_type=x.weak_type)
        if x.shape != shape and x.shape != ():
            x = broadcast_to(x, shape)
        elif x.shape == () and shape != ():
            x = broadcast_to(x, shape)
        return x
    if isinstance(x, np.ndarray) and x.ndim > 0:
        raise TraceError(
            "kernels cannot capture NumPy arrays (jaxpr constvars); pass "
            "arrays as kernel operands"
        )
    return literal(x, dtype, weak=True)


def _stage(_name: str, _ins: list[Any], _shape: tuple[int, ...], _dtype: np.dtype, _weak: bool = False, **params: Any) -> Tracer:
    b = current_builder()
    (out,) = b.add(_name, _ins, [ShapedArray(_shape, _dtype, _weak)], **params)
    return out


def _nary(name: str, *args: Any, out_dtype: np.dtype | None = None, **params: Any) -> Any:
    if not builtins.any(_is_tracer(a) for a in args):
        # All-constant: stage on a literal broadcast so the op stays traced.
        args = (full((), args[0], dtype=default_dtype(args[0])),) + args[1:]
    dt = _result_dtype(args)
    shape = _broadcast_shapes(*[_shape_of(a) for a in args])
    ins = [_as_operand(a, dt, shape) for a in args]
    weak = builtins.all(_weak(a) for a in args)
    return _stage(name, ins, shape, out_dtype or dt, weak if out_dtype is None else False, **params)


def _unary(name: str, x: Any, float_only: bool = False, **params: Any) -> Tracer:
    if not isinstance(x, Tracer):
        x = full((), x, dtype=default_dtype(x))
    if float_only and _kind(x.dtype) != "f":
        x = convert_element_type(x, F32)
    return _stage(name, [x], x.shape, x.dtype, x.weak_type, **params)


# ---------------------------------------------------------------------------
# structural


def convert_element_type(x: Any, dtype: Any, weak_type: bool = False) -> Tracer:
    dt = check_dtype(dtype)
    if not isinstance(x, Tracer):
        return full((), x, dtype=dt)
    if x.dtype == dt and x.weak_type == weak_type:
        return x
    return _stage("convert_element_type", [x], x.shape, dt, weak_type, new_dtype=dt, weak_type=weak_type)


def astype(x: Any, dtype: Any) -> Tracer:
    return convert_element_type(x, dtype)


def bitcast_convert_type(x: Tracer, dtype: Any) -> Tracer:
    dt = check_dtype(dtype)
    if dt.itemsize != x.dtype.itemsize:
        raise TraceError("bitcast_convert_type between different widths is unsupported")
    return _stage("bitcast_convert_type", [x], x.shape, dt, new_dtype=dt)


def broadcast_in_dim(x: Any, shape: Sequence[int], broadcast_dimensions: Sequence[int]) -> Tracer:
    shape = tuple(int(s) for s in shape)
    if not isinstance(x, Tracer):
        lit = literal(x, default_dtype(x))
        return _stage("broadcast_in_dim", [lit], shape, lit.aval.dtype, True, shape=shape, broadcast_dimensions=tuple(broadcast_dimensions), sharding=None)
    return _stage(
        "broadcast_in_dim", [x], shape, x.dtype, x.weak_type,
        shape=shape, broadcast_dimensions=tuple(int(d) for d in broadcast_dimensions), sharding=None,
    )


def broadcast_to(x: Any, shape: Sequence[int]) -> Tracer:
    shape = tuple(int(s) for s in shape)
    xs = _shape_of(x)
    if isinstance(x, Tracer) and xs == shape:
        return x
    if len(xs) > len(shape):
        raise TraceError(f"cannot broadcast {xs} to {shape}")
    lead = len(shape) - len(xs)
    for d, s in enumerate(xs):
        if s != 1 and s != shape[lead + d]:
            raise TraceError(f"cannot broadcast {xs} to {shape}")
    # Size-1 dims that grow: JAX first squeezes them (reshape) and then
    # broadcasts; we express both through broadcast_in_dim directly.
    if isinstance(x, Tracer) and builtins.any(s == 1 and shape[lead + d] != 1 for d, s in enumerate(xs)):
        keep = [d for d, s in enumerate(xs) if not (s == 1 and shape[lead + d] != 1)]
        x = reshape(x, tuple(xs[d] for d in keep))
        return broadcast_in_dim(x, shape, tuple(lead + d for d in keep))
    return broadcast_in_dim(x, shape, tuple(range(lead, len(shape))))


def reshape(x: Tracer, new_sizes: Sequence[int]) -> Tracer:
    new = list(new_sizes)
    if -1 in new:
        k = new.index(-1)
        rest = math.prod(n for i, n in enumerate(new) if i != k)
        new[k] = x.size // rest
    new_t = tuple(int(n) for n in new)
    if math.prod(new_t) != x.size:
        raise TraceError(f"cannot reshape {x.shape} to {new_t}")
    if new_t == x.shape:
        return x
    return _stage("reshape", [x], new_t, x.dtype, x.weak_type, new_sizes=new_t, dimensions=None, sharding=None)


def dot_general(lhs: Any, rhs: Any, dimension_numbers: Any, precision: Any = None,
                preferred_element_type: Any = None) -> Tracer:
    """Stage `dot_general` as JAX does: output dims are the batch dims, then
    the lhs free dims, then the rhs free dims. (Batch dims stage like JAX's
    and are rejected by the emitter, as the reference's emitter does.)"""
    (lc, rc), (lb, rb) = dimension_numbers
    lc, rc, lb, rb = (tuple(int(d) for d in t) for t in (lc, rc, lb, rb))
    if len(lb) != len(rb):
        raise TraceError("dot_general: lhs and rhs batch dims differ in number")
    if not isinstance(lhs, Tracer):
        lhs = asarray(lhs)
    if not isinstance(rhs, Tracer):
        rhs = asarray(rhs)
    if len(lc) != len(rc) or builtins.any(lhs.shape[a] != rhs.shape[b] for a, b in zip(lc, rc)):
        raise TraceError(f"dot_general: contracting dims disagree ({lhs.shape} vs {rhs.shape})")
    dt = _result_dtype([lhs, rhs])
    if lhs.dtype != dt:
        lhs = convert_element_type(lhs, dt)
    if rhs.dtype != dt:
        rhs = convert_element_type(rhs, dt)
    out_dt = np.dtype(preferred_element_type) if preferred_element_type is not None else dt
    shape = tuple(lhs.shape[k] for k in lb) + tuple(d for k, d in enumerate(lhs.shape) if k not in lc + lb) + tuple(
        d for k, d in enumerate(rhs.shape) if k not in rc + rb)
    return _stage("dot_general", [lhs, rhs], shape, out_dt, False,
                  dimension_numbers=((lc, rc), (lb, rb)), precision=precision,
                  preferred_element_type=out_dt, out_sharding=None)


def dot(a: Any, b: Any, *, precision: Any = None, preferred_element_type: Any = None) -> Tracer:
    """`jnp.dot` for rank <= 2: contracts a's last dim with b's first
    (b's only dim when b is a vector)."""
    a_nd = len(_shape_of(a))
    b_nd = len(_shape_of(b))
    if a_nd == 0 or b_nd == 0:
        return multiply(a, b)
    if a_nd > 2 or b_nd > 2:
        raise TraceError("dot: operands of rank > 2 are not supported")
    rc = 0 if b_nd == 1 else b_nd - 2
    return dot_general(a, b, (((a_nd - 1,), (rc,)), ((), ())), precision, preferred_element_type)


def matmul(a: Any, b: Any, *, precision: Any = None, preferred_element_type: Any = None) -> Tracer:
    if len(_shape_of(a)) == 0 or len(_shape_of(b)) == 0:
        raise TraceError("matmul: operands must have rank >= 1")
    return dot(a, b, precision=precision, preferred_element_type=preferred_element_type)


def vdot(a: Tracer, b: Tracer) -> Tracer:
    return dot(reshape(a, (math.prod(a.shape),)), reshape(b, (math.prod(b.shape),)))


def transpose(x: Tracer, axes: Sequence[int] | None = None) -> Tracer:
    perm = tuple(axes) if axes is not None else tuple(reversed(range(x.ndim)))
    shape = tuple(x.shape[p] for p in perm)
    return _stage("transpose", [x], shape, x.dtype, x.weak_type, permutation=perm)


def full(shape: Sequence[int] | int, fill_value: Any, dtype: Any = None) -> Tracer:
    if isinstance(shape, int):
        shape = (shape,)
    dt = check_dtype(dtype) if dtype is not None else _dtype_of(fill_value)
    if isinstance(fill_value, Tracer):
        return broadcast_to(convert_element_type(fill_value, dt), tuple(shape))
    lit = literal(fill_value, dt, weak=dtype is None)
    return _stage("broadcast_in_dim", [lit], tuple(shape), dt, dtype is None, shape=tuple(shape), broadcast_dimensions=(), sharding=None)


def zeros(shape: Sequence[int] | int, dtype: Any = F32) -> Tracer:
    return full(shape, 0, dtype)


def ones(shape: Sequence[int] | int, dtype: Any = F32) -> Tracer:
    return full(shape, 1, dtype)


def full_like(x: Tracer, fill_value: Any, dtype: Any = None) -> Tracer:
    return full(x.shape, fill_value, dtype if dtype is not None else x.dtype)


def zeros_like(x: Tracer, dtype: Any = None) -> Tracer:
    return full_like(x, 0, dtype)


def ones_like(x: Tracer, dtype: Any = None) -> Tracer:
    return full_like(x, 1, dtype)


def asarray(x: Any, dtype: Any = None) -> Any:
    if isinstance(x, Tracer):
        return x if dtype is None else convert_element_type(x, dtype)
    return full((), x, dtype)


array = asarray

# ---------------------------------------------------------------------------
# elementwise


def add(a, b): return _nary("add", a, b)
def subtract(a, b): return _nary("sub", a, b)
def multiply(a, b): return _nary("mul", a, b)
def minimum(a, b): return _nary("min", a, b)
def maximum(a, b): return _nary("max", a, b)


def divide(a: Any, b: Any) -> Tracer:
    dt = _result_dtype((a, b))
    if _kind(dt) != "f":
        a = convert_element_type(a, F32) if isinstance(a, Tracer) else float(a)
        b = convert_element_type(b, F32) if isinstance(b, Tracer) else float(b)
    return _nary("div", a, b)


true_divide = divide


def floor_divide(a: Any, b: Any) -> Tracer:
    dt = _result_dtype((a, b))
    if _kind(dt) == "f":
        return floor(divide(a, b))
    q = _nary("div", a, b)
    r = _nary("rem", a, b)
    fix = logical_and(not_equal(r, 0), not_equal(less(r, 0), less(b, 0)))
    return where(fix, subtract(q, 1), q)


def remainder(a: Any, b: Any) -> Tracer:
    return _nary("rem", a, b)


def power(a: Any, b: Any) -> Tracer:
    if isinstance(b, (int, np.integer)) and not isinstance(b, bool) and isinstance(a, Tracer):
        return integer_pow(a, int(b))
    return _nary("pow", a, b)


def integer_pow(x: Tracer, y: int) -> Tracer:
    return _stage("integer_pow", [x], x.shape, x.dtype, x.weak_type, y=int(y))


def square(x: Tracer) -> Tracer:
    return integer_pow(x, 2)


def negative(x): return _unary("neg", x)


def abs(x: Any) -> Tracer:  # noqa: A001
    return _unary("abs", x)


absolute = abs


def sign(x): return _unary("sign", x)
def exp(x): return _unary("exp", x, True)
def exp2(x): return _unary("exp2", x, True)
def log(x): return _unary("log", x, True)
def log1p(x): return _unary("log1p", x, True)
def expm1(x): return _unary("expm1", x, True)
def sin(x): return _unary("sin", x, True)
def cos(x): return _unary("cos", x, True)
def tan(x): return _unary("tan", x, True)
def tanh(x): return _unary("tanh", x, True)
def sqrt(x): return _unary("sqrt", x, True)
def rsqrt(x): return _unary("rsqrt", x, True)
def round(x, decimals: int = 0):  # noqa: A001
    """Nearest integer, ties to even (numpy's and JAX's jnp.round)."""
    if decimals:
        raise TraceError("jnp.round with decimals != 0 is not supported in kernels")
    return _unary("round", x, True, rounding_method=1)


def rint(x): return round(x)
def floor(x): return _unary("floor", x, True)
def ceil(x): return _unary("ceil", x, True)
def logistic(x): return _unary("logistic", x, True)


def arctan2(a, b): return _nary("atan2", a, b)


def less(a, b): return _nary("lt", a, b, out_dtype=BOOL)
def less_equal(a, b): return _nary("le", a, b, out_dtype=BOOL)
def greater(a, b): return _nary("gt", a, b, out_dtype=BOOL)
def greater_equal(a, b): return _nary("ge", a, b, out_dtype=BOOL)
def equal(a, b): return _nary("eq", a, b, out_dtype=BOOL)
def not_equal(a, b): return _nary("ne", a, b, out_dtype=BOOL)


def _int_or_bool(name: str, a: Any, b: Any) -> Tracer:
    dt = _result_dtype((a, b))
    if _kind(dt) == "f":
        raise TraceError(f"{name} requires integer or bool operands")
    return _nary(name, a, b)


def bitwise_and(a, b): return _int_or_bool("and", a, b)
def bitwise_or(a, b): return _int_or_bool("or", a, b)
def bitwise_xor(a, b): return _int_or_bool("xor", a, b)
logical_and = bitwise_and
logical_or = bitwise_or
logical_xor = bitwise_xor


def invert(x: Tracer) -> Tracer:
    if _kind(x.dtype) == "f":
        raise TraceError("~ requires an integer or bool operand")
    return _unary("not", x)


bitwise_not = invert
logical_not = invert


def right_shift(a: Any, b: Any) -> Tracer:
    dt = _result_dtype((a, b))
    if dt == U32:
        return _nary("shift_right_logical", a, b)
    if dt == I32:
        return _nary("shift_right_arithmetic", a, b)
    raise TraceError(">> requires integer operands")


def left_shift(a: Any, b: Any) -> Tracer:
    return _int_or_bool("shift_left", a, b)


def where(condition: Any, x: Any, y: Any) -> Tracer:
    """`jnp.where` stages `select_n(pred, y, x)`: case 0 when false."""
    if not isinstance(condition, Tracer):
        condition = full((), bool(condition), dtype=BOOL)
    if condition.dtype != BOOL:
        condition = not_equal(condition, 0)
    dt = _result_dtype((x, y))
    shape = _broadcast_shapes(condition.shape, _shape_of(x), _shape_of(y))
    xv = _as_operand(x, dt, shape)
    yv = _as_operand(y, dt, shape)
    if isinstance(xv, Literal) and isinstance(yv, Literal):
        xv = full(shape, xv.val, dt)
    pred = condition if condition.shape == shape else broadcast_to(condition, shape)
    weak = _weak(x) and _weak(y)
    return _stage("select_n", [pred, yv, xv], shape, dt, weak)


def select_n(which: Tracer, *cases: Any) -> Tracer:
    dt = _result_dtype(cases)
    shape = _broadcast_shapes(which.shape, *[_shape_of(c) for c in cases])
    ins = [_as_operand(c, dt, shape) for c in cases]
    return _stage("select_n", [which, *ins], shape, dt)


def clip(x: Any, min: Any = None, max: Any = None) -> Tracer:  # noqa: A002
    if min is not None:
        x = maximum(min, x)
    if max is not None:
        x = minimum(max, x)
    return x


def clamp(lo: Any, x: Tracer, hi: Any) -> Tracer:
    """`lax.clamp(min, x, max)`."""
    return _nary("clamp", lo, x, hi)


# ---------------------------------------------------------------------------
# reductions


def _reduce(name: str, x: Tracer, axis: Any, out_dtype: np.dtype | None = None, keepdims: bool = False) -> Tracer:
    if not isinstance(x, Tracer):
        x = asarray(x)
    if axis is None:
        axes = tuple(range(x.ndim))
    elif x.ndim == 0:
        raise TraceError(f"{name}: axis {axis} is out of range for a rank-0 value")
    elif isinstance(axis, int):
        axes = (axis % x.ndim,)
    else:
        axes = tuple(int(a) % x.ndim for a in axis)
    axes = tuple(sorted(set(axes)))
    shape = tuple(s for d, s in enumerate(x.shape) if d not in axes)
    r = _stage(name, [x], shape, out_dtype or x.dtype, axes=axes, out_sharding=None)
    if keepdims:
        # JAX stages keepdims as a broadcast_in_dim onto the size-1 axes.
        kshape = tuple(1 if d in axes else s for d, s in enumerate(x.shape))
        r = broadcast_in_dim(r, kshape, tuple(d for d in range(x.ndim) if d not in axes))
    return r


def sum(x: Tracer, axis: Any = None, keepdims: bool = False) -> Tracer:  # noqa: A001
    if isinstance(x, Tracer) and x.dtype == BOOL:
        x = convert_element_type(x, I32)
    return _reduce("reduce_sum", x, axis, keepdims=keepdims)


def max(x: Tracer, axis: Any = None, keepdims: bool = False) -> Tracer:  # noqa: A001
    return _reduce("reduce_max", x, axis, keepdims=keepdims)


def min(x: Tracer, axis: Any = None, keepdims: bool = False) -> Tracer:  # noqa: A001
    return _reduce("reduce_min", x, axis, keepdims=keepdims)


def any(x: Tracer, axis: Any = None, keepdims: bool = False) -> Tracer:  # noqa: A001
    if x.dtype != BOOL:
        x = not_equal(x, 0)
    return _reduce("reduce_or", x, axis, keepdims=keepdims)


def all(x: Tracer, axis: Any = None, keepdims: bool = False) -> Tracer:  # noqa: A001
    if x.dtype != BOOL:
        x = not_equal(x, 0)
    return _reduce("reduce_and", x, axis, keepdims=keepdims)


def mean(x: Tracer, axis: Any = None, keepdims: bool = False) -> Tracer:
    """Sum, then divide by the reduced element count (integers promote to
    float32, as in JAX)."""
    if _kind(x.dtype) != "f":
        x = convert_element_type(x, F32)
    s = _reduce("reduce_sum", x, axis, keepdims=keepdims)
    n = x.size // builtins.max(s.size, 1)
    return divide(s, float(n))


# ---------------------------------------------------------------------------
# values


def _value_getitem(x: Tracer, idx: Any) -> Tracer:
    if idx is Ellipsis:
        return x
    raise TraceError(
        "indexing a traced value is unsupported; index the Ref instead "
        "(x_ref[i]) or use reshape/where"
    )


def _is_key(x: Any) -> bool:
    return isinstance(x, Tracer) and isinstance(x.aval, KeyAval)


def broadcasted_iota(dtype: Any, shape: Sequence[int], dimension: int) -> Tracer:
    """`lax.broadcasted_iota`: the index along `dimension`, as `dtype`."""
    dt = check_dtype(dtype)
    shape = tuple(int(s) for s in shape)
    return _stage("iota", [], shape, dt, dtype=dt, shape=shape, dimension=int(dimension), sharding=None)


def arange(n: int, dtype: Any = np.int32) -> Tracer:
    return broadcasted_iota(dtype, (int(n),), 0)
