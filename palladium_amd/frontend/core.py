"""Tracing machinery of the Pallas-like frontend.

A `Builder` records equations for one (sub-)jaxpr; `Tracer`s are the
values user code manipulates. Closing over a tracer of an enclosing
builder (a loop body reading `a` from the kernel scope) captures it as a
const input of the inner jaxpr, the way JAX's `fori_loop`/`while_loop`
stage closed-over values as consts (`src/palladium/emit/rules.py:683-703`,
`812-837` consume that layout).

Dtype rules follow JAX with x64 disabled: Python floats are weakly typed
float32, Python ints weakly typed int32, and a weak operand takes the dtype
of the strong one.
"""

from __future__ import annotations

import contextlib
import math
import threading
from typing import Any, Iterator

import numpy as np

from palladium_amd import dtypes as _dtypes
from palladium_amd.errors import TraceError
from palladium_amd.ir import (
    ClosedJaxpr,
    Jaxpr,
    JaxprEqn,
    KeyAval,
    Literal,
    RefAval,
    ShapedArray,
    Var,
    primitive,
)

F32 = np.dtype(np.float32)
I32 = np.dtype(np.int32)
U32 = np.dtype(np.uint32)
BOOL = np.dtype(np.bool_)

F16 = np.dtype(np.float16)
BF16 = _dtypes.bfloat16

SUPPORTED_DTYPES = (F32, F16, BF16, I32, U32, BOOL)

_state = threading.local()


def _stack() -> list["Builder"]:
    st = getattr(_state, "stack", None)
    if st is None:
        st = _state.stack = []
    return st


def current_builder() -> "Builder":
    st = _stack()
    if not st:
        raise TraceError(
            "palladium_amd frontend op called outside a kernel trace; "
            "kernel functions run only under pallas_call tracing"
        )
    return st[-1]


class Builder:
    """Collects the equations of one jaxpr level."""

    def __init__(self, parent: "Builder | None" = None):
        self.parent = parent
        self.eqns: list[JaxprEqn] = []
        self.invars: list[Var] = []
        # Captured outer values, in first-use order: outer Tracer -> inner Var.
        self.captures: dict[int, tuple["Tracer", Var]] = {}
        self.owned: set[int] = set()

    def new_var(self, aval: ShapedArray) -> Var:
        v = Var(aval)
        self.owned.add(id(v))
        return v

    def arg(self, aval: ShapedArray) -> "Tracer":
        v = self.new_var(aval)
        self.invars.append(v)
        return Tracer(self, v)

    def atom(self, x: Any) -> Any:
        """Var or Literal in this builder's scope for a Tracer or scalar."""
        if isinstance(x, Tracer):
            if x.builder is self:
                return x.var
            key = id(x.var)
            hit = self.captures.get(key)
            if hit is not None:
                return hit[1]
            if self.parent is None:
                raise TraceError("tracer escaped its kernel trace")
            # Make sure every intermediate level sees it too.
            self.parent.atom(x)
            v = self.new_var(x.var.aval)
            self.captures[key] = (x, v)
            return v
        if isinstance(x, Literal):
            return x
        raise TypeError(f"not a traced value: {x!r}")

    def add(self, _name: str, invals: list[Any], out_avals: list[ShapedArray], **params: Any) -> list["Tracer"]:
        ins = [self.atom(v) for v in invals]
        outs = [self.new_var(a) for a in out_avals]
        self.eqns.append(JaxprEqn(ins, outs, primitive(_name), params))
        return [Tracer(self, o) for o in outs]

    def captured_outer(self) -> list["Tracer"]:
        return [t for t, _ in self.captures.values()]

    def captured_vars(self) -> list[Var]:
        return [v for _, v in self.captures.values()]


@contextlib.contextmanager
def building(builder: Builder) -> Iterator[Builder]:
    st = _stack()
    st.append(builder)
    try:
        yield builder
    finally:
        st.pop()


def literal(value: Any, dtype: Any, weak: bool = True) -> Literal:
    dtype = np.dtype(dtype)
    if isinstance(value, np.ndarray) and _dtypes.is_bf16(value.dtype):
        value = float(_dtypes.to_float(value).reshape(()))
    if dtype == BOOL:
        val: Any = bool(value)
    elif _dtypes.is_bf16(dtype):
        val = _dtypes.scalar_f32(value)
    elif dtype.kind == "f":
        val = float(np.asarray(value, dtype=dtype))
    elif dtype.kind in "iu":
        val = int(np.asarray(value).astype(dtype))
    else:
        raise TraceError(f"unsupported literal dtype {dtype}")
    return Literal(val, ShapedArray((), dtype, weak_type=weak))


class Tracer:
    """A traced array value inside a kernel."""

    __slots__ = ("builder", "var")
    __array_priority__ = 1000

    def __init__(self, builder: Builder, var: Var):
        self.builder = builder
        self.var = var

    @property
    def aval(self) -> ShapedArray:
        return self.var.aval

    @property
    def shape(self) -> tuple[int, ...]:
        return self.var.aval.shape

    @property
    def dtype(self) -> np.dtype:
        return self.var.aval.dtype

    @property
    def ndim(self) -> int:
        return len(self.shape)

    @property
    def size(self) -> int:
        return math.prod(self.shape)

    @property
    def weak_type(self) -> bool:
        return self.var.aval.weak_type

    def __repr__(self) -> str:
        return f"Tracer<{self.aval.str_short()}>"

    def __bool__(self) -> bool:
        raise TraceError(
            "a traced value has no concrete truth value; use lax.cond, "
            "lax.while_loop or jnp.where for data-dependent control flow"
        )

    def __index__(self) -> int:
        raise TraceError("a traced value cannot be used as a Python int")

    def __len__(self) -> int:
        if not self.shape:
            raise TypeError("len() of unsized traced value")
        return self.shape[0]

    def __hash__(self) -> int:
        return id(self)

    # Arithmetic / comparison operators route through jnp.
    def __add__(self, o): return _jnp().add(self, o)
    def __radd__(self, o): return _jnp().add(o, self)
    def __sub__(self, o): return _jnp().subtract(self, o)
    def __rsub__(self, o): return _jnp().subtract(o, self)
    def __mul__(self, o): return _jnp().multiply(self, o)
    def __rmul__(self, o): return _jnp().multiply(o, self)
    def __truediv__(self, o): return _jnp().divide(self, o)
    def __rtruediv__(self, o): return _jnp().divide(o, self)
    def __pow__(self, o): return _jnp().power(self, o)
    def __rpow__(self, o): return _jnp().power(o, self)
    def __matmul__(self, o): return _jnp().matmul(self, o)
    def __rmatmul__(self, o): return _jnp().matmul(o, self)
    def __neg__(self): return _jnp().negative(self)
    def __pos__(self): return self
    def __abs__(self): return _jnp().abs(self)
    def __lt__(self, o): return _jnp().less(self, o)
    def __le__(self, o): return _jnp().less_equal(self, o)
    def __gt__(self, o): return _jnp().greater(self, o)
    def __ge__(self, o): return _jnp().greater_equal(self, o)
    def __eq__(self, o): return _jnp().equal(self, o)  # type: ignore[override]
    def __ne__(self, o): return _jnp().not_equal(self, o)  # type: ignore[override]
    def __and__(self, o): return _jnp().bitwise_and(self, o)
    def __rand__(self, o): return _jnp().bitwise_and(o, self)
    def __or__(self, o): return _jnp().bitwise_or(self, o)
    def __ror__(self, o): return _jnp().bitwise_or(o, self)
    def __xor__(self, o): return _jnp().bitwise_xor(self, o)
    def __rxor__(self, o): return _jnp().bitwise_xor(o, self)
    def __invert__(self): return _jnp().invert(self)
    def __rshift__(self, o): return _jnp().right_shift(self, o)
    def __lshift__(self, o): return _jnp().left_shift(self, o)
    def __mod__(self, o): return _jnp().remainder(self, o)
    def __floordiv__(self, o): return _jnp().floor_divide(self, o)

    def astype(self, dtype: Any) -> "Tracer":
        return _jnp().astype(self, dtype)

    def reshape(self, *shape: Any) -> "Tracer":
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        return _jnp().reshape(self, shape)

    def __getitem__(self, idx: Any) -> "Tracer":
        return _jnp()._value_getitem(self, idx)

    @property
    def T(self) -> "Tracer":
        return _jnp().transpose(self)


def _jnp():
    from palladium_amd.frontend import jnp

    return jnp


def is_value(x: Any) -> bool:
    return isinstance(x, (Tracer, int, float, bool, np.number, np.bool_)) or (
        isinstance(x, np.ndarray) and x.ndim == 0
    )


def scalar_kind(x: Any) -> str:
    if isinstance(x, (bool, np.bool_)):
        return "b"
    if isinstance(x, (int, np.integer)):
        return "i"
    return "f"


def default_dtype(x: Any) -> np.dtype:
    if isinstance(x, np.generic) or (isinstance(x, np.ndarray) and x.ndim == 0):
        return np.dtype(x.dtype) if np.dtype(x.dtype) in SUPPORTED_DTYPES else {
            "f": F32, "i": I32, "u": U32, "b": BOOL
        }[np.dtype(x.dtype).kind]
    return {"b": BOOL, "i": I32, "f": F32}[scalar_kind(x)]


def check_dtype(dtype: Any) -> np.dtype:
    dt = np.dtype(dtype)
    if dt not in SUPPORTED_DTYPES:
        raise TraceError(
            f"dtype {_dtypes.name(dt)} is not supported in kernels "
            f"(supported: {', '.join(_dtypes.name(d) for d in SUPPORTED_DTYPES)})"
        )
    return dt


def closed(builder: Builder, outs: list[Any]) -> ClosedJaxpr:
    """Finish a sub-builder: captured consts first, then its own args."""
    outvars = [builder.atom(o) for o in outs]
    jaxpr = Jaxpr([], builder.captured_vars() + builder.invars, outvars, builder.eqns)
    return ClosedJaxpr(jaxpr, [])


def key_aval() -> KeyAval:
    return KeyAval(())


def ref_aval(shape: tuple[int, ...], dtype: Any) -> RefAval:
    return RefAval(shape, dtype)
