"""A jaxpr-shaped intermediate representation.

JAX is not importable everywhere this backend runs, so kernels are traced
into this small IR by `palladium_amd.frontend` (a Pallas-like frontend),
or converted from a real JAX kernel jaxpr by `palladium_amd.trace` when JAX
is importable. The attribute names deliberately follow `jax.extend.core`
(`Jaxpr.invars/outvars/eqns/constvars`, `JaxprEqn.primitive.name/params`,
`Var.aval`, `Literal.val`) so lowering rules read the same over either
source, and so user rules written against the reference's
`(env, cursor, eqn)` signature (`src/palladium/emit/core.py:243-256`) keep
working.

Indexed ref accesses carry an `IndexerTree` in `params["tree"]` whose
`unflatten(leaves)` returns `(NDIndexer,)` or `()` exactly like JAX's
`get`/`swap` staging (`src/palladium/emit/rules.py:50,81`).
"""

from __future__ import annotations

import dataclasses
import itertools
from typing import Any

import numpy as np

from palladium_amd.dtypes import name as _dtype_name

__all__ = [
    "ClosedJaxpr",
    "IndexerTree",
    "Jaxpr",
    "JaxprEqn",
    "KeyAval",
    "Literal",
    "NDIndexer",
    "Primitive",
    "RefAval",
    "ShapedArray",
    "Slice",
    "Var",
    "pp_jaxpr",
]

_SHORT = {
    "float32": "f32",
    "float16": "f16",
    "bfloat16": "bf16",
    "float64": "f64",
    "int32": "i32",
    "uint32": "u32",
    "int64": "i64",
    "bool": "bool",
}


class ShapedArray:
    """Abstract value of an array: static shape and dtype.

    `weak_type` marks values that came from Python scalars; binary ops
    take the dtype of their strongly typed operand, as in JAX.
    """

    __slots__ = ("dtype", "shape", "weak_type")

    def __init__(self, shape: tuple[int, ...], dtype: Any, weak_type: bool = False):
        self.shape = tuple(int(d) for d in shape)
        self.dtype = np.dtype(dtype)
        self.weak_type = bool(weak_type)

    @property
    def ndim(self) -> int:
        return len(self.shape)

    @property
    def size(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    def __eq__(self, other: object) -> bool:
        return (
            isinstance(other, ShapedArray)
            and not isinstance(other, (RefAval, KeyAval))
            and self.shape == other.shape
            and self.dtype == other.dtype
        )

    def __hash__(self) -> int:
        return hash((self.shape, self.dtype))

    def str_short(self) -> str:
        dn = _dtype_name(self.dtype)
        name = _SHORT.get(dn, dn)
        return f"{name}[{','.join(str(d) for d in self.shape)}]"

    __repr__ = str_short


class RefAval(ShapedArray):
    """Abstract value of a kernel operand Ref (a block of device memory)."""

    __slots__ = ()

    @property
    def inner_aval(self) -> ShapedArray:
        return ShapedArray(self.shape, self.dtype)

    def str_short(self) -> str:
        return "Ref{" + super().str_short() + "}"

    __repr__ = str_short


class KeyAval(ShapedArray):
    """A Threefry PRNG key (`key<fry>[]` in JAX): a uint32 pair underneath."""

    __slots__ = ()

    def __init__(self, shape: tuple[int, ...] = ()):
        super().__init__(shape, np.uint32)

    def str_short(self) -> str:
        return f"key<fry>[{','.join(str(d) for d in self.shape)}]"

    __repr__ = str_short


_ids = itertools.count()


class Var:
    """A jaxpr variable; identity is object identity, as in JAX."""

    __slots__ = ("aval", "count")

    def __init__(self, aval: ShapedArray):
        self.aval = aval
        self.count = next(_ids)

    def __repr__(self) -> str:
        return f"v{self.count}"


class Literal:
    """An inline constant operand (Python scalar or 0-d array)."""

    __slots__ = ("aval", "val")

    def __init__(self, val: Any, aval: ShapedArray):
        self.val = val
        self.aval = aval

    def __repr__(self) -> str:
        return f"{self.val!r}:{self.aval.str_short()}"


@dataclasses.dataclass(frozen=True)
class Primitive:
    name: str

    def __repr__(self) -> str:
        return self.name


_PRIMS: dict[str, Primitive] = {}


def primitive(name: str) -> Primitive:
    p = _PRIMS.get(name)
    if p is None:
        p = _PRIMS[name] = Primitive(name)
    return p


@dataclasses.dataclass
class JaxprEqn:
    invars: list[Any]
    outvars: list[Var]
    primitive: Primitive
    params: dict[str, Any]


@dataclasses.dataclass
class Jaxpr:
    constvars: list[Var]
    invars: list[Var]
    outvars: list[Any]
    eqns: list[JaxprEqn]

    def __str__(self) -> str:
        return pp_jaxpr(self)


@dataclasses.dataclass
class ClosedJaxpr:
    jaxpr: Jaxpr
    consts: list[Any] = dataclasses.field(default_factory=list)

    @property
    def in_avals(self) -> list[ShapedArray]:
        return [v.aval for v in self.jaxpr.invars]

    @property
    def out_avals(self) -> list[ShapedArray]:
        return [v.aval for v in self.jaxpr.outvars]

    def __str__(self) -> str:
        return pp_jaxpr(self.jaxpr)


@dataclasses.dataclass(frozen=True)
class Slice:
    """`pl.ds(start, size)`: a unit-or-larger stride window of one dim.
    `start` is a Python int or a jaxpr atom (Var/Literal)."""

    start: Any
    size: int
    stride: int = 1


@dataclasses.dataclass(frozen=True)
class NDIndexer:
    """One index per ref dim: a Slice keeps the dim, an atom squeezes it."""

    indices: tuple[Any, ...]
    shape: tuple[int, ...]

    def result_shape(self) -> tuple[int, ...]:
        return tuple(i.size for i in self.indices if isinstance(i, Slice))


class _Leaf:
    """Placeholder for a dynamic index inside an IndexerTree template."""

    __slots__ = ("k",)

    def __init__(self, k: int):
        self.k = k


class IndexerTree:
    """Stand-in for the pytree treedef JAX stores in `get`/`swap` params.

    Holds an NDIndexer template whose dynamic positions are `_Leaf`
    placeholders; `unflatten(leaves)` substitutes the eqn's index invars.
    An empty tree (`x_ref[...]` in older JAX) unflattens to `()`.
    """

    def __init__(self, template: NDIndexer | None, num_leaves: int):
        self.template = template
        self.num_leaves = num_leaves

    def unflatten(self, leaves: list[Any]) -> tuple[NDIndexer, ...]:
        leaves = list(leaves)
        if len(leaves) != self.num_leaves:
            raise ValueError(f"expected {self.num_leaves} index leaves, got {len(leaves)}")
        if self.template is None:
            return ()

        def sub(x: Any) -> Any:
            return leaves[x.k] if isinstance(x, _Leaf) else x

        out = []
        for idx in self.template.indices:
            if isinstance(idx, Slice):
                out.append(Slice(sub(idx.start), idx.size, idx.stride))
            else:
                out.append(sub(idx))
        return (NDIndexer(tuple(out), self.template.shape),)

    def __repr__(self) -> str:
        if self.template is None:
            return "[...]"
        parts = []
        for idx in self.template.indices:
            if isinstance(idx, Slice):
                st = f"#{idx.start.k}" if isinstance(idx.start, _Leaf) else str(idx.start)
                parts.append(f"{st}:+{idx.size}" + (f":{idx.stride}" if idx.stride != 1 else ""))
            else:
                parts.append(f"#{idx.k}" if isinstance(idx, _Leaf) else repr(idx))
        return "[" + ", ".join(parts) + "]"


def pp_jaxpr(jaxpr: Jaxpr, indent: int = 0) -> str:
    """Readable text form, for debugging and golden IR snapshots."""
    pad = "  " * indent

    def atom(a: Any) -> str:
        return repr(a)

    def decl(v: Var) -> str:
        return f"{v!r}:{v.aval.str_short()}"

    lines = [
        pad
        + "{ lambda "
        + " ".join(decl(v) for v in jaxpr.constvars)
        + " ; "
        + " ".join(decl(v) for v in jaxpr.invars)
        + ". let"
    ]
    for e in jaxpr.eqns:
        simple = {}
        subs = []
        for k, v in e.params.items():
            if isinstance(v, ClosedJaxpr):
                subs.append((k, v.jaxpr))
            elif isinstance(v, Jaxpr):
                subs.append((k, v))
            elif isinstance(v, tuple) and v and all(isinstance(b, ClosedJaxpr) for b in v):
                for i, b in enumerate(v):
                    subs.append((f"{k}[{i}]", b.jaxpr))
            else:
                simple[k] = v
        ps = ", ".join(f"{k}={v!r}" for k, v in simple.items())
        lhs = " ".join(decl(v) for v in e.outvars) or "_"
        lines.append(f"{pad}    {lhs} = {e.primitive.name}[{ps}] " + " ".join(atom(a) for a in e.invars))
        for k, sj in subs:
            lines.append(f"{pad}      {k}:")
            lines.append(pp_jaxpr(sj, indent + 4))
    lines.append(pad + "  in ( " + " ".join(atom(a) for a in jaxpr.outvars) + " ) }")
    return "\n".join(lines)
