"""`jax.experimental.pallas`-shaped kernel staging.

`pallas_call(kernel, out_shape=..., grid=..., in_specs=..., out_specs=...)`
returns a `PallasCall`; `palladium_amd.trace` turns it into a KernelSpec
by tracing the kernel over `Ref`s of the per-instance block shapes and
tracing each BlockSpec index map over int32 grid indices — the same
information the reference extracts from JAX's `grid_mapping`
(`src/palladium/trace.py:102-177`).

Block dims follow `src/palladium/trace.py:83-99`: ints and `Blocked`
keep a dim, `None`/`Squeezed` drop it from the kernel-visible block.
"""

from __future__ import annotations

import dataclasses
import math
import threading
from builtins import max as builtins_max
from builtins import min as builtins_min
from typing import Any, Callable, Sequence

import numpy as np

from palladium_amd.dtypes import name as _dtype_name
from palladium_amd.errors import TraceError
from palladium_amd.frontend import jnp
from palladium_amd.frontend.core import (
    I32,
    Builder,
    Tracer,
    building,
    check_dtype,
    current_builder,
    literal,
)
from palladium_amd.ir import (
    ClosedJaxpr,
    IndexerTree,
    Jaxpr,
    NDIndexer,
    RefAval,
    ShapedArray,
    Slice,
    _Leaf,
)

__all__ = [
    "BlockSpec",
    "Blocked",
    "PallasCall",
    "ShapeDtypeStruct",
    "Slice",
    "Squeezed",
    "ds",
    "dslice",
    "num_programs",
    "pallas_call",
    "program_id",
]


@dataclasses.dataclass(frozen=True)
class ShapeDtypeStruct:
    """`jax.ShapeDtypeStruct`: a shape and dtype, no data."""

    shape: tuple[int, ...]
    dtype: Any

    def __post_init__(self) -> None:
        object.__setattr__(self, "shape", tuple(int(s) for s in self.shape))
        object.__setattr__(self, "dtype", np.dtype(self.dtype))


@dataclasses.dataclass(frozen=True)
class Blocked:
    block_size: int


@dataclasses.dataclass(frozen=True)
class Squeezed:
    pass


squeezed = Squeezed()


@dataclasses.dataclass(frozen=True)
class Element:
    block_size: int


class BlockSpec:
    """Per-instance block of an operand: `block_shape` plus an index map
    from grid indices to block indices (units of blocks)."""

    def __init__(self, block_shape: Sequence[Any] | None = None, index_map: Callable | None = None, **_: Any):
        self.block_shape = tuple(block_shape) if block_shape is not None else None
        self.index_map = index_map

    def __repr__(self) -> str:
        return f"BlockSpec({self.block_shape})"


def ds(start: Any, size: int, stride: int = 1) -> Slice:
    return Slice(start, int(size), int(stride))


dslice = ds


def program_id(axis: int) -> Tracer:
    (out,) = current_builder().add("program_id", [], [ShapedArray((), I32)], axis=int(axis))
    return out


def num_programs(axis: int) -> int:
    grid = getattr(_grid_state, "grid", None)
    if grid is None:
        raise TraceError("num_programs is only available while tracing a kernel")
    return int(grid[axis])


class _GridState:
    grid: tuple[int, ...] | None = None


_grid_state = _GridState()

# While `palladium_amd.trace` runs a plain function, pallas_calls append
# (call, args) here and return zero placeholders instead of running.
_recording = threading.local()


class Ref:
    """A kernel operand block; index it to load (`get`) or store (`swap`)."""

    def __init__(self, tracer: Tracer):
        self._t = tracer

    @property
    def shape(self) -> tuple[int, ...]:
        return self._t.shape

    @property
    def dtype(self) -> np.dtype:
        return self._t.dtype

    @property
    def ndim(self) -> int:
        return len(self.shape)

    def _indexer(self, idx: Any) -> tuple[IndexerTree, list[Any]]:
        shape = self.shape
        if idx is Ellipsis or (isinstance(idx, tuple) and idx == ()):
            idx = (Ellipsis,)
        if not isinstance(idx, tuple):
            idx = (idx,)
        # Expand a single Ellipsis into full slices.
        n_ell = sum(1 for i in idx if i is Ellipsis)
        if n_ell > 1:
            raise TraceError("only one Ellipsis allowed in a ref index")
        if n_ell:
            k = idx.index(Ellipsis)
            fill = len(shape) - (len(idx) - 1)
            idx = idx[:k] + (slice(None),) * fill + idx[k + 1 :]
        if len(idx) < len(shape):
            idx = idx + (slice(None),) * (len(shape) - len(idx))
        if len(idx) != len(shape):
            raise TraceError(f"too many indices for ref of shape {shape}")
        leaves: list[Any] = []
        out = []
        b = current_builder()
        for d, (i, n) in enumerate(zip(idx, shape)):
            if isinstance(i, slice):
                step = 1 if i.step is None else i.step
                if isinstance(step, Tracer) or int(step) < 1:
                    raise TraceError(f"ref access dim {d}: step {i.step} must be a positive int")
                step = int(step)
                start = 0 if i.start is None else i.start
                stop = n if i.stop is None else i.stop
                if isinstance(start, Tracer) or isinstance(stop, Tracer):
                    raise TraceError("dynamic Python slices are unsupported; use pl.ds(start, size)")
                start, stop = int(start), int(stop)
                start = start + n if start < 0 else start
                stop = stop + n if stop < 0 else builtins_min(stop, n)
                # a strided window stages as JAX's does; the emitter rejects it
                out.append(Slice(start, builtins_max(0, -(-(stop - start) // step)), step))
            elif isinstance(i, Slice):
                st = i.start
                if isinstance(st, Tracer):
                    leaves.append(_as_i32(st))
                    st = _Leaf(len(leaves) - 1)
                out.append(Slice(st, i.size, i.stride))
            else:
                if isinstance(i, Tracer):
                    if i.shape != ():
                        raise TraceError("ref indices must be scalars")
                    leaves.append(_as_i32(i))
                else:
                    v = int(i)
                    if v < 0:
                        v += n
                    leaves.append(literal(v, I32, weak=False))
                out.append(_Leaf(len(leaves) - 1))
        return IndexerTree(NDIndexer(tuple(out), tuple(shape)), len(leaves)), leaves

    def __getitem__(self, idx: Any) -> Tracer:
        tree, leaves = self._indexer(idx)
        shape = NDIndexer(tree.unflatten(leaves)[0].indices, self.shape).result_shape()
        (out,) = current_builder().add("get", [self._t, *leaves], [ShapedArray(shape, self.dtype)], tree=tree)
        return out

    def __setitem__(self, idx: Any, value: Any) -> None:
        tree, leaves = self._indexer(idx)
        shape = NDIndexer(tree.unflatten(leaves)[0].indices, self.shape).result_shape()
        if isinstance(value, Tracer):
            if value.dtype != self.dtype:
                if value.weak_type:
                    value = jnp.convert_element_type(value, self.dtype)
                else:
                    raise TraceError(
                        f"storing {_dtype_name(value.dtype)} into a {_dtype_name(self.dtype)} ref; cast explicitly"
                    )
            if value.shape != shape:
                if math.prod(value.shape) == math.prod(shape):
                    value = jnp.reshape(value, shape)
                else:
                    value = jnp.broadcast_to(value, shape)
        else:
            value = jnp.full(shape, value, self.dtype)
        current_builder().add("swap", [self._t, value, *leaves], [ShapedArray(shape, self.dtype)], tree=tree)


def _as_i32(t: Tracer) -> Tracer:
    return t if t.dtype == I32 else jnp.convert_element_type(t, I32)


def _normalize_shapes(out_shape: Any) -> tuple[list[ShapeDtypeStruct], bool]:
    if isinstance(out_shape, (list, tuple)):
        return [ShapeDtypeStruct(s.shape, s.dtype) for s in out_shape], True
    return [ShapeDtypeStruct(out_shape.shape, out_shape.dtype)], False


def block_dims(block_shape: tuple[Any, ...] | None, array_shape: tuple[int, ...]) -> list[int | None]:
    """Per-dim block size, None for squeezed dims."""
    if block_shape is None:
        return list(array_shape)
    if len(block_shape) != len(array_shape):
        raise TraceError(f"block shape {block_shape} does not match array rank {len(array_shape)}")
    dims: list[int | None] = []
    for d in block_shape:
        if d is None or isinstance(d, Squeezed):
            dims.append(None)
        elif isinstance(d, Blocked):
            dims.append(int(d.block_size))
        elif isinstance(d, (int, np.integer)):
            dims.append(int(d))
        else:
            raise TraceError(
                f"unsupported block dim type {type(d).__name__}: only int, "
                "pl.Blocked, and pl.Squeezed dims are lowered (pl.Element, "
                "pl.Indirect, and pl.BoundedSlice indexing is unimplemented)"
            )
    return dims


def trace_index_map(spec: BlockSpec | None, grid: tuple[int, ...], rank: int) -> ClosedJaxpr:
    """Stage a BlockSpec index map as a jaxpr over int32 grid indices."""
    b = Builder(None)
    with building(b):
        args = [b.arg(ShapedArray((), I32)) for _ in grid]
        if spec is None or spec.index_map is None:
            outs: Any = (0,) * rank
        else:
            outs = spec.index_map(*args)
        if not isinstance(outs, (tuple, list)):
            outs = (outs,)
        if len(outs) != rank:
            raise TraceError(f"index map returned {len(outs)} indices for a rank-{rank} array")
        atoms = []
        for o in outs:
            if isinstance(o, Tracer):
                atoms.append(b.atom(_as_i32(o)))
            else:
                atoms.append(literal(int(o), I32, weak=False))
    return ClosedJaxpr(Jaxpr([], b.invars, atoms, b.eqns), [])


class PallasCall:
    """The staged `pl.pallas_call`: kernel + launch geometry, no data."""

    def __init__(
        self,
        kernel: Callable,
        out_shape: Any,
        *,
        grid: Any = (),
        in_specs: Any = None,
        out_specs: Any = None,
        name: str | None = None,
        interpret: bool = False,
        **extra: Any,
    ):
        if extra.get("scratch_shapes"):
            raise TraceError("scratch_shapes are not supported yet")
        if "grid_spec" in extra and extra["grid_spec"] is not None:
            raise TraceError("PrefetchScalarGridSpec is not supported")
        self.kernel = kernel
        self.out_shapes, self.multiple_results = _normalize_shapes(out_shape)
        if isinstance(grid, (int, np.integer)):
            grid = (int(grid),)
        self.grid = tuple(int(g) for g in grid)
        self.in_specs = in_specs
        self.out_specs = out_specs
        self.name = name
        self.interpret = interpret

    def _spec_list(self, specs: Any, n: int, what: str) -> list[BlockSpec | None]:
        if specs is None:
            return [None] * n
        if isinstance(specs, BlockSpec):
            specs = [specs] if n == 1 else None
            if specs is None:
                raise TraceError(f"{what}: one BlockSpec given for {n} operands")
        specs = list(specs)
        if len(specs) != n:
            raise TraceError(f"{what}: {len(specs)} BlockSpecs for {n} operands")
        return specs

    def __call__(self, *args: Any) -> Any:
        calls = getattr(_recording, "calls", None)
        if calls is not None:
            calls.append((self, args))
            outs = tuple(np.zeros(s.shape, s.dtype) for s in self.out_shapes)
            return outs if self.multiple_results else outs[0]
        if self.interpret:
            from palladium_amd.interpret import interpret_call

            return interpret_call(self, *args)
        raise TraceError(
            "a staged pallas_call runs through palladium_amd.hip_call (GPU) "
            "or interpret=True (CPU interpreter)"
        )


def pallas_call(kernel: Callable, out_shape: Any = None, **kwargs: Any) -> PallasCall:
    if out_shape is None:
        raise TraceError("pallas_call needs out_shape")
    return PallasCall(kernel, out_shape, **kwargs)


def kernel_refs(builder: Builder, avals: list[RefAval]) -> list[Ref]:
    return [Ref(builder.arg(a)) for a in avals]


def check_operand_dtype(dtype: Any) -> np.dtype:
    return check_dtype(dtype)
