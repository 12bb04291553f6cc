"""Step 1 of the pipeline: a pallas_call to a KernelSpec.

Same contract as the reference tracer (`src/palladium/trace.py:26-177`):
a KernelSpec carries the kernel jaxpr over Refs, the grid (`(1,)` when
gridless), and per-operand BlockInfo (kernel-visible block shape,
full array shape, dtype, index-map jaxpr in units of blocks).

Two sources are accepted:
- a `palladium_amd.frontend.pl.PallasCall` (the JAX-free frontend);
- with JAX importable, any callable that invokes exactly one
  `jax.experimental.pallas.pallas_call` (see `palladium_amd.jax_adapter`).
"""

from __future__ import annotations

import dataclasses
import math
from typing import Any, Callable

import numpy as np

from palladium_amd.errors import TraceError
from palladium_amd.frontend import pl as _pl
from palladium_amd.frontend.core import Builder, building, check_dtype
from palladium_amd.ir import ClosedJaxpr, Jaxpr, RefAval

__all__ = ["BlockInfo", "KernelSpec", "trace"]


@dataclasses.dataclass(frozen=True)
class BlockInfo:
    """How one operand of the kernel is cut into per-instance pieces.

    block_shape: the shape a kernel body indexes, with the dimensions the
    BlockSpec marks as squeezed left out. array_shape: the whole operand in
    HBM. dtype: the element type (block and array agree). index_map_jaxpr:
    the BlockSpec's index map as a closed jaxpr, taking the grid indices to
    a block index (multiply by the block shape for an element offset).
    full_block_shape: block_shape at the array's rank, squeezed dimensions
    restored as size 1 (None means: derive it by left-padding with 1s).
    """

    block_shape: tuple[int, ...]
    array_shape: tuple[int, ...]
    dtype: np.dtype
    index_map_jaxpr: ClosedJaxpr
    full_block_shape: tuple[int, ...] | None = None

    def full_block(self) -> tuple[int, ...]:
        if self.full_block_shape is not None:
            return self.full_block_shape
        missing = len(self.array_shape) - len(self.block_shape)
        return (1,) * missing + tuple(self.block_shape)


@dataclasses.dataclass(frozen=True)
class KernelSpec:
    """A traced pallas_call, ready for the emitter.

    name: the entry-point symbol of the emitted HIP kernel. jaxpr: the
    kernel body, a stateful jaxpr whose parameters are Refs, the inputs
    first and then the outputs. grid: the program-instance grid (a gridless
    call has grid (1,)). inputs / outputs: one BlockInfo per operand, in the
    jaxpr's parameter order. raw_params: whatever else the pallas_call was
    given, kept as passed.
    """

    name: str
    jaxpr: Jaxpr
    grid: tuple[int, ...]
    inputs: tuple[BlockInfo, ...]
    outputs: tuple[BlockInfo, ...]
    raw_params: dict[str, Any]

    @property
    def num_programs(self) -> int:
        """Total number of program instances (one GPU thread each)."""
        return math.prod(self.grid)


def _shape_dtype(a: Any) -> tuple[tuple[int, ...], np.dtype]:
    shape = tuple(int(s) for s in getattr(a, "shape", np.shape(a)))
    dtype = getattr(a, "dtype", None)
    if dtype is None:
        dtype = np.asarray(a).dtype
    return shape, np.dtype(dtype)


def _trace_frontend(call: "_pl.PallasCall", example_args: tuple) -> KernelSpec:
    grid = call.grid or (1,)
    in_sd = [_shape_dtype(a) for a in example_args]
    for i, (_, dt) in enumerate(in_sd):
        try:
            check_dtype(dt)
        except TraceError as e:
            raise TraceError(f"argument {i}: {e}") from None
    out_sd = [(s.shape, s.dtype) for s in call.out_shapes]
    in_specs = call._spec_list(call.in_specs, len(in_sd), "in_specs")
    out_specs = call._spec_list(call.out_specs, len(out_sd), "out_specs")

    def infos(specs, sds) -> tuple[BlockInfo, ...]:
        out = []
        for spec, (shape, dtype) in zip(specs, sds):
            dims = _pl.block_dims(spec.block_shape if spec is not None else None, shape)
            block = tuple(d for d in dims if d is not None)
            full = tuple(1 if d is None else d for d in dims)
            imj = _pl.trace_index_map(spec, grid if call.grid else (), len(shape))
            out.append(BlockInfo(block, shape, dtype, imj, full))
        return tuple(out)

    inputs = infos(in_specs, in_sd)
    outputs = infos(out_specs, out_sd)
    b = Builder(None)
    prev = _pl._grid_state.grid
    _pl._grid_state.grid = grid
    try:
        with building(b):
            refs = _pl.kernel_refs(b, [RefAval(i.block_shape, i.dtype) for i in (*inputs, *outputs)])
            call.kernel(*refs)
    finally:
        _pl._grid_state.grid = prev
    jaxpr = Jaxpr([], b.invars, [], b.eqns)
    name = call.name or getattr(call.kernel, "__name__", None) or "palladium_kernel"
    if not name.isidentifier() or name == "<lambda>":
        name = "palladium_kernel"
    return KernelSpec(
        name=name,
        jaxpr=jaxpr,
        grid=tuple(grid),
        inputs=inputs,
        outputs=outputs,
        raw_params={"grid": call.grid},
    )


def _trace_function(fn: Callable, example_args: tuple) -> KernelSpec:
    """Run `fn` with every frontend pallas_call recorded instead of run
    (placeholders flow on to later code); exactly one must be found
    (reference: `src/palladium/trace.py:118-150`)."""
    args = [np.zeros(*_shape_dtype(a)) for a in example_args]
    _pl._recording.calls = []
    try:
        fn(*args)
        calls = _pl._recording.calls
    finally:
        _pl._recording.calls = None
    if len(calls) != 1:
        raise TraceError(
            f"found {len(calls)} pallas_call(s) in {getattr(fn, '__name__', 'the function')}; "
            "palladium_amd compiles exactly one pallas_call per trace"
            + ("" if calls else " (pass palladium_amd.frontend.pl.pallas_call(...))")
        )
    call, call_args = calls[0]
    return _trace_frontend(call, call_args)


def trace(pallas_fn: Callable, *example_args: Any) -> KernelSpec:
    """Extract a KernelSpec from a staged pallas_call.

    Parameters
    ----------
    pallas_fn : PallasCall or callable
        `palladium_amd.frontend.pl.pallas_call(...)`, or (with JAX
        importable) any function invoking exactly one JAX pallas_call.
    *example_args
        Arrays or ShapeDtypeStructs fixing shapes and dtypes; no data is read.

    Raises
    ------
    TraceError
        Zero or several pallas_calls, scalar prefetch, unsupported block
        dims or dtypes.
    """
    if isinstance(pallas_fn, _pl.PallasCall):
        return _trace_frontend(pallas_fn, example_args)
    try:
        import jax  # noqa: F401
    except ImportError:
        return _trace_function(pallas_fn, example_args)
    from palladium_amd.jax_adapter import trace_jax

    return trace_jax(pallas_fn, *example_args)
