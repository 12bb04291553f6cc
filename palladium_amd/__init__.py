"""palladium_amd: Pallas kernels on AMD Instinct MI355X (gfx950) via HIP.

Pipeline: trace (Pallas -> KernelSpec) -> emit (KernelSpec -> HIP C++)
-> bind (hiprtc -> callable on a HIP stream). `hip_call` composes the
three behind a `pl.pallas_call`-shaped entry point, as the reference's
`metal_call` does (`src/palladium/__init__.py:83-226`); `debug_hip`
exposes the intermediate text; `hip_call_jit` dispatches inside `jax.jit`
through the C-ABI handler.

Kernels are written against `palladium_amd.frontend` (`pl`, `lax`, `jnp`,
`random`: the JAX-free Pallas frontend) or, where JAX is importable,
against `jax.experimental.pallas` itself.
"""

from __future__ import annotations

import functools
import threading
from collections.abc import Callable
from typing import Any

import numpy as np

from palladium_amd import runtime
from palladium_amd.diagnostics import KernelDiagnostics, explain_spec, log_compile
from palladium_amd.dispatch import BoundKernel, PendingResult, bind
from palladium_amd.emit import emit_hip, emit_jaxpr, rule
from palladium_amd.dtypes import name as _dtype_name
from palladium_amd.emit.core import CTYPES as _CTYPES
from palladium_amd.errors import (
    CompileError,
    DispatchError,
    EmitError,
    PalladiumError,
    TraceError,
    UnsupportedPrimitiveError,
)
from palladium_amd.ffi import FfiCallable, hip_call_jit
from palladium_amd.interpret import check_block_bounds, interpret_call
from palladium_amd.runtime import MathMode
from palladium_amd.trace import BlockInfo, KernelSpec, trace

__all__ = [
    "BlockInfo",
    "BoundKernel",
    "CompileError",
    "DispatchError",
    "EmitError",
    "FfiCallable",
    "HipCallable",
    "KernelDiagnostics",
    "KernelSpec",
    "MathMode",
    "PalladiumError",
    "PendingResult",
    "TraceError",
    "UnsupportedPrimitiveError",
    "bind",
    "debug_hip",
    "emit_hip",
    "emit_jaxpr",
    "hip_call",
    "hip_call_jit",
    "rule",
    "trace",
]

__version__ = "0.1.0"

CacheKey = tuple[tuple[tuple[int, ...], str], ...]


def _check_dtypes(args: tuple) -> None:
    """Reject unsupported element types before tracing, with the fix in
    the message (reference: `src/palladium/__init__.py:58-80`)."""
    for i, a in enumerate(args):
        dtype = getattr(a, "dtype", None)
        name = _dtype_name(dtype if dtype is not None else np.asarray(a).dtype)
        if name not in _CTYPES:
            hint = (
                "; float64 usually means jax_enable_x64 is on, disable it or cast to float32"
                if name == "float64"
                else ""
            )
            raise DispatchError(
                f"argument {i} has dtype {name}, which palladium cannot lower "
                f"(supported: {', '.join(_CTYPES)}){hint}"
            )


def _use_jax(frontend: str) -> bool:
    if frontend == "palladium":
        return False
    if frontend == "jax":
        return True
    try:
        import jax.experimental.pallas  # noqa: F401
    except ImportError:
        return False
    return True


def _stage(kernel: Callable, pallas_kwargs: dict[str, Any], frontend: str) -> tuple[Any, Any]:
    if _use_jax(frontend):
        import jax.experimental.pallas as jpl

        return jpl.pallas_call(kernel, **pallas_kwargs), jpl.pallas_call(kernel, **pallas_kwargs, interpret=True)
    from palladium_amd.frontend import pl

    return pl.pallas_call(kernel, **pallas_kwargs), pl.pallas_call(kernel, **pallas_kwargs, interpret=True)


class HipCallable:
    """The palladium_amd pipeline behind a `pl.pallas_call`-shaped call.

    Retraces per input shape/dtype; identical shapes hit `cache`.

    Attributes
    ----------
    interpret : callable
        The same pallas_call with `interpret=True`: the CPU interpreter (IEEE
        order; under REPRODUCIBLE math, that mode's fused multiply-adds,
        division and power, so it reproduces the device bit for bit).
    cache : dict
        Input-shape signature -> compiled `BoundKernel`
        (`cache[key].hip_source` is the emitted text).
    """

    def __init__(self, kernel: Callable, pallas_kwargs: dict[str, Any], math_mode: Any,
                 threadgroup: int | tuple[int, ...] | None, frontend: str = "auto") -> None:
        self._staged, self.interpret = _stage(kernel, pallas_kwargs, frontend)
        self._math_mode = MathMode(runtime._mode_value(math_mode))
        if self._math_mode == MathMode.REPRODUCIBLE and not _use_jax(frontend):
            # the interpreter in this mode's arithmetic: device results bit for bit
            self.interpret = functools.partial(interpret_call, self._staged, math_mode=self._math_mode)
        self._threadgroup = threadgroup
        self.cache: dict[CacheKey, BoundKernel] = {}
        # Guards trace/emit/compile on a miss: concurrent first calls on
        # the same shape compile exactly once.
        self._lock = threading.Lock()

    @property
    def math_mode(self) -> MathMode:
        return self._math_mode

    def explain(self, *args: Any, compile: bool = True) -> KernelDiagnostics:
        """Launch geometry, emitted size and (compiled without a GPU)
        register/LDS/scratch use for these input shapes. Dispatches nothing."""
        _check_dtypes(args)
        return explain_spec(trace(self._staged, *args), self._threadgroup, self._math_mode, compile=compile)

    def bound(self, *args: Any) -> BoundKernel:
        """The compiled kernel for these input shapes (compiling on a miss)."""
        args = tuple(a if hasattr(a, "shape") and hasattr(a, "dtype") else np.asarray(a) for a in args)
        key: CacheKey = tuple((tuple(a.shape), np.dtype(a.dtype).str) for a in args)
        b = self.cache.get(key)
        if b is None:
            with self._lock:
                b = self.cache.get(key)
                if b is None:
                    _check_dtypes(tuple(args))
                    spec = trace(self._staged, *args)
                    check_block_bounds(spec)
                    log_compile(spec, self._threadgroup, self._math_mode)
                    from palladium_amd.dispatch import _block_of, _tile_of

                    b = bind(spec, emit_hip(spec, block=_block_of(self._threadgroup), math_mode=self._math_mode,
                                     tile=_tile_of(self._threadgroup)),
                             math_mode=self._math_mode, threadgroup=self._threadgroup)
                    self.cache[key] = b
        return b

    def pin(self, *args: Any) -> Callable[[], np.ndarray | tuple[np.ndarray, ...]]:
        """Upload inputs once; return a zero-argument re-dispatch callable."""
        arrays = [np.asarray(a) for a in args]
        return self.bound(*arrays).pinned(*arrays)

    def launch(self, *args: Any) -> PendingResult:
        arrays = [np.asarray(a) for a in args]
        return self.bound(*arrays).launch(*arrays)

    def __call__(self, *args: Any) -> np.ndarray | tuple[np.ndarray, ...]:
        """Run the kernel on the GPU; NumPy in, NumPy out."""
        arrays = [np.asarray(a) for a in args]
        return self.bound(*arrays)(*arrays)


def debug_hip(kernel: Callable, *example_args: Any, **pallas_kwargs: Any) -> str:
    """Trace `kernel` through pallas_call and return the emitted HIP source,
    exactly as `hip_call` with the same keywords would compile it (FAST
    math, the default, applies its jaxpr rewrites before emission).
    Nothing is compiled or dispatched."""
    threadgroup = pallas_kwargs.pop("threadgroup", None)
    math_mode = pallas_kwargs.pop("math_mode", MathMode.FAST)
    frontend = pallas_kwargs.pop("frontend", "auto")
    staged, _ = _stage(kernel, pallas_kwargs, frontend)
    from palladium_amd.dispatch import _block_of, _tile_of

    return emit_hip(trace(staged, *example_args), block=_block_of(threadgroup), math_mode=math_mode,
                    tile=_tile_of(threadgroup))


def hip_call(kernel: Callable, **pallas_kwargs: Any) -> HipCallable:
    """`pl.pallas_call`, but the kernel runs on the MI355X.

    Parameters
    ----------
    kernel : callable
        A Pallas kernel function (operates on Refs).
    **pallas_kwargs
        The usual `pl.pallas_call` keywords (out_shape, grid, in_specs,
        out_specs, name), plus `math_mode` (MathMode, FAST by default),
        `threadgroup` (workgroup lanes, a multiple of 64; default 256) and
        `frontend` ("auto", "palladium" or "jax").

    Notes
    -----
    FAST math contracts and reassociates float arithmetic, so results are
    not bit-equal to the CPU interpreter; use SAFE for IEEE op order (and
    for compensated arithmetic).
    """
    math_mode = pallas_kwargs.pop("math_mode", MathMode.FAST)
    threadgroup = pallas_kwargs.pop("threadgroup", None)
    frontend = pallas_kwargs.pop("frontend", "auto")
    return HipCallable(kernel, pallas_kwargs, math_mode, threadgroup, frontend)
