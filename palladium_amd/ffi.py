"""jax.ffi bridge: palladium_amd kernels as a jax.jit-composable primitive.

Mirrors the reference's `FfiCallable`/`metal_call_jit`
(`src/palladium/ffi.py:90-221`): trace and emit are cached per input
shape, and `jax.ffi.ffi_call` dispatches to the native target
`palladium_hip_dispatch` with the source, entry point name, grid, block and
math mode as attributes. The handler (`csrc/xla_ffi_handler.cc`) is a thin
shim over the C ABI's `ph_dispatch`; it is built only where the XLA FFI
headers exist (`jax.ffi.include_dir()`), as `libpalladium_hip_ffi.so`.

Only the sequential `vmap_method`s are accepted: the grid is baked per
unbatched shape, so whole-batch methods would dispatch it over batched
buffers (`src/palladium/ffi.py:82-87,118-125`).
"""

from __future__ import annotations

import ctypes
import functools
import os
import threading
from collections.abc import Callable
from pathlib import Path
from typing import Any

from palladium_amd.dtypes import name as _dtype_name

from palladium_amd.diagnostics import KernelDiagnostics, explain_spec, log_compile
from palladium_amd.emit import emit_hip, launch_geometry
from palladium_amd.runtime import REPRODUCIBLE_ORDINAL, MathMode, math_mode_ordinal
from palladium_amd.trace import KernelSpec, trace

__all__ = ["FfiCallable", "hip_call_jit"]

_TARGET_NAME = "palladium_hip_dispatch"
_LIBRARY_NAME = "libpalladium_hip_ffi.so"
_SAFE_VMAP_METHODS = (None, "sequential", "sequential_unrolled")

_REGISTER_LOCK = threading.Lock()
_registered = False


def _library_path() -> Path:
    override = os.environ.get("PALLADIUM_FFI_LIBRARY")
    if override:
        return Path(override)
    p = Path(__file__).resolve().parent / _LIBRARY_NAME
    if not p.is_file():
        raise FileNotFoundError(
            f"palladium_amd's jax.ffi handler ({_LIBRARY_NAME}) isn't built; run "
            "`python -m palladium_amd.build --ffi` on a machine with jax installed, "
            "or set PALLADIUM_FFI_LIBRARY"
        )
    return p


def _register() -> None:
    """Load the handler and register it once per process (locked)."""
    global _registered
    if _registered:
        return
    with _REGISTER_LOCK:
        if _registered:
            return
        import jax

        handle = ctypes.CDLL(str(_library_path()))
        capsule = jax.ffi.pycapsule(handle.palladium_hip_dispatch)
        jax.ffi.register_ffi_target(_TARGET_NAME, capsule, platform="cpu")
        # jax on ROCm: arrays already live in HBM, so the same target name
        # resolves to the device-buffer handler on XLA's own stream.
        if any(d.platform == "rocm" for d in jax.devices()):
            rocm = jax.ffi.pycapsule(handle.palladium_hip_dispatch_rocm)
            jax.ffi.register_ffi_target(_TARGET_NAME, rocm, platform="ROCM")
        _registered = True


class FfiCallable:
    """A palladium_amd kernel registered as a jax.ffi target.

    Attributes
    ----------
    interpret : callable
        The same pallas_call with `interpret=True` (under REPRODUCIBLE math,
        in that mode's arithmetic, as `HipCallable.interpret`).
    """

    def __init__(self, kernel: Callable, pallas_kwargs: dict[str, Any], math_mode: Any,
                 vmap_method: str | None = None, threadgroup: Any = None) -> None:
        if vmap_method not in _SAFE_VMAP_METHODS:
            raise ValueError(
                f"vmap_method {vmap_method!r} is not supported: the launch grid is "
                "baked per unbatched shape, so whole-batch methods would dispatch it "
                "over batched buffers. Use 'sequential' or 'sequential_unrolled' (one "
                "dispatch per batch element), or put the batch dimension in the Pallas "
                "grid instead."
            )
        from palladium_amd import _stage, _use_jax

        self._staged, self.interpret = _stage(kernel, pallas_kwargs, "auto")
        self._math_mode = math_mode_ordinal(math_mode)
        if self._math_mode == REPRODUCIBLE_ORDINAL and not _use_jax("auto"):
            # the interpreter in this mode's arithmetic, as HipCallable's
            from palladium_amd.interpret import interpret_call

            self.interpret = functools.partial(interpret_call, self._staged, math_mode=self._math_mode)
        self._vmap_method = vmap_method
        self._threadgroup = threadgroup
        self._cache: dict[tuple, tuple[KernelSpec, str]] = {}
        self._lock = threading.Lock()

    def explain(self, *args: Any, compile: bool = True) -> KernelDiagnostics:
        return explain_spec(trace(self._staged, *args), self._threadgroup, self._math_mode, compile=compile)

    def spec_and_source(self, args: tuple) -> tuple[KernelSpec, str]:
        key = tuple((tuple(a.shape), _dtype_name(a.dtype)) for a in args)
        entry = self._cache.get(key)
        if entry is None:
            with self._lock:
                entry = self._cache.get(key)
                if entry is None:
                    from palladium_amd.dispatch import _block_of, _tile_of

                    from palladium_amd.interpret import check_block_bounds

                    spec = trace(self._staged, *args)
                    check_block_bounds(spec)
                    log_compile(spec, self._threadgroup, self._math_mode)
                    entry = (spec, emit_hip(spec, block=_block_of(self._threadgroup), math_mode=self._math_mode,
                                     tile=_tile_of(self._threadgroup)))
                    self._cache[key] = entry
        return entry

    def ffi_attributes(self, args: tuple) -> dict[str, Any]:
        """The attribute dict handed to the native handler for these shapes."""
        from palladium_amd.dispatch import _block_of

        spec, src = self.spec_and_source(args)
        geo = launch_geometry(spec, _block_of(self._threadgroup))
        grid = tuple(spec.grid) + (1, 1, 1)
        if len(spec.grid) > 3:
            grid = (spec.num_programs, 1, 1)
        return dict(
            hip_source=src,
            function_name=spec.name,
            grid_x=int(grid[0]),
            grid_y=int(grid[1]),
            grid_z=int(grid[2]),
            block_x=int(geo.block),
            lanes=int(geo.lanes),
            math_mode=int(self._math_mode),
        )

    def __call__(self, *args: Any) -> Any:
        try:
            import jax
        except ImportError as e:
            raise ImportError(
                "hip_call_jit dispatches through jax.ffi and needs jax installed; "
                "without jax, use palladium_amd.hip_call (same kernel, NumPy in/out)"
            ) from e

        _register()
        spec, _ = self.spec_and_source(args)
        attrs = self.ffi_attributes(args)
        outs = [jax.ShapeDtypeStruct(i.array_shape, i.dtype) for i in spec.outputs]
        result_shapes = outs[0] if len(outs) == 1 else outs
        return jax.ffi.ffi_call(_TARGET_NAME, result_shapes, vmap_method=self._vmap_method)(*args, **attrs)


def hip_call_jit(kernel: Callable, **pallas_kwargs: Any) -> FfiCallable:
    """`pl.pallas_call` dispatched to the MI355X, composable with `jax.jit`.

    Extra keywords: `math_mode` (FAST default), `vmap_method`
    ('sequential' / 'sequential_unrolled'; None rejects `jax.vmap`),
    `threadgroup`.
    """
    math_mode = pallas_kwargs.pop("math_mode", MathMode.FAST)
    vmap_method = pallas_kwargs.pop("vmap_method", None)
    threadgroup = pallas_kwargs.pop("threadgroup", None)
    return FfiCallable(kernel, pallas_kwargs, math_mode, vmap_method, threadgroup)
