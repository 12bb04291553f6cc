"""Exception hierarchy: everything palladium_amd raises derives from
PalladiumError, split by pipeline stage (trace, emit, compile, dispatch).

Mirrors the reference taxonomy (`src/palladium/errors.py:19-44`):
TraceError doubles as ValueError and DispatchError as TypeError, so call
sites written against the reference keep their `except` clauses.
CompileError is this backend's analogue of metal-runtime's CompileError
(raised by hiprtc failures, with the numbered source attached).
"""

from __future__ import annotations

__all__ = [
    "CompileError",
    "DispatchError",
    "EmitError",
    "PalladiumError",
    "TraceError",
    "UnsupportedPrimitiveError",
]


class PalladiumError(Exception):
    """Base class for all palladium_amd errors."""


class TraceError(PalladiumError, ValueError):
    """The pallas_call cannot be traced into a KernelSpec (zero or several
    pallas_calls, scalar prefetch, unknown block dim types)."""


class EmitError(PalladiumError):
    """The emitter cannot lower this kernel (unsupported shapes, dtypes,
    primitive parameters or memory layout)."""


class UnsupportedPrimitiveError(EmitError, NotImplementedError):
    """The kernel stages a primitive with no registered lowering rule.
    Extensible via `palladium_amd.rule`."""


class DispatchError(PalladiumError, TypeError):
    """A compiled kernel was called with arguments that do not match its
    traced spec (wrong count, shape, or dtype)."""


class CompileError(PalladiumError, RuntimeError):
    """hiprtc rejected the emitted HIP source, or the code object could
    not be loaded on the device."""
