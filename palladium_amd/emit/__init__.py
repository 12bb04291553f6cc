"""jaxpr -> HIP C++ emission for gfx950 (one program instance per lane)."""

from palladium_amd.emit import rules as _rules  # noqa: F401  (registers RULES)
from palladium_amd.emit.core import (
    RULES,
    Cursor,
    CVal,
    EmitError,
    Environment,
    LaunchGeometry,
    declare,
    emit_hip,
    emit_jaxpr,
    launch_geometry,
    rule,
)
from palladium_amd.emit.rules import ELEMENTWISE

__all__ = [
    "ELEMENTWISE",
    "RULES",
    "CVal",
    "Cursor",
    "EmitError",
    "Environment",
    "LaunchGeometry",
    "declare",
    "emit_hip",
    "emit_jaxpr",
    "launch_geometry",
    "rule",
]
