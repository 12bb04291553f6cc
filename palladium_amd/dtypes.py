"""bfloat16 on the host, with or without `ml_dtypes`.

The reference accepts `ml_dtypes.bfloat16` arrays on its eager path and
ships their bytes as uint16 (`src/palladium/dispatch.py:47-61`,
`src/palladium/__init__.py:59-66`). Here:

- `bfloat16` is `np.dtype(ml_dtypes.bfloat16)` when ml_dtypes is
  importable (it is wherever JAX is), so arrays a JAX user already holds
  pass straight through;
- otherwise it is a 2-byte structured dtype with one field named
  "bfloat16". NumPy refuses arithmetic on it (no silent uint16 math), its
  bytes are the bf16 bit patterns, and `from_float` / `to_float` convert.

Kernel semantics for bf16 values (device and interpreter alike): every
operation is evaluated in float32 and its result rounded to bf16, round to
nearest even. For + - * / and sqrt this equals the correctly rounded bf16
result (float32 carries more than 2*8+2 significand bits, so the double
rounding is innocuous).
"""

from __future__ import annotations

from typing import Any

import numpy as np

__all__ = ["bfloat16", "bfloat16_type", "from_float", "is_bf16", "kind", "name", "round_f32", "to_float"]

try:  # pragma: no cover - depends on the environment
    import ml_dtypes as _ml

    bfloat16 = np.dtype(_ml.bfloat16)
    bfloat16_type: Any = _ml.bfloat16
    HAVE_ML_DTYPES = True
except ImportError:
    bfloat16 = np.dtype([("bfloat16", "<u2")])
    HAVE_ML_DTYPES = False

    class bfloat16_type:  # noqa: N801 - mirrors ml_dtypes.bfloat16
        """Scalar constructor and dtype specifier for the surrogate:
        `bfloat16_type(1.5)` is a 0-d bfloat16 array, and
        `np.dtype(bfloat16_type)` is the surrogate dtype."""

        dtype = bfloat16

        def __new__(cls, value: Any = 0.0) -> np.ndarray:  # type: ignore[misc]
            return from_float(scalar_f32(value)).reshape(())


def is_bf16(dt: Any) -> bool:
    try:
        d = np.dtype(dt)
    except TypeError:
        return False
    return d == bfloat16 or d.name == "bfloat16"


def name(dt: Any) -> str:
    """The dtype's name, with the surrogate reporting "bfloat16"."""
    return "bfloat16" if is_bf16(dt) else np.dtype(dt).name


def kind(dt: Any) -> str:
    """NumPy kind code, with bfloat16 reported as a float ("f")."""
    return "f" if is_bf16(dt) else np.dtype(dt).kind


def round_f32(x: Any) -> np.ndarray:
    """float32 values rounded to the nearest bfloat16 (ties to even),
    returned as float32. NaNs stay NaN (quieted); infinities and signed
    zeros are kept."""
    f = np.ascontiguousarray(np.asarray(x, np.float32))
    u = f.view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    with np.errstate(over="ignore"):
        r = (u + np.uint32(0x7FFF) + lsb) & np.uint32(0xFFFF0000)
    nan = np.isnan(f)
    if nan.any():
        r = np.where(nan, (u & np.uint32(0xFFFF0000)) | np.uint32(0x00400000), r)
    return np.asarray(r, np.uint32).view(np.float32).reshape(f.shape)


def scalar_f32(value: Any) -> float:
    """A Python scalar, NumPy scalar or 0-d array (bfloat16 included) as
    its float value rounded to bfloat16."""
    a = np.asarray(value)
    if is_bf16(a.dtype):
        return float(to_float(a).reshape(()))
    return float(round_f32(np.float32(a.astype(np.float64)) if a.dtype.kind != "f" else a.astype(np.float32)).reshape(()))


def bits_from_f32(x: Any) -> np.ndarray:
    """uint16 bit patterns of `x` rounded to bfloat16."""
    return (round_f32(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def f32_from_bits(bits: Any) -> np.ndarray:
    """Exact float32 values of bfloat16 bit patterns."""
    b = np.asarray(bits, np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def from_float(x: Any) -> np.ndarray:
    """An array of dtype `bfloat16` holding `x` rounded to bf16."""
    return bits_from_f32(x).view(bfloat16)


def to_float(a: np.ndarray) -> np.ndarray:
    """float32 copy of a bfloat16 array (exact)."""
    a = np.ascontiguousarray(a)
    if not is_bf16(a.dtype):
        raise TypeError(f"expected a bfloat16 array, got {a.dtype}")
    return f32_from_bits(a.view(np.uint16))


def as_bits(a: np.ndarray) -> np.ndarray:
    """The uint16 bit patterns of a bfloat16 array (a view when contiguous)."""
    return np.ascontiguousarray(a).view(np.uint16)
