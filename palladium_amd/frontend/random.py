"""`jax.random`-shaped counter-based RNG for kernels (Threefry-2x32-20).

In-kernel calls stage the primitives JAX stages
(`random_wrap`, `random_unwrap`, `random_bits`, `random_fold_in`), and
`uniform` stages JAX's exact float conversion sequence
(`src/palladium/emit/rules.py:106-201`; `tests/test_10_random_bits.py:42-54`).
`threefry2x32_p` exposes the raw `threefry2x32` primitive, one hash of a
`(k0, k1)` key over a `(x0, x1)` counter, which is how a kernel states
"counter = (path, step)" with a single hash per draw.

Host-side helpers (`key`, `PRNGKey`, `key_data`) return the uint32 key
data JAX produces for a 32-bit seed: `(0, seed)`.
"""

from __future__ import annotations

from typing import Any, Sequence

import numpy as np

from palladium_amd.errors import TraceError
from palladium_amd.frontend import jnp
from palladium_amd.frontend.core import F32, U32, Tracer, current_builder, literal
from palladium_amd.ir import KeyAval, ShapedArray


def key(seed: int) -> np.ndarray:
    """Host-side: uint32 key data of `jax.random.key(seed)`, `(hi, lo)`."""
    seed = int(seed)
    return np.array([(seed >> 32) & 0xFFFFFFFF, seed & 0xFFFFFFFF], dtype=np.uint32)


PRNGKey = key


def wrap_key_data(data: Tracer, impl: str = "threefry2x32") -> Tracer:
    if impl not in ("threefry2x32", "threefry"):
        raise TraceError(f"only the threefry2x32 PRNG impl is supported, got {impl!r}")
    if not isinstance(data, Tracer) or data.shape != (2,) or data.dtype != U32:
        raise TraceError("wrap_key_data expects a uint32[2] key-data value")
    (k,) = current_builder().add("random_wrap", [data], [KeyAval(())], impl="threefry2x32")
    return k


def key_data(k: Any) -> Any:
    if isinstance(k, np.ndarray):
        return k
    if not (isinstance(k, Tracer) and isinstance(k.aval, KeyAval)):
        raise TraceError("key_data expects a PRNG key")
    (d,) = current_builder().add("random_unwrap", [k], [ShapedArray((2,), U32)])
    return d


def _as_key(k: Any) -> Tracer:
    if isinstance(k, Tracer) and isinstance(k.aval, KeyAval):
        return k
    if isinstance(k, Tracer) and k.shape == (2,) and k.dtype == U32:
        return wrap_key_data(k)
    raise TraceError("expected a PRNG key (wrap uint32[2] key data with wrap_key_data)")


def fold_in(k: Any, data: Any) -> Tracer:
    """A fresh key from `(key, data)`: threefry(key, (0, data))."""
    k = _as_key(k)
    if isinstance(data, Tracer):
        d = data if data.dtype == U32 else jnp.convert_element_type(data, U32)
        if d.shape not in ((), (1,)):
            raise TraceError("fold_in data must be a scalar")
    else:
        d = literal(int(data) & 0xFFFFFFFF, U32, weak=False)
    (out,) = current_builder().add("random_fold_in", [k, d], [KeyAval(())])
    return out


def bits(k: Any, shape: Sequence[int] = (), dtype: Any = np.uint32) -> Tracer:
    """uint32 bits; element i hashes counter (0, i) and returns x0 ^ x1."""
    if np.dtype(dtype) != U32:
        raise TraceError("random bits: only bit_width=32 (uint32) is implemented")
    k = _as_key(k)
    shape = tuple(int(s) for s in shape)
    (out,) = current_builder().add("random_bits", [k], [ShapedArray(shape, U32)], bit_width=32, shape=shape)
    return out


def uniform(k: Any, shape: Sequence[int] = (), dtype: Any = np.float32, minval: float = 0.0, maxval: float = 1.0) -> Tracer:
    """JAX's float conversion: mantissa bits under exponent 0 give a float
    in [1, 2); subtract 1, scale, shift, then clamp below by minval."""
    if np.dtype(dtype) != F32:
        raise TraceError("uniform: only float32 is supported")
    return bits_to_uniform(bits(k, shape), minval, maxval)


def bits_to_uniform(b: Tracer, minval: float = 0.0, maxval: float = 1.0) -> Tracer:
    """JAX's uint32 -> float32 uniform conversion, staged op for op."""
    shifted = jnp.right_shift(b, np.uint32(9))
    fb = jnp.bitwise_or(shifted, np.uint32(0x3F800000))
    floats = jnp.bitcast_convert_type(fb, F32) - np.float32(1.0)
    scaled = floats * np.float32(maxval - minval) + np.float32(minval)
    return jnp.maximum(np.float32(minval), scaled)


def normal(k: Any, shape: Sequence[int] = (), dtype: Any = np.float32) -> Tracer:
    raise TraceError("random.normal is not lowered; build it from uniform (Box-Muller)")


def threefry2x32_p(k0: Any, k1: Any, x0: Any, x1: Any) -> tuple[Tracer, Tracer]:
    """Raw Threefry-2x32-20 block: hash counter (x0, x1) under key (k0, k1)."""
    ops = [jnp.convert_element_type(v, U32) if isinstance(v, Tracer) else v for v in (k0, k1, x0, x1)]
    if not any(isinstance(v, Tracer) for v in ops):
        raise TraceError("threefry2x32_p needs at least one traced operand")
    shape = jnp._broadcast_shapes(*[jnp._shape_of(v) for v in ops])
    ins = [jnp._as_operand(v, U32, shape) for v in ops]
    outs = current_builder().add("threefry2x32", ins, [ShapedArray(shape, U32), ShapedArray(shape, U32)])
    return outs[0], outs[1]
