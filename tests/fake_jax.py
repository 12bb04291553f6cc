"""A stand-in for the few `jax` entry points palladium_amd.ffi uses
(`jax.ffi.ffi_call/pycapsule/register_ffi_target`, `jax.ShapeDtypeStruct`,
`jax.devices`), for testing `hip_call_jit` where JAX is not installed.

`ffi_call(target, result_shapes)(*args, **attrs)` does what the C++
handler in palladium_amd/csrc/xla_ffi_handler.cc does with XLA's buffers:
it hands the attributes, in the handler's order, and the input/output
buffers to the C ABI's `ph_dispatch`. Everything above that call (attribute
construction, result shapes, the per-shape cache, the vmap guard) is the
real palladium_amd.ffi code path.
"""

from __future__ import annotations

import ctypes
import types

import numpy as np

_HANDLER_ATTRS = ("grid_x", "grid_y", "grid_z", "block_x", "lanes", "math_mode")


class ShapeDtypeStruct:
    def __init__(self, shape, dtype):
        self.shape = tuple(shape)
        self.dtype = np.dtype(dtype)


def _dispatch(args, outs, attrs):
    from palladium_amd import runtime as rt

    src = attrs["hip_source"].encode()
    name = attrs["function_name"].encode()
    ins = [np.ascontiguousarray(a) for a in args]
    in_p = (ctypes.c_void_p * max(len(ins), 1))(*[a.ctypes.data for a in ins])
    in_b = (ctypes.c_size_t * max(len(ins), 1))(*[a.nbytes for a in ins])
    out_p = (ctypes.c_void_p * max(len(outs), 1))(*[o.ctypes.data for o in outs])
    out_b = (ctypes.c_size_t * max(len(outs), 1))(*[o.nbytes for o in outs])
    err = ctypes.c_void_p()
    rc = rt.lib().ph_dispatch(src, len(src), name, *[int(attrs[k]) for k in _HANDLER_ATTRS],
                              in_p, in_b, len(ins), out_p, out_b, len(outs), ctypes.byref(err))
    if rc != 0:
        msg = ctypes.string_at(err.value).decode() if err.value else "ph_dispatch failed"
        rt.lib().ph_free_error(err)
        raise RuntimeError(msg)


def make():
    registry = {}
    calls = []

    def ffi_call(target, result_shapes, vmap_method=None):
        assert target in registry, f"{target} not registered"

        def run(*args, **attrs):
            calls.append((target, dict(attrs), vmap_method))
            multi = isinstance(result_shapes, (list, tuple))
            shapes = list(result_shapes) if multi else [result_shapes]
            outs = [np.empty(s.shape, s.dtype) for s in shapes]
            _dispatch(args, outs, attrs)
            return tuple(outs) if multi else outs[0]

        return run

    ffi = types.SimpleNamespace(
        ffi_call=ffi_call,
        pycapsule=lambda fn: fn,
        register_ffi_target=lambda name, capsule, platform="cpu": registry.__setitem__((name), (capsule, platform)),
    )
    mod = types.ModuleType("jax")
    mod.ffi = ffi
    mod.ShapeDtypeStruct = ShapeDtypeStruct
    mod.devices = lambda: []
    mod.registry = registry
    mod.calls = calls
    return mod
