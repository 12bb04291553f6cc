"""The HIP runtime layer: ctypes over `libpalladium_hip.so`.

This module plays the role metal-runtime plays for the reference
(`src/palladium/dispatch.py:18`, `examples/03_sde_montecarlo.py:79-94`,
`examples/04_reaction_diffusion.py:92-109`): math modes, compiled
kernels, device buffers, streams, events, and a `Batch` that queues many
launches (optionally as one HIP graph) with device-side timing.

Nothing here falls back to the CPU: if the native library is missing,
every entry point raises, naming the build command.
"""

from __future__ import annotations

import ctypes
import enum
import os
import threading
from pathlib import Path
from typing import Any, Sequence

import numpy as np

from palladium_amd import dtypes as _dtypes

from palladium_amd.errors import CompileError, PalladiumError

__all__ = [
    "Batch",
    "Buffer",
    "Event",
    "HipError",
    "Kernel",
    "MathMode",
    "Stream",
    "compile_code_object",
    "device_available",
    "device_name",
    "lib",
    "run",
]

PH_OK, PH_ERR_INVALID, PH_ERR_COMPILE, PH_ERR_RUNTIME = 0, 1, 2, 3
_LIB_NAME = "libpalladium_hip.so"


class HipError(PalladiumError, RuntimeError):
    """A HIP runtime call failed (allocation, copy, launch, sync)."""


class MathMode(str, enum.Enum):
    """Floating-point contract of a compiled kernel.

    SAFE: IEEE op order, no contraction, correctly rounded division and
    square root, deterministic `pow`. RELAXED: FMA contraction. FAST
    (default, as in the reference): contraction, reassociation, approximate
    transcendentals and division; infinities and NaNs are still honoured.
    REPRODUCIBLE (no counterpart in the reference): FAST's algebra with
    every operation deterministic, so a host restates the results bit for
    bit. The program takes FAST's jaxpr rewrites (common factors, affine
    shifts, power laws as exp2/log2, carried logs); then a float32 `a*b + c`
    whose product has no other use becomes one fused multiply-add (correctly
    rounded, so C's `fmaf` gives the same value); float32 `a / b` is
    `a * RN(1/b)`; `pow`, `log2` and `exp2` are deterministic
    double-precision functions rounded once to float. Other transcendentals
    and everything else are as SAFE.
    """

    SAFE = "safe"
    RELAXED = "relaxed"
    FAST = "fast"
    REPRODUCIBLE = "reproducible"

    @property
    def ordinal(self) -> int:
        return _MATH_MODE_ORDINALS[self.value]


# Same ordinals as the reference's C API (src/palladium/ffi.py:38), plus
# REPRODUCIBLE = 3, which the reference does not have.
_MATH_MODE_ORDINALS = {"safe": 0, "relaxed": 1, "fast": 2, "reproducible": 3}
REPRODUCIBLE_ORDINAL = 3


def math_mode_ordinal(mode: Any) -> int:
    value = mode.value if hasattr(mode, "value") else mode
    if isinstance(value, int):
        if value not in (0, 1, 2, 3):
            raise ValueError(f"math_mode ordinal {value} out of range")
        return value
    try:
        return _MATH_MODE_ORDINALS[str(value).lower()]
    except KeyError:
        raise ValueError(f"unknown math_mode {mode!r} (safe, relaxed, fast, reproducible)") from None


def library_path() -> Path:
    override = os.environ.get("PALLADIUM_HIP_LIBRARY")
    if override:
        return Path(override)
    return Path(__file__).resolve().parent / _LIB_NAME


_lib: ctypes.CDLL | None = None
_lib_lock = threading.Lock()

_P = ctypes.c_void_p
_PP = ctypes.POINTER(ctypes.c_void_p)
_ERR = ctypes.POINTER(ctypes.c_char_p)


def _declare(L: ctypes.CDLL) -> None:
    c = ctypes
    sig = {
        "ph_version": (c.c_char_p, []),
        "ph_free_error": (None, [c.c_void_p]),
        "ph_compile_code_object": (c.c_int, [c.c_char_p, c.c_size_t, c.c_char_p, c.c_int, c.c_char_p, _PP, c.POINTER(c.c_size_t), _PP]),
        "ph_free_code_object": (None, [c.c_void_p]),
        "ph_compile_options": (c.c_char_p, [c.c_int]),
        "ph_get_kernel": (c.c_int, [c.c_char_p, c.c_size_t, c.c_char_p, c.c_int, _PP, _PP]),
        "ph_kernel_cache_size": (c.c_size_t, []),
        "ph_load_code_object": (c.c_int, [c.c_void_p, c.c_size_t, c.c_char_p, _PP, _PP]),
        "ph_launch": (c.c_int, [_P, c.c_uint, c.c_uint, c.c_uint, c.c_uint, c.c_uint, c.c_uint, c.c_uint, _P, _PP, _PP]),
        "ph_launch_ptrs": (c.c_int, [_P, c.c_uint, c.c_uint, _P, _PP, c.c_size_t, _PP]),
        "ph_dispatch": (c.c_int, [c.c_char_p, c.c_size_t, c.c_char_p, c.c_int64, c.c_int64, c.c_int64, c.c_int64, c.c_int64,
                                  c.c_int64, _PP, c.POINTER(c.c_size_t), c.c_size_t, _PP, c.POINTER(c.c_size_t),
                                  c.c_size_t, _PP]),
        "ph_dispatch_device": (c.c_int, [c.c_char_p, c.c_size_t, c.c_char_p, c.c_int64, c.c_int64, c.c_int64, c.c_int64,
                                         c.c_int64, c.c_int64, _P, _PP, c.c_size_t, _PP, c.c_size_t, _PP]),
        "ph_device_count": (c.c_int, [c.POINTER(c.c_int)]),
        "ph_device_name": (c.c_int, [c.c_char_p, c.c_size_t]),
        "ph_malloc": (c.c_int, [c.c_size_t, _PP, _PP]),
        "ph_free": (c.c_int, [_P]),
        "ph_host_alloc": (c.c_int, [c.c_size_t, _PP, _PP]),
        "ph_host_free": (c.c_int, [_P]),
        "ph_memcpy_h2d": (c.c_int, [_P, _P, c.c_size_t, _P, _PP]),
        "ph_memcpy_d2h": (c.c_int, [_P, _P, c.c_size_t, _P, _PP]),
        "ph_memcpy_d2h_wait": (c.c_int, [_P, _P, c.c_size_t, _P, _PP]),
        "ph_memcpy_d2d": (c.c_int, [_P, _P, c.c_size_t, _P, _PP]),
        "ph_stream_create": (c.c_int, [_PP, _PP]),
        "ph_stream_destroy": (c.c_int, [_P]),
        "ph_stream_synchronize": (c.c_int, [_P, _PP]),
        "ph_event_create": (c.c_int, [_PP, _PP]),
        "ph_event_destroy": (c.c_int, [_P]),
        "ph_event_record": (c.c_int, [_P, _P, _PP]),
        "ph_event_synchronize": (c.c_int, [_P, _PP]),
        "ph_event_query": (c.c_int, [_P]),
        "ph_event_elapsed_ms": (c.c_int, [_P, _P, c.POINTER(c.c_float), _PP]),
        "ph_device_synchronize": (c.c_int, [_PP]),
        "ph_stream_begin_capture": (c.c_int, [_P, _PP]),
        "ph_stream_end_capture": (c.c_int, [_P, _PP, _PP]),
        "ph_graph_launch": (c.c_int, [_P, _P, _PP]),
        "ph_graph_destroy": (c.c_int, [_P]),
        "ph_dispatch_staging_count": (c.c_size_t, []),
        "ph_noalloc_scratch_bytes": (c.c_size_t, []),
        "ph_dispatch_noalloc": (c.c_int, [_P, c.c_int64, c.c_int64, c.c_int64, c.c_int64, c.c_int64, _P, _PP,
                                          c.POINTER(c.c_size_t), c.c_size_t, _PP, c.POINTER(c.c_size_t),
                                          c.c_size_t, _PP]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def lib() -> ctypes.CDLL:
    """The loaded native library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is None:
            path = library_path()
            if not path.is_file():
                raise HipError(
                    f"palladium_amd's native library ({path}) is not built; run "
                    "`python -m palladium_amd.build` (or __graft_entry__.build())"
                )
            L = ctypes.CDLL(str(path))
            _declare(L)
            _lib = L
    return _lib


def _check(rc: int, err: ctypes.c_void_p, what: str = "") -> None:
    if rc == PH_OK:
        return
    msg = ctypes.cast(err, ctypes.c_char_p).value.decode(errors="replace") if err.value else f"{what} failed"
    if err.value:
        lib().ph_free_error(err)
    if rc == PH_ERR_COMPILE:
        raise CompileError(msg)
    if rc == PH_ERR_INVALID:
        raise ValueError(msg)
    raise HipError(msg)


def _call(fn_name: str, *args: Any) -> None:
    err = ctypes.c_void_p()
    rc = getattr(lib(), fn_name)(*args, ctypes.byref(err))
    _check(rc, err, fn_name)


def device_count() -> int:
    n = ctypes.c_int(0)
    lib().ph_device_count(ctypes.byref(n))
    return n.value


def device_available() -> bool:
    try:
        return device_count() > 0
    except HipError:
        return False


def device_name() -> str:
    buf = ctypes.create_string_buffer(256)
    if lib().ph_device_name(buf, 256) != PH_OK:
        raise HipError("no HIP device")
    return buf.value.decode()


def compile_options(math_mode: Any) -> str:
    return lib().ph_compile_options(math_mode_ordinal(math_mode)).decode()


def compile_code_object(source: str, name: str, math_mode: Any = MathMode.FAST, arch: str = "gfx950") -> bytes:
    """hiprtc-compile `source` to a gfx950 code object; needs no GPU."""
    src = source.encode()
    code = ctypes.c_void_p()
    size = ctypes.c_size_t()
    err = ctypes.c_void_p()
    rc = lib().ph_compile_code_object(src, len(src), name.encode(), math_mode_ordinal(math_mode), arch.encode(),
                                      ctypes.byref(code), ctypes.byref(size), ctypes.byref(err))
    _check(rc, err, "ph_compile_code_object")
    try:
        return ctypes.string_at(code, size.value)
    finally:
        lib().ph_free_code_object(code)


# ---------------------------------------------------------------------------
# streams / events


class Stream:
    """A HIP stream at the default priority."""

    def __init__(self, handle: int | None = None, owned: bool = True):
        if handle is None:
            h = ctypes.c_void_p()
            _call("ph_stream_create", ctypes.byref(h))
            handle = h.value
        self.handle = handle
        self._owned = owned and handle is not None

    @classmethod
    def default(cls) -> "Stream":
        """The null stream."""
        return _DefaultStream()

    def synchronize(self) -> None:
        _call("ph_stream_synchronize", ctypes.c_void_p(self.handle))

    def __del__(self) -> None:
        if getattr(self, "_owned", False) and _lib is not None:
            _lib.ph_stream_destroy(ctypes.c_void_p(self.handle))


class _DefaultStream(Stream):
    def __init__(self) -> None:
        self.handle = None
        self._owned = False


def _stream_handle(stream: Any) -> ctypes.c_void_p:
    if stream is None:
        return ctypes.c_void_p(None)
    if isinstance(stream, Stream):
        return ctypes.c_void_p(stream.handle)
    if hasattr(stream, "cuda_stream"):  # torch.cuda.Stream
        return ctypes.c_void_p(stream.cuda_stream)
    return ctypes.c_void_p(int(stream))


class Event:
    def __init__(self) -> None:
        h = ctypes.c_void_p()
        _call("ph_event_create", ctypes.byref(h))
        self.handle = h.value

    def record(self, stream: Any = None) -> "Event":
        _call("ph_event_record", ctypes.c_void_p(self.handle), _stream_handle(stream))
        return self

    def synchronize(self) -> None:
        _call("ph_event_synchronize", ctypes.c_void_p(self.handle))

    def query(self) -> bool:
        r = lib().ph_event_query(ctypes.c_void_p(self.handle))
        if r < 0:
            raise HipError("hipEventQuery failed")
        return r == 1

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        _call("ph_event_elapsed_ms", ctypes.c_void_p(self.handle), ctypes.c_void_p(end.handle), ctypes.byref(ms))
        return float(ms.value)

    def __del__(self) -> None:
        if getattr(self, "handle", None) and _lib is not None:
            _lib.ph_event_destroy(ctypes.c_void_p(self.handle))


def synchronize() -> None:
    _call("ph_device_synchronize")


# ---------------------------------------------------------------------------
# buffers


class Buffer:
    """A device allocation with a shape and dtype (HBM, `hipMalloc`)."""

    def __init__(self, shape: Sequence[int], dtype: Any, ptr: int | None = None, owner: Any = None):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self._owner = owner
        if ptr is None:
            p = ctypes.c_void_p()
            _call("ph_malloc", ctypes.c_size_t(self.nbytes), ctypes.byref(p))
            ptr = p.value
            self._owned = True
        else:
            self._owned = False
        self.ptr = int(ptr)

    @classmethod
    def empty(cls, shape: Sequence[int], dtype: Any = np.float32) -> "Buffer":
        return cls(shape, dtype)

    @classmethod
    def from_numpy(cls, arr: np.ndarray, stream: Any = None) -> "Buffer":
        arr = np.ascontiguousarray(arr)
        b = cls(arr.shape, arr.dtype)
        b.copy_from(arr, stream)
        return b

    @classmethod
    def wrap(cls, obj: Any) -> "Buffer":
        """Zero-copy view of a device array (torch CUDA/HIP tensor or any
        object exposing `__cuda_array_interface__`).

        torch wheels carry their own libamdhip64. Import torch before this
        module loads its native library, so that the library binds to the
        runtime torch already holds: a process with two HIP runtimes loaded
        leaves torch without a device."""
        if hasattr(obj, "data_ptr") and getattr(obj, "is_cuda", False):
            if not obj.is_contiguous():
                raise ValueError("device tensors must be contiguous")
            tname = str(obj.dtype).replace("torch.", "")
            dt = _dtypes.bfloat16 if tname == "bfloat16" else np.dtype(tname)
            return cls(tuple(obj.shape), dt, ptr=obj.data_ptr(), owner=obj)
        cai = getattr(obj, "__cuda_array_interface__", None)
        if cai is not None:
            dt = np.dtype(cai["typestr"])
            strides = cai.get("strides")
            if strides is not None:
                dense = tuple(int(np.prod(cai["shape"][k + 1 :], dtype=np.int64)) * dt.itemsize for k in range(len(cai["shape"])))
                if tuple(strides) != dense:
                    raise ValueError("device arrays must be C-contiguous")
            return cls(cai["shape"], dt, ptr=cai["data"][0], owner=obj)
        raise TypeError(f"cannot wrap {type(obj).__name__} as a device buffer")

    def copy_from(self, arr: np.ndarray, stream: Any = None) -> None:
        """Host -> device copy. With `stream`, the copy is ordered on it and
        may still be reading `arr` on return: the caller keeps `arr` alive
        until the stream passes this point. A non-contiguous `arr` is
        compacted into a temporary first, and then the copy is waited for,
        since nothing would keep the temporary alive."""
        src = np.ascontiguousarray(arr)
        if src.nbytes != self.nbytes:
            raise ValueError(f"copy_from: {src.nbytes} bytes into a {self.nbytes}-byte buffer")
        if self.nbytes:
            _call("ph_memcpy_h2d", ctypes.c_void_p(self.ptr), src.ctypes.data_as(ctypes.c_void_p),
                  ctypes.c_size_t(self.nbytes), _stream_handle(stream))
            if stream is None or src is not arr:
                synchronize_stream(stream)

    def to_numpy(self, stream: Any = None) -> np.ndarray:
        """Copy to a new host array after the work queued on `stream`."""
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            _call("ph_memcpy_d2h_wait", out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(self.ptr),
                  ctypes.c_size_t(self.nbytes), _stream_handle(stream))
        return out

    def __del__(self) -> None:
        if getattr(self, "_owned", False) and _lib is not None:
            _lib.ph_free(ctypes.c_void_p(self.ptr))

    def __repr__(self) -> str:
        return f"Buffer(shape={self.shape}, dtype={self.dtype.name})"


class PinnedBuffer:
    """Page-locked host memory (`hipHostMalloc`): the target of an
    asynchronous device -> host copy."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _call("ph_host_alloc", ctypes.c_size_t(self.nbytes), ctypes.byref(p))
        self.ptr = int(p.value)

    def view(self, shape: Sequence[int], dtype: Any) -> np.ndarray:
        """A NumPy view of the memory (valid while this object lives)."""
        raw = (ctypes.c_char * max(self.nbytes, 1)).from_address(self.ptr)
        return np.frombuffer(raw, dtype=np.uint8, count=self.nbytes).view(np.dtype(dtype)).reshape(tuple(shape))

    def copy_from_device(self, buf: "Buffer", stream: Any = None) -> None:
        """Enqueue buf -> this memory on `stream` (returns at once)."""
        if buf.nbytes > self.nbytes:
            raise ValueError("copy_from_device: pinned buffer too small")
        if buf.nbytes:
            _call("ph_memcpy_d2h", ctypes.c_void_p(self.ptr), ctypes.c_void_p(buf.ptr), ctypes.c_size_t(buf.nbytes),
                  _stream_handle(stream))

    def __del__(self) -> None:
        if getattr(self, "ptr", None) and _lib is not None:
            _lib.ph_host_free(ctypes.c_void_p(self.ptr))


def synchronize_stream(stream: Any) -> None:
    _call("ph_stream_synchronize", _stream_handle(stream))


def device_pointer(obj: Any) -> int:
    if isinstance(obj, Buffer):
        return obj.ptr
    return Buffer.wrap(obj).ptr


# ---------------------------------------------------------------------------
# kernels


class Kernel:
    """Compiled HIP source (hiprtc, gfx950), loaded lazily on first launch.

    Counterpart of `metal_runtime.Kernel(source, name, math_mode)`
    (`src/palladium/dispatch.py:291`). Compilation is cached natively by
    (source, name, math mode, device).
    """

    def __init__(self, source: str, name: str, math_mode: Any = MathMode.FAST):
        self.source = source
        self.name = name
        self.math_mode = MathMode(_mode_value(math_mode))
        self._handle: int | None = None
        self._lock = threading.Lock()

    def load(self) -> int:
        if self._handle is None:
            with self._lock:
                if self._handle is None:
                    from palladium_amd import compile_worker

                    h = ctypes.c_void_p()
                    if compile_worker.isolation_enabled():
                        # compile in the helper process; a compiler crash
                        # there is a CompileError here
                        code = compile_worker.compile_isolated(self.source, self.name, self.math_mode.ordinal)
                        _call("ph_load_code_object", code, len(code), self.name.encode(), ctypes.byref(h))
                    else:
                        src = self.source.encode()
                        _call("ph_get_kernel", src, len(src), self.name.encode(), self.math_mode.ordinal,
                              ctypes.byref(h))
                    self._handle = h.value
        return self._handle

    def code_object(self) -> bytes:
        return compile_code_object(self.source, self.name, self.math_mode)

    def launch_ptrs(self, blocks: int, block: int, ptrs: Sequence[int], stream: Any = None) -> None:
        h = self.load()
        arr = (ctypes.c_void_p * max(len(ptrs), 1))(*ptrs)
        _call("ph_launch_ptrs", ctypes.c_void_p(h), ctypes.c_uint(blocks), ctypes.c_uint(block),
              _stream_handle(stream), arr, ctypes.c_size_t(len(ptrs)))

    def launch(self, grid: Sequence[int], block: Sequence[int], args: Sequence[Any], stream: Any = None, shared: int = 0) -> None:
        """Launch with arbitrary arguments: Buffers / device arrays become
        pointers, NumPy scalars pass by value with their own width."""
        h = self.load()
        holders = []
        for a in args:
            if isinstance(a, Buffer):
                holders.append(ctypes.c_void_p(a.ptr))
            elif isinstance(a, (np.generic,)):
                holders.append(_scalar_ctype(a))
            elif isinstance(a, float):
                holders.append(ctypes.c_float(a))
            elif isinstance(a, int):
                holders.append(ctypes.c_int(a))
            else:
                holders.append(ctypes.c_void_p(device_pointer(a)))
        params = (ctypes.c_void_p * max(len(holders), 1))(*[ctypes.cast(ctypes.pointer(x), ctypes.c_void_p) for x in holders])
        g = tuple(grid) + (1,) * (3 - len(grid))
        b = tuple(block) + (1,) * (3 - len(block))
        _call("ph_launch", ctypes.c_void_p(h), *[ctypes.c_uint(x) for x in g], *[ctypes.c_uint(x) for x in b],
              ctypes.c_uint(shared), _stream_handle(stream), params)


def _mode_value(m: Any) -> str:
    return {0: "safe", 1: "relaxed", 2: "fast", 3: "reproducible"}[math_mode_ordinal(m)]


def _scalar_ctype(a: np.generic) -> Any:
    dt = np.dtype(a.dtype)
    table = {
        "float32": ctypes.c_float, "float64": ctypes.c_double, "int32": ctypes.c_int32,
        "uint32": ctypes.c_uint32, "int64": ctypes.c_int64, "uint64": ctypes.c_uint64,
    }
    if dt.name not in table:
        raise TypeError(f"unsupported kernel scalar dtype {dt}")
    return table[dt.name](a.item())


def run(kernel: Kernel, grid: int | Sequence[int], buffers: Sequence[Any], scalars: Sequence[Any] = (),
        block: int = 256, stream: Any = None, wait: bool = True) -> None:
    """One launch of a hand-written kernel: `grid` threads (1-D) or
    `grid` workgroups x `block` lanes when `grid` is a tuple of blocks.
    Mirrors `metal_runtime.run(kernel, grid=N, buffers=..., scalars=...)`
    (`examples/03_sde_montecarlo.py:90`)."""
    if isinstance(grid, int):
        blocks = ((grid + block - 1) // block,)
    else:
        blocks = tuple(grid)
    kernel.launch(blocks, (block,), [*buffers, *scalars], stream)
    if wait:
        synchronize_stream(stream)


class Batch:
    """Queue many launches, submit them together, time them on device.

    The counterpart of `mr.Batch` in the reference's Gray-Scott driver
    (`examples/04_reaction_diffusion.py:100-109`). `commit(graph=True)`
    captures the queued launches into one HIP graph (launched once);
    `gpu_time` is the device time between events bracketing the batch.
    """

    def __init__(self, stream: Any = None):
        self.stream = stream if stream is not None else Stream()
        self._items: list[tuple[Kernel, int, int, list[int]]] = []
        self._start: Event | None = None
        self._stop: Event | None = None
        self._graph: int | None = None

    def add(self, kernel: Kernel, blocks: int, block: int, ptrs: Sequence[int]) -> "Batch":
        self._items.append((kernel, int(blocks), int(block), [int(p) for p in ptrs]))
        return self

    def _enqueue(self) -> None:
        for k, nb, b, ptrs in self._items:
            k.launch_ptrs(nb, b, ptrs, self.stream)

    def commit(self, graph: bool = False) -> "Batch":
        for k, *_ in self._items:
            k.load()
        self._release_graph()  # a re-commit replaces the previous graph
        self._start = Event()
        self._stop = Event()
        if graph:
            _call("ph_stream_begin_capture", _stream_handle(self.stream))
            g = ctypes.c_void_p()
            try:
                self._enqueue()
            except BaseException:
                # End the capture so the stream is usable again; the launch
                # error is the one worth reporting.
                err = ctypes.c_void_p()
                if lib().ph_stream_end_capture(_stream_handle(self.stream), ctypes.byref(g), ctypes.byref(err)) == PH_OK:
                    lib().ph_graph_destroy(g)
                elif err.value:
                    lib().ph_free_error(err)
                raise
            _call("ph_stream_end_capture", _stream_handle(self.stream), ctypes.byref(g))
            self._graph = g.value
            self._start.record(self.stream)
            _call("ph_graph_launch", ctypes.c_void_p(self._graph), _stream_handle(self.stream))
        else:
            self._start.record(self.stream)
            self._enqueue()
        self._stop.record(self.stream)
        return self

    def wait(self) -> None:
        if self._stop is None:
            raise HipError("Batch.wait before commit")
        self._stop.synchronize()

    @property
    def gpu_time(self) -> float:
        """Seconds of device time for the committed batch."""
        self.wait()
        return self._start.elapsed_ms(self._stop) / 1e3

    def _release_graph(self) -> None:
        if getattr(self, "_graph", None) and _lib is not None:
            # The graph may still be running: let it finish before destroying it.
            err = ctypes.c_void_p()
            if self._stop is not None:
                _lib.ph_event_synchronize(ctypes.c_void_p(self._stop.handle), ctypes.byref(err))
                if err.value:
                    _lib.ph_free_error(err)
            _lib.ph_graph_destroy(ctypes.c_void_p(self._graph))
        self._graph = None

    def __del__(self) -> None:
        self._release_graph()
