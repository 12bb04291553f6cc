"""Step 3 of the pipeline: compile emitted HIP with hiprtc and run it.

`bind(spec, source)` returns a `BoundKernel` with the reference's
NumPy-in/NumPy-out contract (`src/palladium/dispatch.py:89-314`): strict
arity/dtype/shape checks raising DispatchError with the same messages,
input device buffers reused across calls after waiting on the previous
launch, fresh outputs per call, a per-kernel launch lock, async `launch`
returning a `PendingResult`, and `pinned` re-dispatch without uploads.

Additions for MI355X: `launch_device` runs on caller-owned device arrays
(no host staging, for benches and for composing with torch), and each
BoundKernel owns a HIP stream so launches from different kernels overlap.

`PALLADIUM_DUMP_HIP=1` prints each kernel's source before compiling; a
directory path writes `<name>_<hash>.hip` files
(as `PALLADIUM_DUMP_MSL`, `src/palladium/dispatch.py:27-38`).
"""

from __future__ import annotations

import dataclasses
import hashlib
import os
import threading
from collections.abc import Callable
from pathlib import Path
from typing import Any

import numpy as np

from palladium_amd import runtime as rt
from palladium_amd.dtypes import name as _dtype_name
from palladium_amd.emit.core import LaunchGeometry, launch_geometry
from palladium_amd.errors import CompileError, DispatchError
from palladium_amd.trace import KernelSpec

__all__ = ["BoundKernel", "PendingResult", "bind"]

# Launches a BoundKernel keeps in flight before `launch` blocks.
IN_FLIGHT = 4


def _dump_hip(name: str, source: str) -> None:
    dump = os.environ.get("PALLADIUM_DUMP_HIP")
    if not dump:
        return
    if dump == "1" or dump.lower() == "stdout":
        print(f"// palladium_amd kernel: {name}\n{source}")
        return
    directory = Path(dump)
    directory.mkdir(parents=True, exist_ok=True)
    digest = hashlib.sha256(source.encode()).hexdigest()[:12]
    (directory / f"{name}_{digest}.hip").write_text(source)


def numbered(source: str) -> str:
    return "\n".join(f"{n:4d} | {line}" for n, line in enumerate(source.splitlines(), 1))


@dataclasses.dataclass
class PendingResult:
    """A launched kernel that may still be running.

    Attributes
    ----------
    event : runtime.Event
        Recorded after the launch on the kernel's stream.
    stream : runtime.Stream

    The device outputs are private: they belong to one of the kernel's
    IN_FLIGHT buffer sets, which a later launch overwrites. `wait()`
    returns host copies that stay valid.
    """

    event: rt.Event
    _out_bufs: list[rt.Buffer]
    stream: Any
    # Host arrays an asynchronous upload may still be reading.
    host_inputs: tuple = dataclasses.field(default=(), repr=False)
    # Pinned host copies of the outputs, filled by copies queued right after
    # the launch (None: read the device buffers back on wait()).
    staged: list[rt.PinnedBuffer] | None = dataclasses.field(default=None, repr=False)
    _results: tuple | None = dataclasses.field(default=None, repr=False)
    _lock: threading.Lock = dataclasses.field(default_factory=threading.Lock, repr=False)

    def done(self) -> bool:
        return self.event.query()

    def _settle(self) -> tuple:
        """Wait for the launch and its queued readbacks once, and keep the
        outputs as fresh host arrays (the staging may then be reused)."""
        with self._lock:
            if self._results is None:
                self.event.synchronize()
                self.host_inputs = ()
                if self.staged is not None:
                    self._results = tuple(np.array(p.view(b.shape, b.dtype)) for p, b in zip(self.staged, self._out_bufs))
                    self.staged = None
                else:
                    self._results = tuple(b.to_numpy(self.stream) for b in self._out_bufs)
            return self._results

    def wait(self) -> np.ndarray | tuple[np.ndarray, ...]:
        """Block until the GPU is done, then return the outputs (fresh
        arrays, the same ones on every call)."""
        outs = self._settle()
        return outs[0] if len(outs) == 1 else outs


@dataclasses.dataclass(frozen=True)
class BoundKernel:
    """A compiled HIP kernel behind a NumPy-in/NumPy-out call.

    Attributes
    ----------
    spec : KernelSpec
    kernel : runtime.Kernel
    hip_source : str
        Exact source that compiled.
    threadgroup : int or None
        Workgroup size (lanes); None means the default (256).
    geometry : LaunchGeometry
    """

    spec: KernelSpec
    kernel: rt.Kernel
    hip_source: str
    threadgroup: int | tuple[int, ...] | None = None
    geometry: LaunchGeometry | None = None
    # Buffer sets for launches in flight: set k (inputs, device outputs and
    # pinned host staging for the outputs) serves launches k, k + IN_FLIGHT,
    # ...; a launch waits only for the last launch that used its set, so
    # uploads, kernels and readbacks of successive calls overlap.
    _ring: list[tuple[list[rt.Buffer], list[rt.Buffer], list[rt.PinnedBuffer]]] = dataclasses.field(
        default_factory=list, compare=False, repr=False)
    _ring_pending: list[PendingResult | None] = dataclasses.field(default_factory=list, compare=False, repr=False)
    _ring_next: list[int] = dataclasses.field(default_factory=lambda: [0], compare=False, repr=False)
    _launch_lock: threading.Lock = dataclasses.field(default_factory=threading.Lock, compare=False, repr=False)
    _stream: list[rt.Stream] = dataclasses.field(default_factory=list, compare=False, repr=False)

    @property
    def stream(self) -> rt.Stream:
        if not self._stream:
            self._stream.append(rt.Stream())
        return self._stream[0]

    def _geo(self) -> LaunchGeometry:
        return self.geometry or launch_geometry(self.spec, _block_of(self.threadgroup))

    def _check_args(self, arrays: tuple) -> list[np.ndarray]:
        spec = self.spec
        if len(arrays) != len(spec.inputs):
            raise DispatchError(f"kernel takes {len(spec.inputs)} arrays, got {len(arrays)}")
        out = []
        for i, (a, info) in enumerate(zip(arrays, spec.inputs)):
            arr = np.asarray(a)
            if arr.dtype != info.dtype:
                raise DispatchError(
                    f"argument {i}: dtype {_dtype_name(arr.dtype)} does not match the traced "
                    f"{_dtype_name(info.dtype)}; cast explicitly"
                )
            if arr.shape != info.array_shape:
                raise DispatchError(f"argument {i}: expected shape {info.array_shape}, got {arr.shape}")
            out.append(np.ascontiguousarray(arr))
        return out

    def _new_outputs(self) -> list[rt.Buffer]:
        return [rt.Buffer.empty(info.array_shape, info.dtype) for info in self.spec.outputs]

    def launch(self, *arrays: np.ndarray) -> PendingResult:
        """Upload inputs and launch without blocking on the result.

        Thread-safe: uploads and launches are serialised on a per-kernel
        lock; waits are not locked. Up to IN_FLIGHT launches may be queued:
        each uses one of IN_FLIGHT input buffer sets in turn, after waiting
        out the launch that last read that set.

        Raises
        ------
        DispatchError
            Argument count, shape or dtype mismatch. Dtypes are never cast.
        """
        arrs = self._check_args(arrays)
        with self._launch_lock:
            k = self._ring_next[0]
            self._ring_next[0] = (k + 1) % IN_FLIGHT
            if len(self._ring) <= k:
                outs = self._new_outputs()
                self._ring.append(([rt.Buffer.empty(a.shape, a.dtype) for a in arrs], outs,
                                   [rt.PinnedBuffer(b.nbytes) for b in outs]))
                self._ring_pending.append(None)
            previous = self._ring_pending[k]
            if previous is not None:
                previous._settle()  # its outputs leave the set's staging first
            in_bufs, out_bufs, staging = self._ring[k]
            stream = self.stream
            for buf, a in zip(in_bufs, arrs):
                buf.copy_from(a, stream)
            geo = self._geo()
            self.kernel.launch_ptrs(geo.blocks, geo.block, [b.ptr for b in in_bufs] + [b.ptr for b in out_bufs], stream)
            for pin, buf in zip(staging, out_bufs):
                pin.copy_from_device(buf, stream)
            pending = PendingResult(rt.Event().record(stream), out_bufs, stream, host_inputs=tuple(arrs),
                                    staged=list(staging))
            self._ring_pending[k] = pending
            return pending

    def __call__(self, *arrays: np.ndarray) -> np.ndarray | tuple[np.ndarray, ...]:
        """Launch over the grid and return the outputs (NumPy)."""
        return self.launch(*arrays).wait()

    def pinned(self, *arrays: np.ndarray) -> Callable[[], np.ndarray | tuple[np.ndarray, ...]]:
        """Upload once; return a zero-argument callable that re-dispatches
        on the pinned device buffers with fresh outputs
        (`src/palladium/dispatch.py:230-255`). The pinned inputs live in
        buffers of their own, so later `launch` calls cannot overwrite them."""
        arrs = self._check_args(arrays)
        pinned = [rt.Buffer.empty(a.shape, a.dtype) for a in arrs]
        for buf, a in zip(pinned, arrs):
            buf.copy_from(a)  # synchronous: the host arrays may go away
        # one output set and its pinned readback staging, for this callable
        outs = self._new_outputs()
        staging = [rt.PinnedBuffer(b.nbytes) for b in outs]
        call_lock = threading.Lock()

        def call() -> np.ndarray | tuple[np.ndarray, ...]:
            with call_lock:  # the output set is reused call after call
                with self._launch_lock:
                    stream = self.stream
                    geo = self._geo()
                    self.kernel.launch_ptrs(geo.blocks, geo.block, [b.ptr for b in pinned] + [b.ptr for b in outs],
                                            stream)
                    for pin, buf in zip(staging, outs):
                        pin.copy_from_device(buf, stream)
                    pending = PendingResult(rt.Event().record(stream), outs, stream, staged=list(staging))
                return pending.wait()

        return call

    def launch_device(self, *operands: Any, stream: Any = None) -> None:
        """Launch on device-resident operands (inputs then outputs): runtime
        Buffers, torch tensors on the GPU, or `__cuda_array_interface__`
        objects. No copies, no synchronisation; shapes and dtypes are
        checked against the spec."""
        infos = list(self.spec.inputs) + list(self.spec.outputs)
        if len(operands) != len(infos):
            raise DispatchError(f"kernel takes {len(infos)} device operands (inputs then outputs), got {len(operands)}")
        ptrs = []
        for i, (o, info) in enumerate(zip(operands, infos)):
            b = o if isinstance(o, rt.Buffer) else rt.Buffer.wrap(o)
            if b.dtype != info.dtype:
                raise DispatchError(
                    f"operand {i}: dtype {_dtype_name(b.dtype)} does not match the traced {_dtype_name(info.dtype)}"
                )
            if b.shape != tuple(info.array_shape):
                raise DispatchError(f"operand {i}: expected shape {info.array_shape}, got {b.shape}")
            ptrs.append(b.ptr)
        geo = self._geo()
        self.kernel.launch_ptrs(geo.blocks, geo.block, ptrs, stream if stream is not None else self.stream)


def _tile_of(threadgroup: Any) -> tuple[int, int] | None:
    """The (axis-0, axis-1) instance tile of a 2-D threadgroup: Metal's
    threadsPerThreadgroup (x, y) over a grid whose x is program_id(0), as
    the reference dispatches it. None for an int, a 1-D tuple, or a 3-D
    tuple with z > 1 (those only set the workgroup size)."""
    if threadgroup is None or isinstance(threadgroup, int):
        return None
    tg = [int(t) for t in threadgroup]
    if len(tg) < 2 or any(t != 1 for t in tg[2:]):
        return None
    return tg[0], tg[1]


def _block_of(threadgroup: Any) -> int | None:
    if threadgroup is None:
        return None
    if isinstance(threadgroup, int):
        return threadgroup
    tg = [int(t) for t in threadgroup]
    n = 1
    for t in tg:
        n *= t
    return n


def bind(spec: KernelSpec, hip_source: str, *, math_mode: Any = rt.MathMode.FAST,
         threadgroup: int | tuple[int, ...] | None = None) -> BoundKernel:
    """Wrap emitted HIP source as a dispatchable kernel.

    The source compiles (hiprtc, gfx950) on first launch, or eagerly here
    when a device is present, so compile errors surface at bind time with
    the line-numbered source attached.

    Raises
    ------
    CompileError
        hiprtc rejected the source.
    """
    _dump_hip(spec.name, hip_source)
    kernel = rt.Kernel(hip_source, spec.name, math_mode)
    try:
        if rt.device_available():
            kernel.load()
        else:
            kernel.code_object()
    except CompileError as e:
        raise CompileError(f"{e}\n\npalladium_amd-emitted source:\n{numbered(hip_source)}") from None
    return BoundKernel(
        spec=spec,
        kernel=kernel,
        hip_source=hip_source,
        threadgroup=threadgroup,
        geometry=launch_geometry(spec, _block_of(threadgroup)),
    )
