"""Kernel diagnostics: launch geometry, source size and gfx950 resource use.

`HipCallable.explain` / `FfiCallable.explain` return KernelDiagnostics
(reference: `src/palladium/diagnostics.py:20-82`); `PALLADIUM_EXPLAIN=1`
prints one stderr line per newly compiled kernel. Beyond the reference's
fields, `explain` compiles the source with hiprtc (no GPU needed) and reads
the code object's AMDGPU metadata note: VGPRs, SGPRs, AGPRs, spills,
scratch and LDS bytes, and the resulting waves per SIMD.
"""

from __future__ import annotations

import dataclasses
import os
import struct
import sys
from typing import Any

from palladium_amd.emit import emit_hip, launch_geometry
from palladium_amd.trace import KernelSpec

__all__ = ["KernelDiagnostics", "ResourceUsage", "code_object_resources", "explain_spec"]

# CDNA3/CDNA4 SIMD: 512 VGPRs per lane-slot budget, at most 8 waves/SIMD.
_VGPRS_PER_SIMD = 512
_MAX_WAVES_PER_SIMD = 8


# Per-instance scratch above this size earns a hint in the explain text: a
# large gridless block runs as one thread walking arrays in scratch memory.
SCRATCH_HINT_BYTES = 4096


@dataclasses.dataclass(frozen=True)
class ResourceUsage:
    vgprs: int
    agprs: int
    sgprs: int
    vgpr_spills: int
    sgpr_spills: int
    scratch_bytes: int
    lds_bytes: int
    waves_per_simd: int


@dataclasses.dataclass(frozen=True)
class KernelDiagnostics:
    """How one traced kernel executes.

    Attributes
    ----------
    name : str
        HIP entry point name.
    grid : tuple of int
        Pallas grid (program instances per axis).
    threadgroup : tuple of int or None
        Explicit workgroup size, None for the default.
    hip_lines : int
        Line count of the emitted source.
    blocks, block : int
        HIP launch: workgroups x lanes per workgroup.
    resources : ResourceUsage or None
        Register/LDS/scratch use of the compiled code object (None when
        not compiled).
    """

    name: str
    grid: tuple[int, ...]
    threadgroup: tuple[int, ...] | None
    hip_lines: int
    blocks: int = 0
    block: int = 0
    resources: ResourceUsage | None = None
    # threads per program instance: 1, or the block rows a lane-parallel
    # kernel spreads across lanes
    lanes: int = 1

    @property
    def msl_lines(self) -> int:
        """Source line count under the reference's field name."""
        return self.hip_lines

    def __str__(self) -> str:
        parts = [f"palladium kernel {self.name}: grid={self.grid}"]
        if self.threadgroup is not None:
            parts.append(f"threadgroup={self.threadgroup}")
        parts.append(f"hip_lines={self.hip_lines}")
        parts.append(f"launch={self.blocks}x{self.block}")
        if self.lanes > 1:
            parts.append(f"lanes/instance={self.lanes}")
        r = self.resources
        if r is not None:
            parts.append(
                f"vgprs={r.vgprs} sgprs={r.sgprs} spills={r.vgpr_spills + r.sgpr_spills} "
                f"scratch={r.scratch_bytes}B lds={r.lds_bytes}B waves/simd={r.waves_per_simd}"
            )
        text = " ".join(parts)
        if r is not None and r.scratch_bytes > SCRATCH_HINT_BYTES:
            text += (
                f"\n  hint: each program instance keeps {r.scratch_bytes} B of arrays in scratch "
                "memory; split the work with a grid and BlockSpecs so each instance holds a "
                "small block"
            )
        return text


def _notes(code: bytes) -> list[tuple[str, int, bytes]]:
    """(name, type, desc) of every ELF note in a 64-bit little-endian object."""
    if code[:4] != b"\x7fELF" or code[4] != 2:
        raise ValueError("not an ELF64 code object")
    e_shoff = struct.unpack_from("<Q", code, 0x28)[0]
    e_shentsize, e_shnum = struct.unpack_from("<HH", code, 0x3A)
    out = []
    for i in range(e_shnum):
        off = e_shoff + i * e_shentsize
        sh_type = struct.unpack_from("<I", code, off + 4)[0]
        if sh_type != 7:  # SHT_NOTE
            continue
        sh_offset, sh_size = struct.unpack_from("<QQ", code, off + 0x18)
        pos, end = sh_offset, sh_offset + sh_size
        while pos + 12 <= end:
            namesz, descsz, ntype = struct.unpack_from("<III", code, pos)
            pos += 12
            name = code[pos : pos + namesz].rstrip(b"\0").decode(errors="replace")
            pos += (namesz + 3) & ~3
            desc = code[pos : pos + descsz]
            pos += (descsz + 3) & ~3
            out.append((name, ntype, desc))
    return out


def code_object_resources(code: bytes, kernel_name: str) -> ResourceUsage:
    """Resource use of `kernel_name` from the NT_AMDGPU_METADATA note."""
    import msgpack

    for name, ntype, desc in _notes(code):
        if name == "AMDGPU" and ntype == 32:
            meta = msgpack.unpackb(desc, raw=False)
            for k in meta.get("amdhsa.kernels", []):
                if k.get(".name") == kernel_name:
                    vgprs = int(k.get(".vgpr_count", 0))
                    agprs = int(k.get(".agpr_count", 0))
                    regs = max(vgprs + agprs, 1)
                    granule = 8
                    regs = (regs + granule - 1) // granule * granule
                    waves = max(0, min(_MAX_WAVES_PER_SIMD, _VGPRS_PER_SIMD // regs))
                    return ResourceUsage(
                        vgprs=vgprs,
                        agprs=agprs,
                        sgprs=int(k.get(".sgpr_count", 0)),
                        vgpr_spills=int(k.get(".vgpr_spill_count", 0)),
                        sgpr_spills=int(k.get(".sgpr_spill_count", 0)),
                        scratch_bytes=int(k.get(".private_segment_fixed_size", 0)),
                        lds_bytes=int(k.get(".group_segment_fixed_size", 0)),
                        waves_per_simd=waves,
                    )
    raise ValueError(f"kernel {kernel_name} not found in the code object metadata")


def _tg_tuple(threadgroup: Any) -> tuple[int, ...] | None:
    if threadgroup is None:
        return None
    if isinstance(threadgroup, int):
        return (threadgroup,)
    return tuple(int(t) for t in threadgroup)


def explain_spec(spec: KernelSpec, threadgroup: Any = None, math_mode: Any = None,
                 compile: bool = True) -> KernelDiagnostics:
    """Diagnostics for a traced spec: emits HIP and, with `compile`,
    compiles it (hiprtc, no GPU) to report register and memory use."""
    from palladium_amd.dispatch import _block_of

    block = _block_of(threadgroup)
    src = emit_hip(spec, block=block, math_mode=math_mode)
    geo = launch_geometry(spec, block)
    res = None
    if compile:
        from palladium_amd import runtime as rt

        code = rt.compile_code_object(src, spec.name, math_mode if math_mode is not None else rt.MathMode.FAST)
        res = code_object_resources(code, spec.name)
    return KernelDiagnostics(
        name=spec.name,
        grid=tuple(int(g) for g in spec.grid),
        threadgroup=_tg_tuple(threadgroup),
        hip_lines=len(src.splitlines()),
        blocks=geo.blocks,
        block=geo.block,
        resources=res,
        lanes=geo.lanes,
    )


def _explain_enabled() -> bool:
    return os.environ.get("PALLADIUM_EXPLAIN", "") not in ("", "0")


def log_compile(spec: KernelSpec, threadgroup: Any = None, math_mode: Any = None) -> None:
    """One stderr line per compiled kernel when PALLADIUM_EXPLAIN is set."""
    if _explain_enabled():
        print(explain_spec(spec, threadgroup, math_mode), file=sys.stderr)
