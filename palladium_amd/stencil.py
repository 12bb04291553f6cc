"""Gray-Scott with temporal blocking: K time steps per pass through HBM.

The emitted per-step kernel (`workloads.gray_scott_call`, the Pallas path of
`examples/04_reaction_diffusion.py:61-74`) reads both fields and writes both
fields every step: 16 bytes per cell-step, so at best HBM (or Infinity Cache)
bandwidth / 16 cell-steps per second. This hand-written kernel (in the way
`df32.py` is hand-written: HIP source through `runtime.Kernel`) advances a
workgroup's tile K steps at once. It stages the tile plus a K-cell halo of
both fields in LDS (periodic wraparound applied at the load), then applies
the update K times on a region that shrinks by one cell per side per step
(each step computes its cells into registers, waits at a barrier, and
writes them back over the one LDS buffer; or ping-pongs two buffers), and
writes back only the tile. Reads per pass: (TH + 2K)(TW + 2K) / (TH TW)
times the tile; writes: the tile; so a cell-step costs about 8/K (1 +
halo) + 8/K bytes of HBM instead of 16.

Every cell value of every intermediate step is computed with the same
operations in the same order as the per-step kernel (and the C oracle,
`oracle/oracle.c:oracle_gray_scott_step`): the halo cells are recomputed,
not approximated, so under SAFE the fields after any number of steps are
bit-identical to the oracle's.
"""

from __future__ import annotations

import dataclasses
from typing import Any

import numpy as np

from palladium_amd import runtime as rt
from palladium_amd.emit.core import format_float

__all__ = ["FusedGrayScott", "fused_source", "gray_scott_fused_run"]

WORKGROUP = 256
NUM_XCDS = 8


def _update(src: str, dst_u: str, dst_v: str, lit: dict) -> list[str]:
    """One cell's Gray-Scott update from LDS buffer `src` at (rr, cc), in
    the op order of the per-step kernel and the oracle."""
    u, v = f"su{src}", f"sv{src}"
    return [
        f"const float uc = {u}[rr][cc], vc = {v}[rr][cc];",
        f"float lu = {u}[rr + 1][cc] + {u}[rr - 1][cc];",
        f"lu = lu + {u}[rr][cc + 1];",
        f"lu = lu + {u}[rr][cc - 1];",
        "lu = lu - 4.0f * uc;",
        f"float lv = {v}[rr + 1][cc] + {v}[rr - 1][cc];",
        f"lv = lv + {v}[rr][cc + 1];",
        f"lv = lv + {v}[rr][cc - 1];",
        "lv = lv - 4.0f * vc;",
        "const float uvv = (uc * vc) * vc;",
        f"float a = {lit['DU']} * lu;",
        "a = a - uvv;",
        f"a = a + {lit['F']} * (1.0f - uc);",
        f"float b = {lit['DV']} * lv;",
        "b = b + uvv;",
        f"b = b - {lit['FK']} * vc;",
        f"{dst_u} = uc + {lit['DT']} * a;",
        f"{dst_v} = vc + {lit['DT']} * b;",
    ]


def fused_source(n: int, k: int, th: int, tw: int, du: float, dv: float, f: float, fk: float, dt: float,
                 single_buffer: bool = False) -> str:
    """HIP source of a K-step Gray-Scott pass over an n x n periodic grid,
    one (th x tw) output tile per 256-lane workgroup. With `single_buffer`
    each step computes its cells into registers, waits, and writes them back
    over the same LDS buffer (half the LDS, one more barrier per step)."""
    if n % th or n % tw:
        raise ValueError(f"tile {th}x{tw} must divide the grid {n}x{n}")
    if k < 1 or k > min(th, tw) // 2:
        raise ValueError(f"steps per pass {k} out of range for a {th}x{tw} tile")
    r, c = th + 2 * k, tw + 2 * k
    tiles_j = n // tw
    blocks = (n // th) * tiles_j
    per, rem = divmod(blocks, NUM_XCDS)
    lit = {name: format_float(v) for name, v in (("DU", du), ("DV", dv), ("F", f), ("FK", fk), ("DT", dt))}
    nbuf = 1 if single_buffer else 2
    lines = [
        f"// Gray-Scott, {k} steps per pass, {th}x{tw} tiles, {n}x{n} periodic grid.",
        f'extern "C" __global__ void __launch_bounds__({WORKGROUP})',
        "gray_scott_fused(const float* __restrict__ u_in, const float* __restrict__ v_in,",
        "                 float* __restrict__ u_out, float* __restrict__ v_out)",
        "{",
    ]
    for bi in range(nbuf):
        lines.append(f"    __shared__ float su{bi}[{r}][{c}];")
        lines.append(f"    __shared__ float sv{bi}[{r}][{c}];")
    lines += [
        "    /* XCD k (workgroups k, k + 8, ...) takes a contiguous range of tiles, so",
        "       tiles sharing halo rows share an L2. */",
        f"    const unsigned int xcd = blockIdx.x % {NUM_XCDS}u, slot = blockIdx.x / {NUM_XCDS}u;",
        f"    const unsigned int blk = (xcd < {rem}u) ? xcd * {per + 1}u + slot",
        f"                                           : {rem * (per + 1)}u + (xcd - {rem}u) * {per}u + slot;",
        f"    const int i0 = (int)(blk / {tiles_j}u) * {th};",
        f"    const int j0 = (int)(blk % {tiles_j}u) * {tw};",
        "    const int tid = (int)threadIdx.x;",
        f"    /* Stage the tile and a {k}-cell halo, wrapping around the grid. */",
        f"    for (int idx = tid; idx < {r * c}; idx += {WORKGROUP}) {{",
        f"        const int rr = idx / {c}, cc = idx % {c};",
        f"        int gi = i0 - {k} + rr, gj = j0 - {k} + cc;",
        f"        gi = gi < 0 ? gi + {n} : (gi >= {n} ? gi - {n} : gi);",
        f"        gj = gj < 0 ? gj + {n} : (gj >= {n} ? gj - {n} : gj);",
        f"        su0[rr][cc] = u_in[gi * {n} + gj];",
        f"        sv0[rr][cc] = v_in[gi * {n} + gj];",
        "    }",
        "    __syncthreads();",
    ]
    for st in range(1, k + 1):
        h, w = r - 2 * st, c - 2 * st
        cells = h * w
        per_thread = -(-cells // WORKGROUP)
        src = 0 if single_buffer else (st - 1) % 2
        dst = 0 if single_buffer else st % 2
        lines.append(f"    /* step {st}: rows [{st}, {r - st}), cols [{st}, {c - st}) */")
        if single_buffer:
            lines.append(f"    float nu{st}[{per_thread}], nv{st}[{per_thread}];")
            lines.append("    #pragma unroll")
            lines.append(f"    for (int q = 0; q < {per_thread}; ++q) {{")
            lines.append(f"        const int idx = tid + q * {WORKGROUP};")
            lines.append(f"        if (idx < {cells}) {{")
            lines.append(f"            const int rr = {st} + idx / {w}, cc = {st} + idx % {w};")
            lines += ["            " + x for x in _update(str(src), f"nu{st}[q]", f"nv{st}[q]", lit)]
            lines.append("        }")
            lines.append("    }")
            lines.append("    __syncthreads();")
            lines.append("    #pragma unroll")
            lines.append(f"    for (int q = 0; q < {per_thread}; ++q) {{")
            lines.append(f"        const int idx = tid + q * {WORKGROUP};")
            lines.append(f"        if (idx < {cells}) {{")
            lines.append(f"            const int rr = {st} + idx / {w}, cc = {st} + idx % {w};")
            lines.append(f"            su0[rr][cc] = nu{st}[q];")
            lines.append(f"            sv0[rr][cc] = nv{st}[q];")
            lines.append("        }")
            lines.append("    }")
        else:
            lines.append(f"    for (int idx = tid; idx < {cells}; idx += {WORKGROUP}) {{")
            lines.append(f"        const int rr = {st} + idx / {w}, cc = {st} + idx % {w};")
            lines += ["        " + x for x in _update(str(src), f"su{dst}[rr][cc]", f"sv{dst}[rr][cc]", lit)]
            lines.append("    }")
        lines.append("    __syncthreads();")
    fin = 0 if single_buffer else k % 2
    lines += [
        f"    /* The tile, {k} steps on. */",
        f"    for (int idx = tid; idx < {th * tw}; idx += {WORKGROUP}) {{",
        f"        const int rr = idx / {tw}, cc = idx % {tw};",
        f"        const int g = (i0 + rr) * {n} + j0 + cc;",
        f"        u_out[g] = su{fin}[{k} + rr][{k} + cc];",
        f"        v_out[g] = sv{fin}[{k} + rr][{k} + cc];",
        "    }",
        "}",
        "",
    ]
    return "\n".join(lines)


@dataclasses.dataclass
class FusedGrayScott:
    """A compiled K-step pass (and, for step counts K does not divide, a
    one-step pass of the same code). The defaults (4 steps per pass, 32 x 64
    tiles, one LDS buffer) measured fastest on MI355X at 4096^2 among 1-8
    steps per pass, 8-64 x 64-256 tiles and one or two buffers."""

    n: int
    k: int = 4
    th: int = 32
    tw: int = 64
    math_mode: Any = "fast"
    cfg: Any = None
    single_buffer: bool = True

    def __post_init__(self) -> None:
        from palladium_amd.workloads import GS_CFG

        cfg = self.cfg or GS_CFG
        consts = (float(np.float32(cfg.du)), float(np.float32(cfg.dv)), float(np.float32(cfg.f)),
                  float(np.float32(cfg.f + cfg.k)), float(np.float32(cfg.dt)))
        self._src = {kk: fused_source(self.n, kk, self.th, self.tw, *consts, single_buffer=self.single_buffer)
                     for kk in {self.k, 1}}
        self._kernels = {kk: rt.Kernel(src, "gray_scott_fused", self.math_mode) for kk, src in self._src.items()}
        self.blocks = (self.n // self.th) * (self.n // self.tw)

    def source(self, k: int | None = None) -> str:
        return self._src[k or self.k]

    def launches(self, steps: int) -> list[int]:
        return [self.k] * (steps // self.k) + [1] * (steps % self.k)


def gray_scott_fused_run(fused: FusedGrayScott, u0: np.ndarray, v0: np.ndarray, steps: int, graph: bool = True):
    """`steps` Gray-Scott steps in passes of `fused.k`, ping-ponging two
    buffer pairs, queued as one batch (one HIP graph when `graph`).
    Returns (u, v, device seconds)."""
    if u0.shape != (fused.n, fused.n) or v0.shape != u0.shape:
        raise ValueError(f"fields must be {fused.n}x{fused.n}")
    bufs = [
        [rt.Buffer.from_numpy(np.ascontiguousarray(u0, np.float32)),
         rt.Buffer.from_numpy(np.ascontiguousarray(v0, np.float32))],
        [rt.Buffer.empty(u0.shape, np.float32), rt.Buffer.empty(v0.shape, np.float32)],
    ]
    stream = rt.Stream()
    batch = rt.Batch(stream=stream)
    src = 0
    for kk in fused.launches(steps):
        dst = 1 - src
        batch.add(fused._kernels[kk], fused.blocks, WORKGROUP, [b.ptr for b in bufs[src]] + [b.ptr for b in bufs[dst]])
        src = dst
    batch.commit(graph=graph)
    batch.wait()
    return bufs[src][0].to_numpy(stream), bufs[src][1].to_numpy(stream), batch.gpu_time
