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

__all__ = ["FusedGrayScott", "RegisterGrayScott", "fused_source", "gray_scott_fused_run", "register_source"]

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


WAVE = 64
# DPP controls for a whole-wave rotation by one lane: after `wave_rol:1`
# lane l holds what lane l + 1 held (its right-hand neighbour's column),
# after `wave_ror:1` what lane l - 1 held.
_DPP_FROM_RIGHT = 0x134
_DPP_FROM_LEFT = 0x13C


def _reg_update(lit: dict, up: tuple, mid: tuple, down: tuple, left: tuple, right: tuple, out: tuple,
                tag: str) -> list[str]:
    """One cell of the next step from its column's three rows of this step
    (each a (u, v) pair of register names) and its left and right
    neighbours (expressions: a register of this lane, or one rotated in from
    the neighbouring lane). The op order of `_update`."""
    lines = []
    for i, f in enumerate("uv"):
        lines += [
            f"float l{f}{tag} = {down[i]} + {up[i]};",
            f"l{f}{tag} = l{f}{tag} + {right[i]};",
            f"l{f}{tag} = l{f}{tag} + {left[i]};",
            f"l{f}{tag} = l{f}{tag} - 4.0f * {mid[i]};",
        ]
    uc, vc = mid
    lines += [
        f"const float uvv{tag} = ({uc} * {vc}) * {vc};",
        f"float a{tag} = {lit['DU']} * lu{tag};",
        f"a{tag} = a{tag} - uvv{tag};",
        f"a{tag} = a{tag} + {lit['F']} * (1.0f - {uc});",
        f"float b{tag} = {lit['DV']} * lv{tag};",
        f"b{tag} = b{tag} + uvv{tag};",
        f"b{tag} = b{tag} - {lit['FK']} * {vc};",
        f"const float {out[0]} = {uc} + {lit['DT']} * a{tag};",
        f"const float {out[1]} = {vc} + {lit['DT']} * b{tag};",
    ]
    return lines


def register_geometry(n: int, k: int, rows: int, cols: int = 1) -> tuple[int, int]:
    """(waves, workgroups) of a register pass: one wave per strip of `rows`
    rows by 64 `cols` - 2K columns (the last strip of each kind may reach
    past the grid), four waves per workgroup."""
    waves = -(-n // rows) * -(-n // (WAVE * cols - 2 * k))
    return waves, -(-waves // (WORKGROUP // WAVE))


def register_source(n: int, k: int, rows: int, du: float, dv: float, f: float, fk: float, dt: float,
                    group: int = 8, cols: int = 1) -> str:
    """HIP source of a K-step Gray-Scott pass with no LDS: each wave owns a
    strip of `rows` grid rows by 64 C - 2K columns, C = `cols`. Lane l holds
    strip columns C l .. C l + C - 1 (grid columns j0 - K + those) and walks
    down them from row i0 - K to row i0 + rows + K - 1 (in odd bands of
    strips, up from i0 + rows + K - 1 to i0 - K), one input row at a time.
    For each step t it keeps the last two rows of step t - 1 in registers
    (the up and down neighbours); a column's left and right neighbours are
    the lane's own registers, except at the lane's first and last column,
    whose outer neighbours come from the adjacent lanes through DPP wave
    rotations (so a lane of C columns rotates 2 values per field and step
    where C lanes of one column would rotate 2 C; on gfx950 a DPP add costs
    several plain ones). Input row r yields step-t row r - t, so step K's
    row r - K leaves the pipeline as row r comes in. The outer columns and
    the first rows of each step read values that are not yet (or no longer)
    valid; each step moves that region in by one column and one row per
    side, so after K steps strip columns K .. 64 C - 1 - K and rows
    K .. K + rows - 1 are exact, and only those are stored. Rows come in
    `group` at a time, the next group's loads issued before the current
    group's arithmetic. Row and column indices wrap around the grid, so
    every load is in bounds; the last strip of a row (and of a column) may
    reach past the grid, and its columns (rows) outside it store nothing."""
    w = WAVE * cols - 2 * k
    if cols < 1:
        raise ValueError(f"columns per lane {cols} must be positive")
    if k < 1 or w < 1:
        raise ValueError(f"steps per pass {k} out of range for a {WAVE}-lane wave of {cols} columns per lane")
    if rows < 1:
        raise ValueError(f"strip height {rows} must be positive")
    if n * n * 4 >= 1 << 31:
        raise ValueError(f"grid {n}x{n} exceeds the 2 GiB a buffer descriptor addresses")
    if rows + 2 * k > n or n < WAVE * cols:
        raise ValueError(f"grid {n}x{n} too small for {rows}-row strips with a {k}-row halo "
                         f"(and one {WAVE}-lane wave of {cols} columns per lane)")
    h = rows + 2 * k
    groups = -(-h // group)
    strips_j = -(-n // w)
    waves, blocks = register_geometry(n, k, rows, cols)
    per, rem = divmod(blocks, NUM_XCDS)
    lit = {name: format_float(v) for name, v in (("DU", du), ("DV", dv), ("F", f), ("FK", fk), ("DT", dt))}
    C = cols
    # With K and n multiples of C, a lane's C columns start at a multiple of
    # C: contiguous, aligned, never split by the periodic wrap or an edge of
    # the grid or the strip, so each row moves as one C-wide access.
    vec = C in (2, 4) and k % C == 0 and n % C == 0
    lines = [
        f"// Gray-Scott, {k} steps per pass in registers, {rows}x{w} strips, {C} columns per lane, "
        f"{n}x{n} periodic grid.",
        f"typedef unsigned int ph_u32x{C} __attribute__((ext_vector_type({C})));" if vec else "",
        "#define PH_RSRC_WORD3 0x00020000  /* gfx9 buffer descriptor word 3: 32-bit elements, raw */",
        "#define PH_DROP ((int)0x80000000)  /* an offset past every field: the store is dropped */",
        "static __device__ __forceinline__ float ph_from_right(float x) {",
        f"    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), {_DPP_FROM_RIGHT:#x}, 0xf, 0xf, true));",
        "}",
        "static __device__ __forceinline__ float ph_from_left(float x) {",
        f"    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), {_DPP_FROM_LEFT:#x}, 0xf, 0xf, true));",
        "}",
        f'extern "C" __global__ void __launch_bounds__({WORKGROUP})',
        "gray_scott_regs(const float* __restrict__ u_in, const float* __restrict__ v_in,",
        "                float* __restrict__ u_out, float* __restrict__ v_out)",
        "{",
        f"    const unsigned int xcd = blockIdx.x % {NUM_XCDS}u, slot = blockIdx.x / {NUM_XCDS}u;",
        f"    const unsigned int blk = (xcd < {rem}u) ? xcd * {per + 1}u + slot",
        f"                                           : {rem * (per + 1)}u + (xcd - {rem}u) * {per}u + slot;",
        "    /* The strip, and with it every row index, is the same for all lanes",
        "       of a wave; readfirstlane lets the compiler keep them in scalar",
        "       registers. */",
        f"    const unsigned int strip = __builtin_amdgcn_readfirstlane(blk * {WORKGROUP // WAVE}u + threadIdx.x / {WAVE}u);",
        f"    if (strip >= {waves}u) return;  /* whole waves only */",
        f"    const int lane = (int)(threadIdx.x % {WAVE}u);",
        f"    const int i0 = (int)(strip / {strips_j}u) * {rows};",
        f"    const int j0 = (int)(strip % {strips_j}u) * {w};",
    ]
    for c in range(C):
        sc = f"(lane * {C} + {c})" if C > 1 else "lane"
        lines += [
            f"    int gj{c} = j0 - {k} + {sc};",
            f"    gj{c} = gj{c} < 0 ? gj{c} + {n} : (gj{c} >= {n} ? gj{c} - {n} : gj{c});",
            f"    const bool owner{c} = {sc} >= {k} && {sc} < {WAVE * C - k} && j0 + {sc} - {k} < {n};",
        ]
    lines += [
        "    /* Memory goes through buffer descriptors. A lane's column offset is",
        "       fixed for the whole walk (vector register); the row is a scalar",
        "       offset (loads) or the base of a per-row descriptor (stores), so",
        "       no per-row address arithmetic runs on the VALU. A column that must",
        "       not be stored has an offset past the end and a row that must not",
        "       be stored a descriptor of no bytes: the hardware drops those",
        "       stores, so no branch separates the stores from the loads (a",
        "       branch would make the wait for each group's loads drain the",
        "       previous group's stores). */",
        f"    const __amdgpu_buffer_rsrc_t u_src = __builtin_amdgcn_make_buffer_rsrc((void*)u_in, (short)0, {n * n * 4}, PH_RSRC_WORD3);",
        f"    const __amdgpu_buffer_rsrc_t v_src = __builtin_amdgcn_make_buffer_rsrc((void*)v_in, (short)0, {n * n * 4}, PH_RSRC_WORD3);",
    ]
    for c in (range(1) if vec else range(C)):
        sc = f"(lane * {C} + {c})" if C > 1 else "lane"
        lines += [
            f"    const int lo{c} = gj{c} * 4;  /* load column offset */",
            f"    const int so{c} = owner{c} ? (j0 + {sc} - {k}) * 4 : PH_DROP;  /* store column offset */",
        ]
    lines += [
        "    /* Odd bands of strips walk up, even ones down: a band's last halo rows",
        "       are then read at about the time the next band reads them too, which",
        "       keeps them in L2. Pipeline row p is grid row (base + dir * p) % n. */",
        f"    const bool up = ((strip / {strips_j}u) & 1u) != 0u;",
        f"    const int base = up ? i0 + {rows - 1 + k + n} : i0 + {n - k};",
        "    const int dir = up ? -1 : 1;",
        "    float " + ", ".join(f"pu{t}_{i}_{c} = 0.0f, pv{t}_{i}_{c} = 0.0f"
                                for t in range(k) for i in (1, 2) for c in range(C)) + ";",
    ]
    vt = f"float{C}" if vec else None
    comps = "xyzw"

    def load_row(dst_u: str, dst_v: str, gi: str, decl: str) -> list[str]:
        """Lines loading grid row `gi` of this lane's columns into dst_u{c}, dst_v{c}."""
        row = f"({gi}) * {4 * n}"
        if vec:
            out = [f"{{ const ph_u32x{C} _u = __builtin_amdgcn_raw_buffer_load_b{32 * C}(u_src, lo0, {row}, 0), "
                   f"_v = __builtin_amdgcn_raw_buffer_load_b{32 * C}(v_src, lo0, {row}, 0);"]
            out += [f"  {dst_u}{c} = __uint_as_float(_u.{comps[c]}); {dst_v}{c} = __uint_as_float(_v.{comps[c]});"
                    for c in range(C)]
            return out + ["}"]
        return [" ".join(f"{dst_u}{c} = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(u_src, lo{c}, {row}, 0)); "
                         f"{dst_v}{c} = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(v_src, lo{c}, {row}, 0));"
                         for c in range(C))]

    for g in range(group):
        lines.append(f"    float " + ", ".join(f"qu{g}_{c}, qv{g}_{c}" for c in range(C)) + ";")
        lines.append(f"    {{ const int gi = (int)((unsigned int)(base + dir * {min(g, h - 1)}) % {n}u);")
        lines += ["        " + x for x in load_row(f"qu{g}_", f"qv{g}_", "gi", "")]
        lines.append("    }")
    lines += [f"    for (int r0 = 0; r0 < {groups * group}; r0 += {group}) {{"]
    # The next group's loads are unconditional (past the strip's end they
    # read its last row again, a cache hit): behind a branch, the wait for
    # this group's rows would also wait for the first of them.
    for g in range(group):
        lines.append(f"        const int p{g} = r0 + {group + g} < {h - 1} ? r0 + {group + g} : {h - 1};")
        lines.append(f"        const int gi{g} = (int)((unsigned int)(base + dir * p{g}) % {n}u);")
        lines.append("        float " + ", ".join(f"nu{g}_{c}, nv{g}_{c}" for c in range(C)) + ";")
        lines += ["        " + x for x in load_row(f"nu{g}_", f"nv{g}_", f"gi{g}", "")]
    for g in range(group):
        lines.append(f"        {{ /* input row r0 + {g} */")
        cur = [(f"qu{g}_{c}", f"qv{g}_{c}") for c in range(C)]
        for t in range(k):
            mid = [(f"pu{t}_1_{c}", f"pv{t}_1_{c}") for c in range(C)]
            # the outer neighbours of the lane's edge columns, one rotation each
            lines.append(f"            const float ru{g}_{t} = ph_from_right({mid[0][0]}), "
                         f"rv{g}_{t} = ph_from_right({mid[0][1]});")
            lines.append(f"            const float lu{g}_{t}_ = ph_from_left({mid[C - 1][0]}), "
                         f"lv{g}_{t}_ = ph_from_left({mid[C - 1][1]});")
            outs = []
            for c in range(C):
                left = mid[c - 1] if c > 0 else (f"lu{g}_{t}_", f"lv{g}_{t}_")
                right = mid[c + 1] if c < C - 1 else (f"ru{g}_{t}", f"rv{g}_{t}")
                out = (f"yu{g}_{t}_{c}", f"yv{g}_{t}_{c}")
                lines += ["            " + x for x in _reg_update(lit, (f"pu{t}_2_{c}", f"pv{t}_2_{c}"), mid[c],
                                                                  cur[c], left, right, out, f"{g}_{t}_{c}")]
                outs.append(out)
            for c in range(C):
                lines.append(f"            pu{t}_2_{c} = pu{t}_1_{c}; pv{t}_2_{c} = pv{t}_1_{c}; "
                             f"pu{t}_1_{c} = {cur[c][0]}; pv{t}_1_{c} = {cur[c][1]};")
            cur = outs
        lines.append(f"            const int a = r0 + {g} - {2 * k};  /* output row, strip-relative */")
        lines.append(f"            const int ga = up ? i0 + {rows - 1} - a : i0 + a;  /* its grid row */")
        lines.append(f"            const bool row_kept = a >= 0 && a < {rows} && ga < {n};")
        lines.append(f"            const int row_at = row_kept ? ga * {n} : 0;")
        lines.append(f"            const int row_bytes = row_kept ? {4 * n} : 0;")
        lines.append("            const __amdgpu_buffer_rsrc_t u_row = __builtin_amdgcn_make_buffer_rsrc("
                     "u_out + row_at, (short)0, row_bytes, PH_RSRC_WORD3);")
        lines.append("            const __amdgpu_buffer_rsrc_t v_row = __builtin_amdgcn_make_buffer_rsrc("
                     "v_out + row_at, (short)0, row_bytes, PH_RSRC_WORD3);")
        if vec:
            # one owner flag for the lane: its columns are all in or all out
            for i, rs in ((0, "u_row"), (1, "v_row")):
                vals = ", ".join(f"__float_as_uint({cur[c][i]})" for c in range(C))
                lines.append(f"            __builtin_amdgcn_raw_buffer_store_b{32 * C}((ph_u32x{C}){{{vals}}}, {rs}, so0, 0, 0);")
        else:
            for c in range(C):
                lines.append(f"            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint({cur[c][0]}), u_row, so{c}, 0, 0);")
                lines.append(f"            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint({cur[c][1]}), v_row, so{c}, 0, 0);")
        lines.append("        }")
    for g in range(group):
        lines.append("        " + " ".join(f"qu{g}_{c} = nu{g}_{c}; qv{g}_{c} = nv{g}_{c};" for c in range(C)))
    lines += ["    }", "}", ""]
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
        consts = _consts(self.cfg)
        self._src = {kk: fused_source(self.n, kk, self.th, self.tw, *consts, single_buffer=self.single_buffer)
                     for kk in {self.k, 1}}
        self._kernels = {kk: rt.Kernel(src, "gray_scott_fused", self.math_mode) for kk, src in self._src.items()}
        self.blocks = (self.n // self.th) * (self.n // self.tw)

    def blocks_for(self, k: int) -> int:
        return self.blocks

    def describe(self) -> str:
        return f"LDS pass: {self.th}x{self.tw} tiles, {'one buffer' if self.single_buffer else 'two buffers'}"

    def source(self, k: int | None = None) -> str:
        return self._src[k or self.k]

    def launches(self, steps: int) -> list[int]:
        return [self.k] * (steps // self.k) + [1] * (steps % self.k)


def _consts(cfg: Any) -> tuple:
    from palladium_amd.workloads import GS_CFG

    cfg = cfg or GS_CFG
    return (float(np.float32(cfg.du)), float(np.float32(cfg.dv)), float(np.float32(cfg.f)),
            float(np.float32(cfg.f + cfg.k)), float(np.float32(cfg.dt)))


@dataclasses.dataclass
class RegisterGrayScott:
    """A compiled K-step register pass (`register_source`) and a one-step
    pass of the same code for step counts K does not divide."""

    n: int
    k: int = 6
    rows: int = 64
    group: int = 4
    math_mode: Any = "fast"
    cfg: Any = None
    cols: int = 1

    def __post_init__(self) -> None:
        consts = _consts(self.cfg)
        self._src = {kk: register_source(self.n, kk, self.rows, *consts, group=self.group, cols=self.cols)
                     for kk in {self.k, 1}}
        self._kernels = {kk: rt.Kernel(src, "gray_scott_regs", self.math_mode) for kk, src in self._src.items()}
        self._blocks = {kk: register_geometry(self.n, kk, self.rows, self.cols)[1] for kk in self._src}

    def blocks_for(self, k: int) -> int:
        return self._blocks[k]

    def describe(self) -> str:
        return (f"register pass: {self.rows}x{WAVE * self.cols - 2 * self.k} strips, one wave each, "
                f"{self.cols} column(s) per lane, rows in groups of {self.group}")

    def source(self, k: int | None = None) -> str:
        return self._src[k or self.k]

    def launches(self, steps: int) -> list[int]:
        return [self.k] * (steps // self.k) + [1] * (steps % self.k)


def gray_scott_fused_run(fused: FusedGrayScott | RegisterGrayScott, u0: np.ndarray, v0: np.ndarray, steps: int, graph: bool = True):
    """`steps` Gray-Scott steps in passes of `fused.k`, ping-ponging two
    buffer pairs, queued as one batch (one HIP graph when `graph`).
    Returns (u, v, device seconds)."""
    if u0.shape != (fused.n, fused.n) or v0.shape != u0.shape:
        raise ValueError(f"fields must be {fused.n}x{fused.n}")
    if steps < 0:
        raise ValueError(f"steps must be non-negative, got {steps}")
    if steps == 0:
        return np.array(u0, np.float32), np.array(v0, np.float32), 0.0
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
        batch.add(fused._kernels[kk], fused.blocks_for(kk), WORKGROUP, [b.ptr for b in bufs[src]] + [b.ptr for b in bufs[dst]])
        src = dst
    batch.commit(graph=graph)
    batch.wait()
    return bufs[src][0].to_numpy(stream), bufs[src][1].to_numpy(stream), batch.gpu_time
