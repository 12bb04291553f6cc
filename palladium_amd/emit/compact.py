"""Workgroup lane compaction for divergent `while_loop`s.

An adaptive solver's per-lane `while_loop` keeps a wavefront issuing until
its slowest lane finishes; on config 2 (Van der Pol, mu log-uniform) half
the lane-attempts of a wavefront do no work. When a kernel's loop runs one
program instance per lane with nothing lane-specific inside it, the
instance is only its loop state: the carries and the loop's operands. Then
the state of a live instance can move to another lane, and a 1,024-lane
workgroup can repack its live instances into its lowest wavefronts every
`EPOCH` iterations, so emptied wavefronts stop issuing:

    epoch:  run up to EPOCH predicated iterations (a wavefront leaves the
            epoch early once none of its lanes is live);
            lanes whose instance finished store its carries in LDS at the
            instance's own slot;
            count the live lanes per wavefront (ballot, popcount);
            if packing frees a wavefront, live lanes write their state to
            LDS at their rank among the live (prefix over wavefronts +
            mbcnt) and lanes [0, live) read it back;
            stop when no lane of the workgroup is live.
    after:  every lane reloads its own instance's final carries.

Each instance runs exactly the operations it ran before, in the same
order: results are bit-identical with and without compaction. Wavefront w
of a 1,024-lane workgroup shares its SIMD with w ± 4, w ± 8 ... (measured
on MI355X: consecutive wavefronts land on the CU's four SIMDs in turn), so
packing into the lowest wavefronts keeps the four SIMDs evenly loaded.

The control flow around each barrier is uniform over the workgroup (the
epoch loop stops on a count read from LDS), and no lane returns early (a
grid that does not fill its last workgroup keeps the extra lanes, which
hold no instance), so every wavefront meets every barrier.
"""

from __future__ import annotations

import dataclasses
import os
from typing import Any

import numpy as np

from palladium_amd.ir import KeyAval

WORKGROUP = 1024
EPOCH = 64
# Loop iterations per pass of the epoch loop (see emit_compacting_while), by
# math mode. More iterations per pass spread the pass's counter and branch
# over more attempts; SAFE's deterministic pow makes its iteration about 2.5
# times FAST's code, and past 16 of them its loop no longer fits the
# instruction cache two CUs share (64 KiB). Measured on BS3: FAST 0.698 /
# 0.690 / 0.673 / 0.667 / 0.659 / 0.652 ms at 1 / 2 / 4 / 8 / 16 / 32, SAFE
# 2.14 / 2.13 / 2.10 / 2.08 / 2.07 / 2.08, SAFE 2.12 at 64.
EPOCH_UNROLL = {"safe": 16, "other": 32}


# A pass holds at most this many traced operations of the loop body, so that
# a large body is not copied 32 times (code size, compile time).
EPOCH_UNROLL_OPS = 4096


def _count_eqns(j: Any) -> int:
    n = 0
    for e in j.eqns:
        n += 1
        for v in e.params.values():
            for sub in (v if isinstance(v, tuple) else (v,)):
                if hasattr(getattr(sub, "jaxpr", sub), "eqns"):
                    n += _count_eqns(getattr(sub, "jaxpr", sub))
    return n


def iterations_per_pass(hip_source: str) -> int:
    """The iterations per machine-loop pass the emitter chose for a
    compacted while loop in `hip_source` (1 if it has none)."""
    import re

    m = re.search(r"// (\d+) iterations per pass", hip_source)
    return int(m.group(1)) if m else 1


def epoch_unroll(math_mode: Any = None, body: Any = None) -> int:
    """Iterations of a compacted while loop per pass of its machine loop:
    the math mode's default, halved until the pass holds at most
    EPOCH_UNROLL_OPS of `body`'s operations (`PALLADIUM_EPOCH_UNROLL`
    overrides both)."""
    from palladium_amd.runtime import math_mode_ordinal

    raw = os.environ.get("PALLADIUM_EPOCH_UNROLL")
    if raw is not None:
        u = int(raw)
        if u < 1 or EPOCH % u:
            raise ValueError(f"PALLADIUM_EPOCH_UNROLL={u} must divide the epoch of {EPOCH} iterations")
        return u
    safe = math_mode is None or math_mode_ordinal(math_mode) in (0, 3)
    u = EPOCH_UNROLL["safe" if safe else "other"]
    n = _count_eqns(getattr(body, "jaxpr", body)) if body is not None else 0
    while u > 1 and u * n > EPOCH_UNROLL_OPS:
        u //= 2
    return u
# LDS per workgroup the compaction may use (2 workgroups per CU fit in 160 KB).
LDS_BUDGET = 78 * 1024

_LANE_SPECIFIC = {"program_id", "num_programs", "get", "swap", "lane_index", "lane_reduce", "while"}
# dtype -> 32-bit LDS words per value
_STORABLE = {"float32": 1, "int32": 1, "uint32": 1, "bool": 1, "float64": 2}


@dataclasses.dataclass(frozen=True)
class CompactPlan:
    index: int  # position of the loop among the top-level eqns


def _jaxpr(j: Any) -> Any:
    return getattr(j, "jaxpr", j)


def _lane_free(jaxpr: Any) -> bool:
    for e in _jaxpr(jaxpr).eqns:
        if e.primitive.name in _LANE_SPECIFIC:
            return False
        for v in e.params.values():
            for sub in (v if isinstance(v, tuple) else (v,)):
                if hasattr(_jaxpr(sub), "eqns") and not _lane_free(sub):
                    return False
    return True


def _storable(v: Any) -> bool:
    aval = getattr(v, "aval", None)
    if aval is None or isinstance(aval, KeyAval):
        return False
    if int(np.prod(aval.shape)) != 1:
        return False
    return np.dtype(aval.dtype).name in _STORABLE


def enabled() -> bool:
    return os.environ.get("PALLADIUM_WHILE_COMPACTION", "1") != "0"


def plan_for(spec: Any, jaxpr: Any, lanes: int, block: int | None) -> CompactPlan | None:
    """The loop to compact, or None. Needs: one lane per instance, a 1-D
    grid, no explicit workgroup size other than 1,024, and exactly one
    top-level `while` whose condition and body touch no ref, program id or
    nested while, with scalar 4-byte-or-bool carries and operands. A grid
    that does not fill whole workgroups keeps its extra lanes: they read
    the last instance's data, never enter the loop and store nothing."""
    if not enabled() or lanes != 1 or len(spec.grid) != 1:
        return None
    if block not in (None, WORKGROUP):
        return None
    whiles = [k for k, e in enumerate(jaxpr.eqns) if e.primitive.name == "while"]
    if len(whiles) != 1:
        return None
    e = jaxpr.eqns[whiles[0]]
    if getattr(e.params["cond_jaxpr"], "consts", None) or getattr(e.params["body_jaxpr"], "consts", None):
        return None
    if not (_lane_free(e.params["cond_jaxpr"]) and _lane_free(e.params["body_jaxpr"])):
        return None
    if not all(_storable(v) for v in list(e.invars) + list(e.outvars)):
        return None
    used = {v for x in jaxpr.eqns for v in x.invars} | set(jaxpr.outvars)
    n_state = sum(_nwords(v) for v in e.invars) + 1  # operands and carries, plus the slot index
    n_kept = sum(_nwords(v) for v in e.outvars if v in used)  # final carries read after the loop
    if (n_state + n_kept) * WORKGROUP * 4 > LDS_BUDGET:
        return None
    return CompactPlan(whiles[0])


def _nwords(v: Any) -> int:
    return _STORABLE[np.dtype(v.aval.dtype).name]


def _store(arr: str, j: int, pos: str, c: Any) -> tuple[list[str], int]:
    """Lines writing value `c` to rows j, j+1, ... of LDS array `arr` at
    column `pos`, and the next free row."""
    e, t = c.expr, c.ctype
    if t == "double":
        bits = f"(unsigned long long)__double_as_longlong({e})"
        return [f"{arr}[{j}][{pos}] = (unsigned int)({bits});",
                f"{arr}[{j + 1}][{pos}] = (unsigned int)(({bits}) >> 32);"], j + 2
    if t == "float":
        word = f"__float_as_uint({e})"
    elif t == "bool":
        word = f"({e} ? 1u : 0u)"
    else:
        word = f"(unsigned int)({e})"
    return [f"{arr}[{j}][{pos}] = {word};"], j + 1


def _load(arr: str, j: int, pos: str, c: Any) -> tuple[str, int]:
    """The line reading `c` back from rows j, ... of `arr`, and the next row."""
    e, t = c.expr, c.ctype
    if t == "double":
        return (f"{e} = __longlong_as_double((long long)(((unsigned long long){arr}[{j + 1}][{pos}] << 32)"
                f" | (unsigned long long){arr}[{j}][{pos}]));"), j + 2
    w = f"{arr}[{j}][{pos}]"
    if t == "float":
        return f"{e} = __uint_as_float({w});", j + 1
    if t == "bool":
        return f"{e} = ({w} != 0u);", j + 1
    return f"{e} = ({t})({w});", j + 1


def _rows(vals: list) -> int:
    return sum(2 if c.ctype == "double" else 1 for c in vals)


def emit_compacting_while(env: Any, cursor: Any, eqn: Any, emit_jaxpr: Any, declare_carries: Any,
                          copy_back: Any) -> None:
    """Emit `eqn` (a top-level `while`) with workgroup lane compaction."""
    cn = int(eqn.params["cond_nconsts"])
    bn = int(eqn.params["body_nconsts"])
    cj = _jaxpr(eqn.params["cond_jaxpr"])
    bj = _jaxpr(eqn.params["body_jaxpr"])
    # The loop's operands move with their instance: private copies.
    consts = []
    for v in eqn.invars[: cn + bn]:
        src = env.val(v)
        name = cursor.fresh("_k")
        cursor.emit(f"{src.ctype} {name} = {src.at('0')};")
        consts.append(dataclasses.replace(src, expr=name, space="local", readonly=False))
    cond_consts, body_consts = consts[:cn], consts[cn:]
    carries = declare_carries(env, cursor, eqn.invars[cn + bn:], eqn.outvars)
    state = consts + carries
    kept = [(k, c) for k, (c, ov) in enumerate(zip(carries, eqn.outvars)) if env.used(ov)]
    nw = WORKGROUP // 64
    buf, res, cnt = cursor.fresh("_cbuf"), cursor.fresh("_cres"), cursor.fresh("_ccnt")
    n_rows, kept_vals = _rows(state), [c for _, c in kept]
    cursor.emit(f"__shared__ unsigned int {buf}[{n_rows + 1}][{WORKGROUP}];")
    if kept:
        cursor.emit(f"__shared__ unsigned int {res}[{_rows(kept_vals)}][{WORKGROUP}];")
    cursor.emit(f"__shared__ int {cnt}[{nw}];")
    slot, own = cursor.fresh("_slot"), cursor.fresh("_own")
    first = f"(_in ? (int)threadIdx.x : -1)" if getattr(env, "compact_in", None) else "(int)threadIdx.x"
    cursor.emit(f"int {slot} = {first};  // the instance this lane holds; -1: none")
    wave = cursor.fresh("_wv")
    cursor.emit(f"const int {wave} = (int)(threadIdx.x >> 6);")
    with cursor.block("while (true)"):
        ep = cursor.fresh("_ep")
        unroll = epoch_unroll(getattr(env, "math_mode", None), bj)
        cursor.emit(f"// {unroll} iterations per pass")
        from palladium_amd.emit.rules import select_guards

        # `unroll` iterations per pass, each with its own exit test (a break
        # in any of them leaves the epoch): the pass's counter and branch are
        # shared among them.
        with cursor.block(f"for (int {ep} = 0; {ep} < {EPOCH}; {ep} += {unroll})"):
            for _ in range(unroll):
                (pred,) = emit_jaxpr(env, cursor, cj, cond_consts + carries)
                live = cursor.fresh("_live")
                cursor.emit(f"const bool {live} = ({pred.at('0')}) && {slot} >= 0;")
                with cursor.block(f"if (!__any({live}))"):
                    cursor.emit("break;")
                outs = emit_jaxpr(env, cursor, bj, body_consts + carries)
                copy_back(cursor, outs, carries, predicate=live, guards=select_guards(env, bj, bn))
        # Epoch boundary: the same condition, on the state as it stands.
        (pred,) = emit_jaxpr(env, cursor, cj, cond_consts + carries)
        cursor.emit(f"bool {own} = ({pred.at('0')}) && {slot} >= 0;")
        with cursor.block(f"if (!{own} && {slot} >= 0)"):
            j = 0
            for c in kept_vals:
                lines, j = _store(res, j, slot, c)
                for line in lines:
                    cursor.emit(line)
            cursor.emit(f"{slot} = -1;")
        mask, total, before, active = (cursor.fresh(p) for p in ("_cm", "_ctot", "_cbef", "_cact"))
        cursor.emit(f"const unsigned long long {mask} = __ballot({own});")
        with cursor.block("if ((threadIdx.x & 63u) == 0u)"):
            cursor.emit(f"{cnt}[{wave}] = (int)__popcll({mask});")
        cursor.emit("__syncthreads();")
        cursor.emit(f"int {total} = 0, {before} = 0, {active} = 0;")
        w = cursor.fresh("_cw")
        with cursor.block(f"for (int {w} = 0; {w} < {nw}; ++{w})"):
            cursor.emit(f"const int _c = {cnt}[{w}];")
            cursor.emit(f"{total} += _c; {before} += ({w} < {wave}) ? _c : 0; {active} += (_c > 0) ? 1 : 0;")
        with cursor.block(f"if ({total} == 0)"):
            cursor.emit("break;")
        # Repack only when it frees a wavefront (the decision is uniform).
        with cursor.block(f"if (({total} + 63) / 64 < {active})"):
            with cursor.block(f"if ({own})"):
                pos = cursor.fresh("_cpos")
                cursor.emit(f"const int {pos} = {before} + (int)__builtin_amdgcn_mbcnt_hi("
                            f"(unsigned int)({mask} >> 32), __builtin_amdgcn_mbcnt_lo((unsigned int){mask}, 0u));")
                j = 0
                for c in state:
                    lines, j = _store(buf, j, pos, c)
                    for line in lines:
                        cursor.emit(line)
                cursor.emit(f"{buf}[{n_rows}][{pos}] = (unsigned int){slot};")
            cursor.emit("__syncthreads();")
            with cursor.block(f"if ((int)threadIdx.x < {total})"):
                j = 0
                for c in state:
                    line, j = _load(buf, j, "threadIdx.x", c)
                    cursor.emit(line)
                cursor.emit(f"{slot} = (int){buf}[{n_rows}][threadIdx.x];")
            with cursor.block("else"):
                cursor.emit(f"{slot} = -1;")
        # Nothing is written to LDS again before every lane has read.
        cursor.emit("__syncthreads();")
    # Every instance has finished: each lane takes its own back.
    j = 0
    for c in kept_vals:
        line, j = _load(res, j, "threadIdx.x", c)
        cursor.emit(line)
