"""Loop-body latency model over a kernel's own gfx950 machine code.

For a latency-bound loop (one adaptive attempt per iteration, each
depending on the step size the previous one chose) the useful bound is not
an instruction-throughput peak but the time one wavefront needs to run one
iteration alone: it issues in program order, and an instruction waits for
the results it reads. `loop_model` reads the disassembly of a code object
(made here by hiprtc, disassembled with ROCm's llvm-objdump), takes the
body of the hot loop (between a backward branch and its target), and
replays it for several iterations under that in-order model:

    start(i) = max(start(i-1) + issue, ready(operands of i))
    ready(results of i) = start(i) + latency(class of i)

with per-class latencies measured on the device (dependent chains of
`v_fma_f32` and of the transcendental unit) and the issue interval of one
wavefront running independent instructions. The cycles per iteration in
the steady state are the chain bound; it is a lower bound for a
wavefront that shares its SIMD with others.
"""

from __future__ import annotations

import dataclasses
import os
import re
import subprocess
import tempfile

__all__ = ["Instr", "LoopModel", "disassemble", "issue_slots", "loop_body", "loop_model", "parse"]

OBJDUMP = os.environ.get("PALLADIUM_OBJDUMP", "/opt/rocm/llvm/bin/llvm-objdump")

TRANSCENDENTAL = ("v_exp_", "v_log_", "v_rcp_", "v_rsq_", "v_sqrt_", "v_sin_", "v_cos_")
_NO_RESULT = ("s_waitcnt", "s_nop", "s_branch", "s_cbranch", "s_endpgm", "s_barrier", "s_setprio",
              "global_store", "buffer_store", "flat_store", "ds_write", "scratch_store")


@dataclasses.dataclass(frozen=True)
class Instr:
    addr: int
    op: str
    dst: tuple[str, ...]
    src: tuple[str, ...]
    target: int | None = None  # branch target address
    imm: int | None = None     # last operand, when it is a plain integer


@dataclasses.dataclass(frozen=True)
class LoopModel:
    instructions: int          # in the loop body
    valu: int
    transcendental: int
    salu: int
    cycles_per_iteration: float  # in units of the latencies given


def disassemble(code: bytes) -> str:
    with tempfile.NamedTemporaryFile(suffix=".co", delete=False) as f:
        f.write(code)
        path = f.name
    try:
        return subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", path], capture_output=True, text=True,
                              check=True).stdout
    finally:
        os.unlink(path)


_LINE = re.compile(r"^\s+([a-z_0-9]+)(?:\s+([^/]*?))?\s*//\s*([0-9A-Fa-f]+):")
_REG = re.compile(r"\b([vs])\[(\d+):(\d+)\]|\b([vs])(\d+)\b|\b(vcc|exec|scc|m0)\b")


def _regs(text: str) -> list[str]:
    out = []
    for m in _REG.finditer(text):
        if m.group(1):
            out += [f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)]
        elif m.group(4):
            out.append(f"{m.group(4)}{m.group(5)}")
        else:
            name = m.group(6)
            out += ["s_vcc_lo", "s_vcc_hi"] if name == "vcc" else [name]
    return out


def parse(asm: str) -> list[Instr]:
    """Instructions of the disassembly, with the registers each writes and
    reads (implicit vcc/scc/exec uses included where the encoding has them)."""
    out: list[Instr] = []
    for line in asm.splitlines():
        m = _LINE.match(line)
        if not m:
            continue
        op, args, addr = m.group(1), (m.group(2) or "").strip(), int(m.group(3), 16)
        target = None
        if op.startswith(("s_branch", "s_cbranch")):
            # `s_branch 65401` is a signed 16-bit dword offset from the next instruction
            try:
                off = int(args.split()[0])
            except (ValueError, IndexError):
                off = 0
            if off >= 32768:
                off -= 65536
            target = addr + 4 + 4 * off
        parts = [p.strip() for p in args.split(",")] if args else []
        dst: list[str] = []
        src: list[str] = []
        if op.startswith(_NO_RESULT) or not parts:
            src = _regs(args)
        else:
            dst = _regs(parts[0])
            src = _regs(",".join(parts[1:]))
            if op.startswith(("v_fmac_", "v_mac_")) or op.startswith("s_and_saveexec") or "saveexec" in op:
                src += dst
        if op.startswith("v_cmp") and op.endswith("_e32"):
            dst, src = ["s_vcc_lo", "s_vcc_hi"], _regs(args)
        if op.startswith(("v_cndmask_b32_e32", "v_addc", "v_subb")) and op.endswith("_e32"):
            src += ["s_vcc_lo", "s_vcc_hi"]
        if op.startswith(("s_cmp", "s_bitcmp")):
            dst, src = ["scc"], _regs(args)
        elif op.startswith("s_") and not op.startswith(("s_waitcnt", "s_nop", "s_branch", "s_cbranch", "s_mov")):
            dst.append("scc")
        if op.startswith(("s_cselect", "s_cbranch_scc", "s_addc", "s_subb")):
            src.append("scc")
        if op.startswith(("v_",)):
            src.append("exec")
        imm = None
        if parts and re.fullmatch(r"-?\d+", parts[-1]):
            imm = int(parts[-1])
        out.append(Instr(addr, op, tuple(dst), tuple(src), target, imm))
    return out


def _hot_trace(instrs: list[Instr], head: int, latch: int, index: dict[int, int]) -> list[Instr] | None:
    """The instructions one iteration of the loop [head, latch] issues when
    every conditional branch falls through (the common path: a wavefront
    skips its rarely-entered cold blocks and stays in the loop) and every
    unconditional branch is followed; None when that path does not come
    back to `latch` (a branch into another loop, or out)."""
    out: list[Instr] = []
    seen: set[int] = set()
    k = head
    while 0 <= k < len(instrs) and k not in seen:
        seen.add(k)
        ins = instrs[k]
        out.append(ins)
        if k == latch:
            return out
        if ins.op == "s_branch" and ins.target is not None:
            nxt = index.get(ins.target)
            if nxt is None:
                return None
            k = nxt
        elif ins.op.startswith(("s_endpgm", "s_setpc")):
            return None
        else:
            k += 1
    return None


def loop_body(instrs: list[Instr]) -> list[Instr]:
    """The hot loop's body: the common path (see `_hot_trace`) of a loop
    whose back-edge that path returns to, so blocks the compiler placed out
    of line for rarely-taken branches, and loops around the hot one, are
    left out. Of several such loops, the shortest holding at least a
    quarter of the vector instructions of the largest. Without any, the
    contiguous span from a backward branch's target to the branch, chosen
    the same way."""
    index = {x.addr: j for j, x in enumerate(instrs)}
    spans = []
    traces = []
    for k, ins in enumerate(instrs):
        if ins.target is not None and ins.target <= ins.addr:
            start = index.get(ins.target)
            if start is None:
                continue
            spans.append((start, k, sum(b.op.startswith("v_") for b in instrs[start:k + 1])))
            tr = _hot_trace(instrs, start, k, index)
            if tr is not None:
                traces.append((tr, sum(b.op.startswith("v_") for b in tr)))
    if traces:
        top = max(t[1] for t in traces)
        return min((t for t in traces if 4 * t[1] >= top), key=lambda t: len(t[0]))[0]
    if not spans:
        raise ValueError("no backward branch: the kernel has no loop")
    top = max(s[2] for s in spans)
    best = min((s for s in spans if 4 * s[2] >= top), key=lambda s: s[1] - s[0])
    return instrs[best[0]:best[1] + 1]


def _latency(op: str, lat_valu: float, lat_trans: float, lat_salu: float) -> float:
    if op.startswith(TRANSCENDENTAL):
        return lat_trans
    if op.startswith("v_"):
        return lat_valu
    if op.startswith(("s_waitcnt", "s_nop", "s_branch", "s_cbranch")):
        return 0.0
    return lat_salu


def loop_model(code_or_asm: bytes | str, lat_valu: float, lat_trans: float, issue: float,
               lat_salu: float | None = None, iterations: int = 16, body_filter=None) -> LoopModel:
    """Cycles (or whatever unit the latencies are in) per iteration of the
    hot loop of a code object, under in-order issue at `issue` per
    instruction with the given result latencies."""
    asm = code_or_asm if isinstance(code_or_asm, str) else disassemble(code_or_asm)
    body = loop_body(parse(asm))
    if body_filter is not None:
        body = [b for b in body if body_filter(b)]
    lat_s = issue if lat_salu is None else lat_salu
    ready: dict[str, float] = {}
    t = 0.0
    marks = []
    for _ in range(iterations):
        for ins in body:
            if ins.op.startswith(("s_waitcnt", "s_nop")):
                continue
            start = max([t] + [ready.get(r, 0.0) for r in ins.src])
            done = start + _latency(ins.op, lat_valu, lat_trans, lat_s)
            for r in ins.dst:
                ready[r] = done
            t = start + issue
        marks.append(max([t] + list(ready.values())))
    half = iterations // 2
    per = (marks[-1] - marks[half - 1]) / (iterations - half)
    ops = [b.op for b in body]
    return LoopModel(
        instructions=len(body),
        valu=sum(o.startswith("v_") for o in ops),
        transcendental=sum(o.startswith(TRANSCENDENTAL) for o in ops),
        salu=sum(o.startswith("s_") for o in ops),
        cycles_per_iteration=per,
    )


# Three-input integer VALU forms priced like v_add3_u32 when no probe of
# their own exists.
_VOP3_INT = ("v_add3_", "v_xad_", "v_lshl_add_", "v_add_lshl_", "v_lshl_or_", "v_and_or_", "v_or3_", "v_xor3_")


def issue_slots(code_or_asm: bytes | str, costs: dict[str, float],
                per_machine_iteration: bool = False) -> tuple[float, dict[str, int]]:
    """FMA-equivalent issue slots of one iteration of the hot loop: each
    vector instruction weighted by its measured cost relative to
    v_fma_f32 (`costs`, keyed by mnemonic without encoding suffix, e.g.
    "v_alignbit_b32", "v_exp_f32"); transcendentals without a probe cost
    what v_exp_f32 does, three-input integer forms what v_add3_u32 does,
    every other vector instruction 1. Scalar instructions are not counted
    (they issue beside vector ones from other wavefronts). Returns the
    slots and the instruction histogram, both per source iteration (a
    machine loop unrolled k times is divided by k), or per pass of the
    machine loop with `per_machine_iteration` (for a loop whose induction
    step is not a count of source iterations)."""
    asm = code_or_asm if isinstance(code_or_asm, str) else disassemble(code_or_asm)
    body = loop_body(parse(asm))
    hist: dict[str, int] = {}
    slots = 0.0
    for ins in body:
        if not ins.op.startswith("v_"):
            continue
        hist[ins.op] = hist.get(ins.op, 0) + 1
        base = re.sub(r"_e(32|64)$", "", ins.op)
        if base in costs:
            slots += costs[base]
        elif ins.op.startswith(TRANSCENDENTAL):
            slots += costs.get("v_exp_f32", 1.0)
        elif ins.op.startswith(_VOP3_INT):
            slots += costs.get("v_add3_u32", 1.0)
        else:
            slots += 1.0
    unroll = 1 if per_machine_iteration else unroll_factor(body)
    return slots / unroll, {k: v / unroll for k, v in hist.items()}


_IND = re.compile(r"^\s*(s_add_i32|s_sub_i32|s_add_u32|s_sub_u32)\s+(s\d+), (s\d+), (-?\d+)\s*//")


def unroll_factor(body: list[Instr], asm_lines: list[str] | None = None) -> int:
    """How many source iterations one pass of the machine loop covers: the
    step of its scalar induction update (`s_add_i32 sN, sN, -4` after
    four-fold unrolling) when that register is also compared in the loop,
    else 1."""
    compared = {r for ins in body if ins.op.startswith(("s_cmp", "s_cmpk")) for r in ins.src}
    for ins in body:
        if ins.op in ("s_add_i32", "s_sub_i32", "s_add_u32", "s_sub_u32") and ins.dst and ins.dst[0] in compared \
                and ins.imm is not None and ins.dst[0] in ins.src:
            return max(1, abs(ins.imm))
    return 1
