"""Core emitter machinery: jaxpr -> HIP C++ for gfx950.

Same extension contract as the reference emitter
(`src/palladium/emit/core.py:84-256`): `CVal` (a lowered atom), `Cursor`
(text position), `Environment` (Var bindings + def-use maps), `declare`,
the `RULES` registry and the `rule(*names)` decorator with rule signature
`(env, cursor, eqn) -> None`, so rules written for the reference port by
changing only the C they print.

What differs is the execution mapping, chosen for CDNA4:
- every program instance is one lane of a 64-wide wavefront; the flat
  program index is the global thread index, decomposed row-major into grid
  coordinates (the last grid axis is fastest, so neighbouring lanes touch
  neighbouring memory for the usual `lambda i, j: ...` layouts);
- values of size 1 are plain scalar locals (`float t7`), never one-element
  arrays, so loop carries live in VGPRs;
- kernel operands are `__restrict__` SoA pointers; small blocks read by a
  get are loaded once into registers, large read-only blocks are aliased;
- workgroups are remapped so each XCD (8 per MI355X, each with its own L2)
  works on a contiguous range of program instances.
"""

from __future__ import annotations

import contextlib
import dataclasses
import itertools
import math
import os
import string
from collections.abc import Callable, Iterator
from typing import Any

import numpy as np

from palladium_amd.dtypes import is_bf16, scalar_f32
from palladium_amd.dtypes import name as dtype_name
from palladium_amd.errors import EmitError, UnsupportedPrimitiveError
from palladium_amd.ir import Jaxpr, JaxprEqn, KeyAval, Literal, NDIndexer, Slice, Var
from palladium_amd.runtime import math_mode_ordinal
from palladium_amd.trace import BlockInfo, KernelSpec

__all__ = [
    "CTYPES",
    "CVal",
    "Cursor",
    "EmitError",
    "Environment",
    "RULES",
    "declare",
    "emit_hip",
    "emit_jaxpr",
    "rule",
]

MAX_PRIMITIVE_ARITY = 6
PRIMITIVE_INVARS = string.ascii_lowercase[:MAX_PRIMITIVE_ARITY]

CTYPES = {
    "float32": "float",
    "float16": "_Float16",
    "bfloat16": "__bf16",
    "int32": "int",
    "uint32": "unsigned int",
    "bool": "bool",
}

# Loads of read-only blocks up to this many elements go to registers;
# larger blocks are aliased and read through the pointer.
REGISTER_BLOCK_LIMIT = 16
# Element loops up to this many trips are fully unrolled.
UNROLL_LIMIT = 64
DEFAULT_BLOCK = 256
NUM_XCDS = 8


# Value types only rewrites introduce (never a kernel operand): the double
# log2 that the SAFE power carries between loop iterations.
INTERNAL_CTYPES = {"float64": "double"}


def ctype_of(dtype: Any) -> str:
    name = dtype_name(dtype)
    c = CTYPES.get(name) or INTERNAL_CTYPES.get(name)
    if c is None:
        raise EmitError(f"dtype {name} has no HIP lowering (supported: {', '.join(CTYPES)})")
    return c


@dataclasses.dataclass(frozen=True)
class CVal:
    """A jaxpr atom lowered to C.

    Attributes
    ----------
    expr : str
        C identifier, literal, or expression (any rvalue for scalars; an
        array or pointer name otherwise).
    shape : tuple of int
        Logical shape; `()` for scalars.
    ctype : str
        C type of one element.
    space : str
        `"local"` for emitter-declared values, `"global"` for kernel
        operand refs and views of them.
    readonly : bool
        True for input refs and views of them.
    """

    expr: str
    shape: tuple[int, ...]
    ctype: str
    space: str = "local"
    readonly: bool = False

    @property
    def size(self) -> int:
        return math.prod(self.shape)

    @property
    def scalar(self) -> bool:
        """Stored as a single C scalar (size-1 local values)."""
        return self.space == "local" and self.size == 1

    def at(self, index: str) -> str:
        """Element `index` (flat, row-major); the scalar itself for
        size-1 locals."""
        if self.scalar:
            return self.expr
        return f"{self.expr}[{index}]"


class Cursor:
    """The write position into one kernel's growing HIP text."""

    def __init__(self) -> None:
        self.lines: list[str] = []
        self.indent = 1
        self._names = itertools.count()

    def emit(self, line: str) -> None:
        self.lines.append("    " * self.indent + line)

    def fresh(self, prefix: str = "t") -> str:
        return f"{prefix}{next(self._names)}"

    @contextlib.contextmanager
    def block(self, header: str) -> Iterator[None]:
        self.emit(header + " {")
        self.indent += 1
        yield
        self.indent -= 1
        self.emit("}")

    def loop(self, count: int, prefix: str = "_i") -> "contextlib.AbstractContextManager[str]":
        """`for (int i = 0; i < count; ++i)`, yields `i`. Loops up to
        UNROLL_LIMIT trips are fully unrolled (constant indices let small
        arrays stay in registers); longer ones are left to the compiler,
        since their arrays live in scratch either way."""

        @contextlib.contextmanager
        def cm() -> Iterator[str]:
            i = self.fresh(prefix)
            if count <= UNROLL_LIMIT:
                self.emit("#pragma unroll")
            with self.block(f"for (int {i} = 0; {i} < {count}; ++{i})"):
                yield i

        return cm()

    def copy(self, dst: CVal, src: CVal, count: int) -> None:
        """dst[i] = src[i] for i < count."""
        if count == 1:
            self.emit(f"{dst.at('0')} = {src.at('0')};")
            return
        with self.loop(count) as i:
            self.emit(f"{dst.at(i)} = {src.at(i)};")


class Environment:
    """Symbol table for one kernel: Var bindings and def-use info."""

    def __init__(self, index_type: str = "int") -> None:
        self.bindings: dict[Var, CVal] = {}
        self.consumers: dict[Var, list[JaxprEqn | None]] = {}
        self.producers: dict[Var, JaxprEqn] = {}
        self.index_type = index_type

    def val(self, atom: Any) -> CVal:
        if isinstance(atom, Literal):
            return literal_cval(atom.val, atom.aval.dtype)
        try:
            return self.bindings[atom]
        except KeyError:
            raise EmitError(f"unbound jaxpr variable {atom!r}") from None

    def bind(self, var: Var, cval: CVal) -> CVal:
        self.bindings[var] = cval
        return cval

    def used(self, var: Var) -> bool:
        return bool(self.consumers.get(var))


def format_float(v: float) -> str:
    f = float(np.float32(v))
    if math.isinf(f):
        return "(-__builtin_inff())" if f < 0 else "__builtin_inff()"
    if math.isnan(f):
        return "__builtin_nanf(\"\")"
    s = repr(f)
    if "e" not in s and "." not in s:
        s += ".0"
    return s + "f"


def literal_cval(v: Any, dtype: Any) -> CVal:
    dt = np.dtype(dtype)
    ctype = ctype_of(dt)
    if is_bf16(dt):
        expr = format_float(scalar_f32(v))
    elif dt.kind == "f":
        # Round to the literal's own type first: a float16 (or bfloat16)
        # literal is emitted as the float32 spelling of its value (exact), so
        # mixed expressions round exactly as the narrow arithmetic would.
        expr = format_float(float(np.asarray(v, dt)))
    elif dt.kind == "b":
        expr = "true" if v else "false"
    elif dt.kind == "u":
        expr = f"{int(v) & 0xFFFFFFFF}u"
    else:
        iv = int(v)
        expr = str(iv) if iv >= 0 else f"({iv})"
    return CVal(expr, (), ctype)


def declare(env: Environment, cursor: Cursor, var: Var, init: str | None = None) -> CVal:
    """Emit storage for `var` and bind it. Size-1 values are scalars
    (`float t3 = init;`), larger ones local arrays (`float t3[n];`)."""
    aval = var.aval
    if isinstance(aval, KeyAval):
        shape: tuple[int, ...] = (2,)
        ctype = "unsigned int"
    else:
        shape = tuple(int(d) for d in aval.shape)
        ctype = ctype_of(aval.dtype)
    name = cursor.fresh()
    size = math.prod(shape)
    if size == 1 and not isinstance(aval, KeyAval):
        cursor.emit(f"{ctype} {name} = {init};" if init is not None else f"{ctype} {name};")
    else:
        if init is not None:
            raise EmitError("array declarations take no scalar initializer")
        cursor.emit(f"{ctype} {name}[{size}];")
    return env.bind(var, CVal(name, shape, ctype))


RuleFn = Callable[[Environment, Cursor, JaxprEqn], None]

RULES: dict[str, RuleFn] = {}


def rule(*names: str) -> Callable[[RuleFn], RuleFn]:
    """Register a lowering rule for one or more primitive names."""

    def register(fn: RuleFn) -> RuleFn:
        for n in names:
            RULES[n] = fn
        return fn

    return register


def emit_jaxpr(env: Environment, cursor: Cursor, jaxpr: Jaxpr, in_vals: list[CVal]) -> list[CVal]:
    """Walk a (sub-)jaxpr, dispatching each equation through RULES.

    Raises
    ------
    EmitError
        If the jaxpr captures arrays as constvars.
    UnsupportedPrimitiveError
        For a primitive with no registered rule.
    """
    if jaxpr.constvars:
        raise EmitError(
            f"the kernel captures {len(jaxpr.constvars)} array(s) from its enclosing scope; "
            "a kernel may close over Python scalars, and arrays must be passed in as operands"
        )
    if len(jaxpr.invars) != len(in_vals):
        raise EmitError(f"jaxpr takes {len(jaxpr.invars)} inputs, got {len(in_vals)}")
    for var, cval in zip(jaxpr.invars, in_vals):
        env.bind(var, cval)
    for eqn in jaxpr.eqns:
        for iv in eqn.invars:
            if isinstance(iv, Var):
                env.consumers.setdefault(iv, []).append(eqn)
        for ov in eqn.outvars:
            env.producers[ov] = eqn
    for ov in jaxpr.outvars:
        if isinstance(ov, Var):
            env.consumers.setdefault(ov, []).append(None)
    for eqn in jaxpr.eqns:
        impl = RULES.get(eqn.primitive.name)
        if impl is None:
            raise UnsupportedPrimitiveError(
                f"no HIP rule for primitive '{eqn.primitive.name}'; add one with @rule(...)"
            )
        impl(env, cursor, eqn)
    return [env.val(v) for v in jaxpr.outvars]


def element_strides(shape: tuple[int, ...]) -> tuple[int, ...]:
    return tuple(math.prod(shape[d + 1 :]) for d in range(len(shape)))


def flat_index(terms: list[tuple[str, int]]) -> str:
    parts = [v if s == 1 else f"{v} * {s}" for v, s in terms if s != 0]
    return " + ".join(parts) or "0"


def check_contiguous(info: BlockInfo, what: str) -> None:
    """A block is one contiguous run of memory iff, scanning from the
    innermost dim, every dim is full up to the first partial one, and every
    dim outside that has block size 1. (The reference accepts the narrower
    "only the leading dim may be partial", `src/palladium/emit/core.py:336-344`;
    leading size-1 dims, e.g. squeezed row blocks of a 3-D array, are
    contiguous too.)"""
    full = info.full_block()
    arr = info.array_shape
    d = len(full) - 1
    while d >= 0 and full[d] == arr[d]:
        d -= 1
    # dims 0..d-1 must be size 1 (dim d may be partial)
    if any(full[k] != 1 for k in range(0, max(d, 0))):
        raise EmitError(
            f"{what}: block {info.block_shape} of array {info.array_shape} is "
            "not contiguous; only the leading non-unit block dim may be partial"
        )


def ref_view(env: Environment, ref: CVal, indexer: NDIndexer) -> CVal:
    """Pointer offset + kept shape for an indexed ref access.

    A Slice keeps its dim, any other index squeezes it into the offset.
    Only the first kept dim may be partial (contiguous access), as in the
    reference (`src/palladium/emit/core.py:469-545`).
    """
    strides = element_strides(tuple(indexer.shape))
    terms: list[str] = []
    kept: list[tuple[int, int]] = []
    it = env.index_type
    for d, (idx, stride) in enumerate(zip(indexer.indices, strides)):
        if isinstance(idx, Slice):
            if idx.stride != 1:
                raise EmitError(f"ref access dim {d}: stride {idx.stride} != 1 is unimplemented")
            kept.append((d, int(idx.size)))
            start = idx.start
            expr = str(int(start)) if isinstance(start, (int, np.integer)) else env.val(start).expr
        else:
            expr = env.val(idx).expr
        if expr not in ("0", "(0)"):
            terms.append(f"({it})({expr}) * {stride}" if stride != 1 else f"({it})({expr})")
    for d, size in kept[1:]:
        if size != indexer.shape[d]:
            raise EmitError(
                f"ref access dim {d}: only the leading sliced dimension may take part of "
                "its extent (strided, non-contiguous views cannot be emitted)"
            )
    offset = " + ".join(terms) or "0"
    shape = tuple(size for _, size in kept)
    base = ref.expr
    expr = f"({base} + {offset})" if offset != "0" else base
    return CVal(expr, shape if shape else (1,), ref.ctype, "global", ref.readonly)


def _emit_block_offset(env: Environment, cursor: Cursor, spec: KernelSpec, info: BlockInfo, pid_vals: list[CVal]) -> str:
    imj = info.index_map_jaxpr.jaxpr
    strides = element_strides(info.array_shape)
    full = info.full_block()
    it = env.index_type
    if not imj.invars or not imj.eqns:
        # Constant or identity-shaped maps fold without emitting code.
        vals = [env.val(o) if isinstance(o, Literal) else None for o in imj.outvars]
        if all(v is not None for v in vals):
            off = sum(int(o.val) * b * s for o, b, s in zip(imj.outvars, full, strides))
            return str(off)
    ins = pid_vals[: len(imj.invars)]
    outs = emit_jaxpr(env, cursor, imj, ins)
    terms = []
    for val, b, s in zip(outs, full, strides):
        if val.expr in ("0", "(0)"):
            continue
        terms.append(f"({it})({val.expr}) * {b * s}")
    return " + ".join(terms) or "0"


def _xcd_remap(nblocks: int) -> list[str]:
    """Block-id remap so XCD k (blocks k, k+8, ...) owns a contiguous range."""
    if nblocks < 2 * NUM_XCDS:
        return ["const unsigned int _blk = blockIdx.x;"]
    per, rem = divmod(nblocks, NUM_XCDS)
    return [
        f"const unsigned int _xcd = blockIdx.x % {NUM_XCDS}u;",
        f"const unsigned int _slot = blockIdx.x / {NUM_XCDS}u;",
        f"const unsigned int _blk = (_xcd < {rem}u) ? _xcd * {per + 1}u + _slot"
        f" : {rem * (per + 1)}u + (_xcd - {rem}u) * {per}u + _slot;",
    ]


def _tile2d(grid: tuple[int, ...], block: int, tile: tuple[int, int] | None = None) -> tuple[int, int] | None:
    """(rows, cols) of the instance tile one workgroup covers on a 2-D grid,
    or None to keep the row-major order: `tile` (a 2-D threadgroup, rows of
    grid axis 0 by columns of axis 1) when it covers the workgroup and
    divides the grid, else block/64 rows of 64. Disabled with
    PALLADIUM_TILE2D=0."""
    import os

    if os.environ.get("PALLADIUM_TILE2D", "1") == "0" or len(grid) != 2:
        return None
    if tile is not None:
        ti, tj = (int(t) for t in tile)
        if ti * tj == block and ti >= 1 and tj >= 1 and grid[0] % ti == 0 and grid[1] % tj == 0:
            return ti, tj
        return None
    tj = int(os.environ.get("PALLADIUM_TILE_COLS", "64"))
    ti = block // tj
    if ti < 2 or grid[1] % tj or grid[0] % ti:
        return None
    return ti, tj


@dataclasses.dataclass(frozen=True)
class LaunchGeometry:
    """How a KernelSpec maps to a HIP launch: a 1-D grid of `blocks`
    workgroups of `block` lanes. `lanes` is 1 when each program instance
    is one lane, or B when an instance's B-row block is spread over B lanes
    (lane-parallel lowering)."""

    block: int
    blocks: int
    num_programs: int
    lanes: int = 1


def launch_geometry(spec: KernelSpec, block: int | None = None, lanes: int | None = None) -> LaunchGeometry:
    from palladium_amd.emit.lanes import lanes_of, workgroup_for

    n = spec.num_programs
    b = int(block) if block else DEFAULT_BLOCK
    if b <= 0 or b > 1024 or b % 64:
        raise EmitError(f"block size {b} must be a positive multiple of 64 and at most 1024")
    if n <= 0:
        raise EmitError(f"grid {spec.grid} has no program instances")
    lanes = lanes if lanes is not None else lanes_of(spec)
    if lanes > 1:
        b = workgroup_for(lanes, block)
    else:
        from palladium_amd.emit.compact import WORKGROUP, plan_for

        if plan_for(spec, spec.jaxpr, lanes, block) is not None:
            b = WORKGROUP  # a compacting while loop repacks 1,024-lane workgroups
    threads = n * lanes
    if threads >= 2**31:
        raise EmitError(f"grid {spec.grid} needs more than 2**31 lanes")
    return LaunchGeometry(b, (threads + b - 1) // b, n, lanes)


_TRANSCENDENTAL = frozenset("exp exp2 log log2 log1p expm1 sin cos tan tanh pow logistic atan2 pow_log "
                            "pow_with_log".split())


def _has_transcendental(jaxpr: Jaxpr) -> bool:
    for e in jaxpr.eqns:
        if e.primitive.name in _TRANSCENDENTAL:
            return True
        for v in e.params.values():
            subs = v if isinstance(v, tuple) else (v,)
            for sub in subs:
                inner = getattr(sub, "jaxpr", sub)
                if isinstance(inner, Jaxpr) and _has_transcendental(inner):
                    return True
    return False


def emit_hip(spec: KernelSpec, kernel_name: str | None = None, block: int | None = None,
             math_mode: Any = None, tile: tuple[int, int] | None = None) -> str:
    """Assemble the complete HIP source for a KernelSpec.

    Signature convention (relied on by the launcher): one pointer per
    operand in jaxpr order, inputs (`const T* __restrict__`) then outputs
    (`T* __restrict__`), and nothing else; the grid and block shapes are
    compile-time constants of the source. With `math_mode` FAST the jaxpr
    first goes through the FAST algebraic rewrites of
    `palladium_amd.emit.optimize`, and, in a kernel with no transcendental
    function, through the product contraction (`contract_products`);
    REPRODUCIBLE takes the same rewrites and always the contraction.

    Raises
    ------
    EmitError
        Non-contiguous blocks, scratch operands, unsupported dtypes.
    UnsupportedPrimitiveError
        A primitive with no registered rule.
    """
    from palladium_amd.emit.prelude import PRELUDE

    from palladium_amd.emit.lanes import lane_transform

    name = kernel_name or spec.name
    plan = lane_transform(spec)
    lanes = plan.lanes if plan else 1
    geo = launch_geometry(spec, block, lanes)
    operands = list(spec.inputs) + list(spec.outputs)
    n_in = len(spec.inputs)
    if len(spec.jaxpr.invars) != len(operands):
        raise EmitError(
            f"kernel has {len(spec.jaxpr.invars)} refs but spec carries "
            f"{len(operands)} operands; scratch_shapes are not supported yet"
        )
    biggest = max([math.prod(i.array_shape) for i in operands] + [geo.num_programs])
    env = Environment("int" if biggest < 2**31 else "long long")
    cursor = Cursor()
    params = []
    for k, info in enumerate(operands):
        check_contiguous(info, f"operand {k}")
        ct = ctype_of(info.dtype)
        qual = "const " if k < n_in else ""
        params.append(f"{qual}{ct}* __restrict__ arg{k}_base")

    body = plan.jaxpr if plan else spec.jaxpr
    from palladium_amd.emit.compact import plan_for
    from palladium_amd.emit.optimize import fold_counters, funnel_shifts

    # The launch geometry was chosen on the traced jaxpr: a rewrite that
    # adds or removes loop carries can move a loop across the LDS budget of
    # lane compaction, so each such rewrite is taken only if it leaves the
    # loop's compaction as the geometry has it.
    compacting = plan is None and geo.block == 1024 and plan_for(spec, spec.jaxpr, lanes, block) is not None

    def keeps_compaction(candidate: Jaxpr) -> bool:
        return (plan_for(spec, candidate, lanes, block) is not None) == compacting

    if math_mode is not None and math_mode_ordinal(math_mode) in (2, 3):
        # REPRODUCIBLE takes FAST's algebra too; its lowering keeps every
        # operation deterministic
        from palladium_amd.emit.optimize import fast_rewrites

        rewritten = fast_rewrites(body)
        if keeps_compaction(rewritten):
            body = rewritten
    if (math_mode is not None and math_mode_ordinal(math_mode) in (0, 3)
          and os.environ.get("PALLADIUM_SHARE_POW_LOGS", "1") != "0"):
        from palladium_amd.emit.optimize import share_pow_logs

        shared = share_pow_logs(body)
        if keeps_compaction(shared):
            body = shared
    if math_mode is not None and (math_mode_ordinal(math_mode) == 3 or
                                  (math_mode_ordinal(math_mode) == 2 and not _has_transcendental(body)
                                   and os.environ.get("PALLADIUM_FAST_CONTRACT", "1") != "0")):
        # FAST pins the fused sites only where nothing transcendental
        # follows: the compiler folds a transcendental's input scaling
        # (exp's log2 e, say) into the FMA before it, which an explicit site
        # prevents
        from palladium_amd.emit.optimize import contract_products

        body = contract_products(body)
    # Exact, every mode; after the rewrites that read the or-and-shift form.
    body = funnel_shifts(body)
    if os.environ.get("PALLADIUM_FOLD_COUNTERS", "1") != "0":
        folded = fold_counters(body)
        if keeps_compaction(folded):
            body = folded

    from palladium_amd.emit.optimize import drop_dead_code

    pruned = drop_dead_code(body)
    if keeps_compaction(pruned):
        body = pruned

    cplan = plan_for(spec, body, lanes, block)
    if (cplan is not None) != compacting:
        raise EmitError("internal: while-loop compaction disagrees with the launch geometry")

    for line in _xcd_remap(geo.blocks):
        cursor.emit(line)
    cursor.emit(f"const unsigned int _flat = _blk * {geo.block}u + threadIdx.x;")
    total = geo.num_programs * lanes
    if cplan is not None and total % geo.block:
        # A compacting loop needs every lane of the workgroup at its
        # barriers: lanes past the grid stay, compute on the last instance's
        # data (clamped index, loads in bounds), never enter the loop and
        # store nothing.
        cursor.emit(f"const bool _in = _flat < {total}u;")
        cursor.emit(f"const unsigned int _flatc = _in ? _flat : {total - 1}u;")
        env.store_guard = "_in"  # type: ignore[attr-defined]
        env.compact_in = "_in"  # type: ignore[attr-defined]
    else:
        cursor.emit(f"if (_flat >= {total}u) return;")
    if lanes > 1:
        cursor.emit(f"const unsigned int _inst = _flat / {lanes}u;")
        cursor.emit(f"const int _lane = (int)(_flat % {lanes}u);")
    env.lanes = lanes  # type: ignore[attr-defined]
    env.math_mode = math_mode  # type: ignore[attr-defined]
    env.grid = tuple(spec.grid)  # type: ignore[attr-defined]
    pid_vals = []
    rem = "_inst" if lanes > 1 else ("_flatc" if getattr(env, "compact_in", None) else "_flat")
    grid = tuple(spec.grid)
    tile = _tile2d(grid, geo.block, tile) if lanes == 1 else None
    if tile is not None:
        # 2-D grids: a workgroup covers a (block/64) x 64 tile of instances,
        # each wavefront one 64-wide row segment, so vertical neighbours of
        # a stencil are in the same workgroup (and L1) instead of in other
        # workgroups.
        ti, tj = tile
        tiles_j = grid[1] // tj
        cursor.emit(f"const unsigned int _tw = _blk % {tiles_j}u;")
        cursor.emit(f"const unsigned int _th = _blk / {tiles_j}u;")
        cursor.emit(f"const int _pid0 = (int)(_th * {ti}u + threadIdx.x / {tj}u);")
        cursor.emit(f"const int _pid1 = (int)(_tw * {tj}u + threadIdx.x % {tj}u);")
    else:
        for axis in reversed(range(len(grid))):
            g = grid[axis]
            if axis == 0:
                expr = rem
            else:
                expr = f"{rem} % {g}u" if g != 1 else "0u"
            cursor.emit(f"const int _pid{axis} = (int)({expr});")
            if axis > 0:
                nxt = cursor.fresh("_q")
                cursor.emit(f"const unsigned int {nxt} = {rem} / {g}u;")
                rem = nxt
    for axis in range(len(grid)):
        pid_vals.append(CVal(f"_pid{axis}", (), "int"))
    env.pids = pid_vals  # type: ignore[attr-defined]
    if plan is not None and plan.rows is not None:
        # Ragged tail: lanes past the last valid row read the last row
        # (in bounds; rows are independent) and store nothing.
        cursor.emit(f"const bool _live = _pid0 * {lanes} + _lane < {plan.rows};")
        cursor.emit(f"const int _lane_ld = _live ? _lane : {plan.rows - 1} - _pid0 * {lanes};")
        env.lane_expr = "_lane_ld"  # type: ignore[attr-defined]
        env.live = "_live"  # type: ignore[attr-defined]

    ref_vals: list[CVal] = []
    for k, info in enumerate(operands):
        ct = ctype_of(info.dtype)
        qual = "const " if k < n_in else ""
        offset = _emit_block_offset(env, cursor, spec, info, pid_vals)
        ptr = f"{qual}{ct}* __restrict__ arg{k}"
        cursor.emit(f"{ptr} = arg{k}_base + {offset};" if offset != "0" else f"{ptr} = arg{k}_base;")
        ref_vals.append(CVal(f"arg{k}", info.block_shape or (1,), ct, "global", k < n_in))

    env.compact = body.eqns[cplan.index] if cplan is not None else None  # type: ignore[attr-defined]
    emit_jaxpr(env, cursor, body, ref_vals)

    head = (
        f'extern "C" __global__ void __launch_bounds__({geo.block})\n{name}(\n    '
        + ",\n    ".join(params)
        + ")\n{"
    )
    return "\n".join(
        [
            f"// palladium_amd kernel {name}: grid={grid} block={geo.block} blocks={geo.blocks} lanes={lanes}",
            PRELUDE,
            head,
            *cursor.lines,
            "}",
            "",
        ]
    )
