"""Lowering rules: one program instance per GPU lane.

Every rule prints HIP C++ through the Cursor and binds its outvars in the
Environment. Size-1 values are scalars, larger values local arrays whose
element loops are fully unrolled (constant trip counts, so SROA keeps them
in registers). Primitive semantics follow the reference's templates
(`src/palladium/emit/core.py:568-601`, `src/palladium/emit/rules.py`),
with each rule citing the reference rule it replaces.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Any, Callable

import numpy as np

from palladium_amd.emit.core import (
    PRIMITIVE_INVARS,
    REGISTER_BLOCK_LIMIT,
    RULES,
    Cursor,
    CVal,
    EmitError,
    Environment,
    ctype_of,
    declare,
    element_strides,
    emit_jaxpr,
    flat_index,
    format_float,
    literal_cval,
    ref_view,
    rule,
)
from palladium_amd.ir import JaxprEqn, KeyAval, Literal, Var
from palladium_amd.runtime import REPRODUCIBLE_ORDINAL, math_mode_ordinal

F32 = "float"
F16 = "_Float16"
BF16 = "__bf16"
FLOAT_CTYPES = (F32, F16, BF16)


def _is_float(c: CVal) -> bool:
    """float32, float16 and bfloat16 share every template: narrow operands
    promote to float in the float functions, and assigning the result to a
    narrow variable rounds it once. bfloat16 operands are widened explicitly
    (`(float)x`), so a template evaluates wholly in float32 whatever the
    compiler's bf16 excess-precision setting."""
    return c.ctype in FLOAT_CTYPES


def _acc_ctype(ctype: str) -> str:
    """Accumulator type of reductions and contractions: bfloat16 sums and
    dot products accumulate in float32 and round once, as XLA's CPU backend
    computes bf16 reductions; other types accumulate in their own type."""
    return F32 if ctype == BF16 else ctype


def _operand(expr: str, src_ctype: str) -> str:
    return f"((float){expr})" if src_ctype == BF16 else expr


# ---------------------------------------------------------------------------
# element-wise templates. Fields a, b, c ... are the operands in jaxpr order.


def _tmpl(opname: str, ops: list[CVal], out_ctype: str) -> str:
    f = _is_float(ops[0]) if ops else False
    if opname == "add":
        return "({a} + {b})"
    if opname == "sub":
        return "({a} - {b})"
    if opname == "mul":
        return "({a} * {b})"
    if opname == "div":
        if f:
            return "({a} / {b})"
        return "ph_udiv({a}, {b})" if out_ctype == "unsigned int" else "ph_idiv({a}, {b})"
    if opname == "rem":
        if f:
            return "fmodf({a}, {b})"
        return "ph_urem({a}, {b})" if out_ctype == "unsigned int" else "ph_irem({a}, {b})"
    if opname == "min":
        return "ph_fmin({a}, {b})" if f else "(({a} < {b}) ? {a} : {b})"
    if opname == "max":
        return "ph_fmax({a}, {b})" if f else "(({a} > {b}) ? {a} : {b})"
    if opname == "pow":
        return "ph_pow({a}, {b})"
    if opname == "alignbit":
        return "__builtin_amdgcn_alignbit({a}, {b}, {c})"
    if opname == "pow_log":
        return "ph_pow_log({a})"
    if opname == "pow_with_log":
        return "ph_pow_with_log({a}, {b}, {c})"
    if opname == "neg":
        return "(-{a})"
    if opname == "abs":
        if f:
            return "fabsf({a})"
        return "({a})" if out_ctype == "unsigned int" else "ph_iabs({a})"
    if opname == "sign":
        return "(({a} > 0.0f) ? 1.0f : (({a} < 0.0f) ? -1.0f : {a}))" if f else "(({a} > 0) - ({a} < 0))"
    unary_f = {
        "exp": "ph_exp({a})",
        "exp2": "ph_exp2({a})",
        "log": "ph_log({a})",
        "log2": "ph_log2({a})",
        "log1p": "log1pf({a})",
        "expm1": "ph_expm1({a})",
        "sin": "ph_sin({a})",
        "cos": "ph_cos({a})",
        "tan": "tanf({a})",
        "tanh": "ph_tanh({a})",
        "sqrt": "sqrtf({a})",
        "rsqrt": "(1.0f / sqrtf({a}))",
        "floor": "floorf({a})",
        "ceil": "ceilf({a})",
        "round": "roundf({a})",
        "logistic": "(1.0f / (1.0f + ph_exp(-{a})))",
        "atan2": "atan2f({a}, {b})",
    }
    if opname in unary_f:
        return unary_f[opname]
    cmp = {"lt": "<", "le": "<=", "gt": ">", "ge": ">=", "eq": "==", "ne": "!="}
    if opname in cmp:
        return "({a} %s {b})" % cmp[opname]
    if opname in ("and", "or", "xor"):
        op = {"and": "&", "or": "|", "xor": "^"}[opname]
        return "({a} %s {b})" % op
    if opname == "not":
        return "(!{a})" if ops[0].ctype == "bool" else "(~{a})"
    if opname == "shift_right_logical":
        if ops[0].ctype == "int":
            return "((int)(((unsigned int){b} < 32u) ? ((unsigned int){a} >> {b}) : 0u))"
        return "((((unsigned int){b}) < 32u) ? ({a} >> {b}) : 0u)"
    if opname == "shift_right_arithmetic":
        return "({a} >> (((unsigned int){b} < 32u) ? {b} : 31))"
    if opname == "shift_left":
        return "((((unsigned int){b}) < 32u) ? ({a} << {b}) : (%s)0)" % ops[0].ctype
    if opname == "clamp":
        # lax.clamp(min, x, max) = min(max(x, lo), hi)
        if f:
            return "ph_fmin(ph_fmax({b}, {a}), {c})"
        return "((({b} > {a}) ? {b} : {a}) < {c} ? (({b} > {a}) ? {b} : {a}) : {c})"
    raise EmitError(f"no element-wise template for {opname}")


# The elementwise subset, for discoverability and rule registration.
ELEMENTWISE = (
    "add sub mul div rem min max pow neg abs sign exp exp2 log log2 log1p expm1 sin cos "
    "tan tanh sqrt rsqrt floor ceil round logistic atan2 lt le gt ge eq ne and or xor "
    "not shift_right_logical shift_right_arithmetic shift_left clamp"
).split()


def _op_index(op: CVal, dst_shape: tuple[int, ...], idx_vars: list[str]) -> str:
    """NumPy right-aligned broadcast of `op` against `dst_shape`."""
    if op.size == 1:
        return "0"
    rank = len(dst_shape)
    diff = rank - len(op.shape)
    strides = element_strides(op.shape)
    return flat_index([(idx_vars[d + diff], strides[d]) for d, s in enumerate(op.shape) if s != 1])


def _emit_elementwise_loops(cursor: Cursor, dst: CVal, body: Callable[[list[str], str], None]) -> None:
    rank = len(dst.shape)
    if dst.size == 1:
        body(["0"] * rank, "0")
        return
    strides = element_strides(dst.shape)
    idx_vars: list[str] = []

    def go(d: int) -> None:
        if d == rank:
            body(idx_vars, flat_index(list(zip(idx_vars, strides))))
            return
        with cursor.loop(dst.shape[d], f"_e{d}_") as i:
            idx_vars.append(i)
            go(d + 1)
            idx_vars.pop()

    go(0)


def _round_to_even(eqn: JaxprEqn) -> bool:
    """lax.round's `rounding_method`: 0 = AWAY_FROM_ZERO (the default,
    C roundf), 1 = TO_NEAREST_EVEN (jnp.round, C rintf)."""
    return int(eqn.params.get("rounding_method", 0)) == 1


# REPRODUCIBLE float32 forms (palladium_amd.runtime.MathMode): division as a
# times the correctly rounded reciprocal, and the fast deterministic power.
_REPRODUCIBLE_F32 = {
    "div": "ph_rdiv({a}, {b})",
    "pow": "ph_rpow({a}, {b})",
    "pow_log": "ph_rpow_log({a})",
    "pow_with_log": "ph_rpow_with_log({a}, {b}, {c})",
    "log2": "ph_dlog2f({a})",
    "exp2": "ph_dexp2f({a})",
}


def _reproducible(env: Environment) -> bool:
    mode = getattr(env, "math_mode", None)
    return mode is not None and math_mode_ordinal(mode) == REPRODUCIBLE_ORDINAL


def _rule_elementwise(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """All pure element-wise primitives (reference: `_rule_elementwise`,
    `src/palladium/emit/rules.py:274-351`). integer_pow expands to repeated
    multiplication; convert/bitcast cast; operands broadcast NumPy-style."""
    ops = [env.val(v) for v in eqn.invars]
    opname = eqn.primitive.name
    out = eqn.outvars[0]
    dst_ctype = ctype_of(out.aval.dtype)
    if opname == "integer_pow":
        y = int(eqn.params["y"])
        if y == 0:
            template = "(%s)1" % dst_ctype
        else:
            body = " * ".join(["{a}"] * abs(y))
            template = f"({body})" if y > 0 else f"(1.0f / ({body}))"
    elif opname == "convert_element_type":
        template = f"(({dst_ctype}){{a}})"
        if dst_ctype == "bool":
            template = "({a} != 0)"
        elif dst_ctype in ("int", "unsigned int") and ops[0].ctype in FLOAT_CTYPES:
            # saturating, NaN -> 0 (a plain cast is undefined out of range)
            template = ("ph_f2u" if dst_ctype == "unsigned int" else "ph_f2i") + "((float){a})"
        elif dst_ctype == BF16 and ops[0].ctype not in (F32, BF16):
            # integers and float16 reach bfloat16 through float32 (one rule
            # for device and interpreter)
            template = f"(({BF16})(float){{a}})"
    elif opname == "bitcast_convert_type":
        template = f"__builtin_bit_cast({dst_ctype}, {{a}})"
    elif opname == "round" and _round_to_even(eqn):
        template = "rintf({a})"  # the default rounding mode: nearest, ties to even
    elif opname == "select_n":
        if len(ops) == 3 and ops[0].ctype == "bool":
            template = "({a} ? {c} : {b})"
        else:
            if ops[0].ctype == "bool" and len(ops) != 3:
                raise EmitError("select_n with a bool predicate takes exactly two cases")
            # Integer selector: case k for k, clamped like lax.select_n.
            n = len(ops) - 1
            fields = PRIMITIVE_INVARS[1 : 1 + n]
            if n > len(PRIMITIVE_INVARS) - 1:
                raise EmitError(f"select_n with {n} cases exceeds the supported arity")
            expr = "{%s}" % fields[-1]
            for k in reversed(range(n - 1)):
                expr = "(({a} <= %d) ? {%s} : %s)" % (k, fields[k], expr)
            template = expr
    elif opname == "fma":
        if dst_ctype != F32:
            raise EmitError("fma is emitted for float32 only")
        na = "-" if eqn.params.get("neg_ab") else ""
        nc = "-" if eqn.params.get("neg_c") else ""
        template = f"__builtin_fmaf({na}{{a}}, {{b}}, {nc}{{c}})"
    elif _reproducible(env) and opname in _REPRODUCIBLE_F32 and ops and ops[0].ctype == F32:
        template = _REPRODUCIBLE_F32[opname]
        if opname == "div" and isinstance(eqn.invars[1], Literal) and np.shape(eqn.invars[1].val) == ():
            # a * RN(1/c) with the reciprocal of a literal divisor rounded here
            recip = np.float32(1.0) / np.float32(eqn.invars[1].val)
            template = f"({{a}} * {format_float(float(recip))})"
            ops = ops[:1]
    else:
        template = _tmpl(opname, ops, dst_ctype)

    n_fields = len({f for f in PRIMITIVE_INVARS if "{" + f + "}" in template})
    if n_fields != len(ops):
        raise EmitError(f"{opname} requires {n_fields} operands, got {len(ops)}")
    widen = opname != "bitcast_convert_type"

    def operand(o: CVal, e: str) -> str:
        return _operand(e, o.ctype) if widen else e

    dst_shape = tuple(int(d) for d in out.aval.shape)
    if math.prod(dst_shape) == 1:
        expr = template.format(**{n: operand(o, o.at("0")) for n, o in zip(PRIMITIVE_INVARS, ops)})
        declare(env, cursor, out, init=expr)
        return
    dst = declare(env, cursor, out)

    def body(idx_vars: list[str], flat: str) -> None:
        vals = {n: operand(o, o.at(_op_index(o, dst_shape, idx_vars))) for n, o in zip(PRIMITIVE_INVARS, ops)}
        cursor.emit(f"{dst.at(flat)} = {template.format(**vals)};")

    _emit_elementwise_loops(cursor, dst, body)


for _name in [*ELEMENTWISE, "integer_pow", "convert_element_type", "bitcast_convert_type", "select_n",
              "pow_log", "pow_with_log", "alignbit", "fma"]:
    RULES[_name] = _rule_elementwise


# ---------------------------------------------------------------------------
# memory


def _indexer(eqn: JaxprEqn, start: int):
    tree = eqn.params["tree"]
    args = tree.unflatten(eqn.invars[start:])
    return args[0] if args else None


@rule("get")
def _rule_get(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """Load from a Ref (reference: `src/palladium/emit/rules.py:38-69`).

    Small blocks are loaded into registers once; read-only blocks larger
    than REGISTER_BLOCK_LIMIT elements are aliased (pointer view), which is
    safe because nothing writes through an input ref.
    """
    src = env.val(eqn.invars[0])
    indexer = _indexer(eqn, 1)
    view = ref_view(env, src, indexer) if indexer is not None else src
    out = eqn.outvars[0]
    out_shape = tuple(int(d) for d in out.aval.shape)
    size = math.prod(out_shape)
    if size == 1:
        declare(env, cursor, out, init=view.at("0"))
        return
    if view.readonly and size > REGISTER_BLOCK_LIMIT:
        env.bind(out, dataclasses.replace(view, shape=out_shape))
        return
    dst = declare(env, cursor, out)
    cursor.copy(dst, view, size)


@rule("swap")
def _rule_swap(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """Store to a Ref (reference: `src/palladium/emit/rules.py:72-88`).
    The outvar (the value the ref held before) is loaded only if used."""
    ref = env.val(eqn.invars[0])
    value = env.val(eqn.invars[1])
    indexer = _indexer(eqn, 2)
    dst = ref_view(env, ref, indexer) if indexer is not None else ref
    if dst.readonly:
        raise EmitError("cannot store into an input ref")
    out = eqn.outvars[0]
    size = math.prod(tuple(int(d) for d in out.aval.shape))
    if env.used(out):
        old = declare(env, cursor, out, init=dst.at("0")) if size == 1 else declare(env, cursor, out)
        if size != 1:
            cursor.copy(old, dst, size)
    guard = None
    if eqn.params.get("lane0_only") and getattr(env, "lanes", 1) > 1:
        guard = "_lane == 0"
    elif eqn.params.get("lane_row") and getattr(env, "live", None):
        guard = env.live  # type: ignore[attr-defined]
    if getattr(env, "store_guard", None):
        # lanes past the grid of a compacting kernel store nothing
        guard = env.store_guard if guard is None else f"({guard}) && {env.store_guard}"  # type: ignore[attr-defined]
    if guard:
        cursor.emit(f"if ({guard}) {{")
        cursor.indent += 1
    if value.size == 1 and size > 1:
        with cursor.loop(size) as i:
            cursor.emit(f"{dst.at(i)} = {value.at('0')};")
    else:
        cursor.copy(dst, value, size)
    if guard:
        cursor.indent -= 1
        cursor.emit("}")


# ---------------------------------------------------------------------------
# structural


@rule("broadcast_in_dim")
def _rule_broadcast_in_dim(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """Size-preserving broadcasts alias; others materialise (reference:
    `src/palladium/emit/rules.py:364-405`)."""
    src = env.val(eqn.invars[0])
    out = eqn.outvars[0]
    shape = tuple(int(d) for d in eqn.params["shape"])
    if src.size == math.prod(shape):
        if src.scalar or src.space == "local" and src.size > 1 or src.space == "global":
            env.bind(out, dataclasses.replace(src, shape=shape))
            return
        # A literal or expression: keep it as a scalar value.
        env.bind(out, dataclasses.replace(src, shape=shape))
        return
    dst = declare(env, cursor, out)
    bdims = tuple(eqn.params["broadcast_dimensions"])
    s_strides = element_strides(src.shape)

    def body(idx_vars: list[str], flat: str) -> None:
        if src.size == 1:
            cursor.emit(f"{dst.at(flat)} = {src.at('0')};")
            return
        sidx = flat_index([(idx_vars[od], s_strides[sd]) for sd, od in enumerate(bdims) if src.shape[sd] != 1])
        cursor.emit(f"{dst.at(flat)} = {src.at(sidx)};")

    _emit_elementwise_loops(cursor, dst, body)


@rule("reshape", "squeeze", "expand_dims")
def _rule_reshape(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """Row-major reinterpretation, no data movement (reference:
    `src/palladium/emit/rules.py:204-219`)."""
    if eqn.params.get("dimensions") is not None:
        raise EmitError("reshape with a dimensions permutation is unimplemented")
    src = env.val(eqn.invars[0])
    shape = tuple(int(d) for d in eqn.outvars[0].aval.shape)
    env.bind(eqn.outvars[0], dataclasses.replace(src, shape=shape))


@rule("transpose")
def _rule_transpose(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """Materialised permuted copy (reference: `src/palladium/emit/rules.py:222-271`)."""
    src = env.val(eqn.invars[0])
    perm = tuple(eqn.params["permutation"])
    out = eqn.outvars[0]
    if src.size == 1:
        env.bind(out, dataclasses.replace(src, shape=tuple(int(d) for d in out.aval.shape)))
        return
    dst = declare(env, cursor, out)
    s_strides = element_strides(src.shape)

    def body(idx_vars: list[str], flat: str) -> None:
        sidx = flat_index([(idx_vars[d], s_strides[perm[d]]) for d in range(len(perm))])
        cursor.emit(f"{dst.at(flat)} = {src.at(sidx)};")

    _emit_elementwise_loops(cursor, dst, body)


# Contractions up to this length are fully unrolled; longer ones stay loops.
DOT_UNROLL_LIMIT = 32


@rule("dot_general")
def _rule_dot_general(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """Per-instance contraction of rank-1/rank-2 operands over one dim
    (reference: `src/palladium/emit/rules.py:408-499`).

    Any single contracting dim on either side is accepted (the reference
    takes only lhs dim 1 with rhs dim 0 and materialises transposes first);
    the operand strides absorb the layout, so `a.T @ b` reads `a` in place.
    Output dims are the lhs free dim then the rhs free dim, as in JAX.
    Accumulation runs in the output ctype (`preferred_element_type`), each
    product formed after converting its operands to it, in k order from
    zero: under SAFE math this is the exact sequence `acc = acc + a*b`. In
    the lane-parallel lowering the lhs rows are spread across lanes, so a
    block matmul `(B, K) @ (K, N)` becomes one `(K,) @ (K, N)` row per lane
    with the rhs read uniformly by the whole wavefront.
    """
    (lc, rc), (lb, rb) = eqn.params["dimension_numbers"]
    if tuple(lb) or tuple(rb):
        raise EmitError("dot_general: batch dims are unimplemented")
    if len(lc) != 1 or len(rc) != 1:
        raise EmitError("dot_general: exactly one contracting dim per operand is implemented")
    lhs = env.val(eqn.invars[0])
    rhs = env.val(eqn.invars[1])
    if len(lhs.shape) not in (1, 2) or len(rhs.shape) not in (1, 2):
        raise EmitError("dot_general: only rank-1/rank-2 operands are implemented")
    lcd, rcd = int(lc[0]), int(rc[0])
    k = lhs.shape[lcd]
    if rhs.shape[rcd] != k:
        raise EmitError(f"dot_general: inner dims disagree ({k} vs {rhs.shape[rcd]})")
    ls, rs = element_strides(lhs.shape), element_strides(rhs.shape)
    lfree = [d for d in range(len(lhs.shape)) if d != lcd]
    rfree = [d for d in range(len(rhs.shape)) if d != rcd]
    m = lhs.shape[lfree[0]] if lfree else 1
    n = rhs.shape[rfree[0]] if rfree else 1
    out = eqn.outvars[0]
    ctype = ctype_of(out.aval.dtype)
    scalar_out = m * n == 1
    dst = None if scalar_out else declare(env, cursor, out)

    act = _acc_ctype(ctype)

    def conv(expr: str, src: CVal) -> str:
        return expr if src.ctype == act else f"(({act}){expr})"

    def term(idx: list[tuple[str, int]]) -> str:
        return flat_index([(v, st) for v, st in idx if v != "0"])

    def contraction(i: str, j: str) -> str:
        acc = cursor.fresh("_acc")
        cursor.emit(f"{act} {acc} = ({act})0;")

        def step(kk: str) -> None:
            li = term(([(i, ls[lfree[0]])] if lfree else []) + [(kk, ls[lcd])])
            ri = term([(kk, rs[rcd])] + ([(j, rs[rfree[0]])] if rfree else []))
            cursor.emit(f"{acc} = {acc} + {conv(lhs.at(li), lhs)} * {conv(rhs.at(ri), rhs)};")

        if k <= DOT_UNROLL_LIMIT:
            with cursor.loop(k, "_k") as kk:
                step(kk)
        else:
            kk = cursor.fresh("_k")
            with cursor.block(f"for (int {kk} = 0; {kk} < {k}; ++{kk})"):
                step(kk)
        return acc

    if scalar_out:
        acc = contraction("0", "0")
        if act != ctype:
            declare(env, cursor, out, init=f"(({ctype}){acc})")
        else:
            env.bind(out, CVal(acc, tuple(int(d) for d in out.aval.shape), ctype))
        return

    def rows(i: str) -> None:
        if n == 1:
            acc = contraction(i, "0")
            cursor.emit(f"{dst.at(term([(i, 1)]) if m > 1 else '0')} = {acc};")
            return
        with cursor.loop(n, "_n") as j:
            acc = contraction(i, j)
            cursor.emit(f"{dst.at(term([(i, n), (j, 1)]))} = {acc};")

    if m == 1:
        rows("0")
    else:
        with cursor.loop(m, "_m") as i:
            rows(i)


@rule("program_id")
def _rule_program_id(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """`pl.program_id(axis)` binds the decoded grid coordinate (reference:
    `src/palladium/emit/rules.py:668-676`)."""
    axis = int(eqn.params["axis"])
    pids = getattr(env, "pids", None)
    if pids is None or axis >= len(pids):
        raise EmitError(f"program_id({axis}) outside a grid of rank {0 if pids is None else len(pids)}")
    env.bind(eqn.outvars[0], pids[axis])


@rule("num_programs")
def _rule_num_programs(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    grid = getattr(env, "grid", None)
    axis = int(eqn.params["axis"])
    if grid is None:
        raise EmitError("num_programs outside a kernel")
    env.bind(eqn.outvars[0], literal_cval(grid[axis], np.int32))


@rule("pjit", "jit", "closed_call", "core_call", "custom_jvp_call", "custom_vjp_call", "remat", "checkpoint")
def _inline_call(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """Inline a nested call by walking its body (reference:
    `src/palladium/emit/rules.py:91-103`)."""
    inner = eqn.params.get("jaxpr") or eqn.params.get("call_jaxpr") or eqn.params.get("fun_jaxpr")
    body = getattr(inner, "jaxpr", inner)
    if getattr(inner, "consts", None):
        raise EmitError(f"{eqn.primitive.name} with consts is unsupported")
    invals = [env.val(v) for v in eqn.invars]
    n = len(body.invars)
    outs = emit_jaxpr(env, cursor, body, invals[-n:] if n < len(invals) else invals)
    for ov, val in zip(eqn.outvars, outs):
        env.bind(ov, val)


# ---------------------------------------------------------------------------
# random


@rule("random_wrap", "random_unwrap")
def _rule_random_alias(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """Key wrap/unwrap are type-level only (reference:
    `src/palladium/emit/rules.py:106-118`)."""
    src = env.val(eqn.invars[0])
    if src.size != 2:
        raise EmitError("only unbatched keys (uint32[2] key data) are supported")
    env.bind(eqn.outvars[0], dataclasses.replace(src, shape=(2,)))


def _key_words(cursor: Cursor, key: CVal) -> tuple[str, str]:
    return key.at("0"), key.at("1")


@rule("random_fold_in")
def _rule_random_fold_in(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """New key = threefry(key, (0, data)) (reference: `src/palladium/emit/rules.py:188-201`)."""
    key = env.val(eqn.invars[0])
    data = env.val(eqn.invars[1])
    k0, k1 = _key_words(cursor, key)
    name = cursor.fresh("_key")
    cursor.emit(f"unsigned int {name}[2];")
    cursor.emit(f"ph_threefry2x32({k0}, {k1}, 0u, (unsigned int)({data.at('0')}), &{name}[0], &{name}[1]);")
    env.bind(eqn.outvars[0], CVal(name, (2,), "unsigned int"))


@rule("random_bits")
def _rule_random_bits(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """bits[i] = x0 ^ x1 of threefry(key, (0, i)), i the flat row-major
    index (reference: `src/palladium/emit/rules.py:168-185`)."""
    if int(eqn.params.get("bit_width", 32)) != 32:
        raise EmitError("random_bits: only bit_width=32 is implemented")
    key = env.val(eqn.invars[0])
    k0, k1 = _key_words(cursor, key)
    out = eqn.outvars[0]
    size = math.prod(tuple(int(d) for d in out.aval.shape))
    a, b = cursor.fresh("_r"), cursor.fresh("_r")
    if size == 1:
        cursor.emit(f"unsigned int {a}, {b};")
        cursor.emit(f"ph_threefry2x32({k0}, {k1}, 0u, 0u, &{a}, &{b});")
        declare(env, cursor, out, init=f"{a} ^ {b}")
        return
    dst = declare(env, cursor, out)
    with cursor.loop(size) as i:
        cursor.emit(f"unsigned int {a}, {b};")
        cursor.emit(f"ph_threefry2x32({k0}, {k1}, 0u, (unsigned int){i}, &{a}, &{b});")
        cursor.emit(f"{dst.at(i)} = {a} ^ {b};")


@rule("threefry2x32")
def _rule_threefry2x32(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """Raw Threefry-2x32-20 block over broadcast uint32 operands
    (k0, k1, x0, x1) -> (y0, y1)."""
    ops = [env.val(v) for v in eqn.invars]
    o0v, o1v = eqn.outvars
    shape = tuple(int(d) for d in o0v.aval.shape)
    if math.prod(shape) == 1:
        a, b = cursor.fresh("_r"), cursor.fresh("_r")
        cursor.emit(f"unsigned int {a}, {b};")
        args = ", ".join(o.at("0") for o in ops)
        cursor.emit(f"ph_threefry2x32({args}, &{a}, &{b});")
        declare(env, cursor, o0v, init=a)
        declare(env, cursor, o1v, init=b)
        return
    d0 = declare(env, cursor, o0v)
    d1 = declare(env, cursor, o1v)

    def body(idx_vars: list[str], flat: str) -> None:
        args = ", ".join(o.at(_op_index(o, shape, idx_vars)) for o in ops)
        cursor.emit(f"ph_threefry2x32({args}, &{d0.at(flat)}, &{d1.at(flat)});")

    _emit_elementwise_loops(cursor, d0, body)


# ---------------------------------------------------------------------------
# reductions


def _emit_reduce(env: Environment, cursor: Cursor, eqn: JaxprEqn, init: str, combine: Callable[[str, str], str]) -> None:
    """Nested loops: kept dims outside, reduced dims accumulating inside
    (reference: `_emit_reduce`, `src/palladium/emit/rules.py:595-642`)."""
    axes = set(int(a) for a in eqn.params["axes"])
    src = env.val(eqn.invars[0])
    rank = len(src.shape)
    kept = [d for d in range(rank) if d not in axes]
    red = [d for d in range(rank) if d in axes]
    out = eqn.outvars[0]
    ctype = ctype_of(out.aval.dtype)
    s_strides = element_strides(src.shape)
    out_shape = tuple(int(d) for d in out.aval.shape)
    d_strides = element_strides(out_shape)
    scalar_out = math.prod(out_shape) == 1
    dst = None if scalar_out else declare(env, cursor, out)
    idx: dict[int, str] = {}

    def loops(dims: list[int], body: Callable[[], None]) -> None:
        if not dims:
            body()
            return
        d = dims[0]
        if src.shape[d] == 1:
            idx[d] = "0"
            loops(dims[1:], body)
            return
        with cursor.loop(src.shape[d], f"_d{d}_") as i:
            idx[d] = i
            loops(dims[1:], body)

    result = {}

    act = _acc_ctype(ctype)

    def accumulate() -> None:
        acc = cursor.fresh("_acc")
        cursor.emit(f"{act} {acc} = {init};")

        def inner() -> None:
            sidx = flat_index([(idx[d], s_strides[d]) for d in range(rank)])
            cursor.emit(f"{acc} = {combine(acc, _operand(src.at(sidx), src.ctype))};")

        loops(red, inner)
        if scalar_out and act != ctype:
            result["acc"] = declare(env, cursor, out, init=f"(({ctype}){acc})").expr
        elif scalar_out:
            result["acc"] = acc
        else:
            didx = flat_index([(idx[d], d_strides[i]) for i, d in enumerate(kept)])
            cursor.emit(f"{dst.at(didx)} = {acc};")

    loops(kept, accumulate)
    if scalar_out and act == ctype:
        env.bind(out, CVal(result["acc"], out_shape, ctype))


def _reduce_init(eqn: JaxprEqn, kind: str) -> str:
    ct = ctype_of(eqn.outvars[0].aval.dtype)
    if kind == "sum":
        return "0.0f" if ct in FLOAT_CTYPES else "0"
    if kind == "max":
        return {"float": "(-__builtin_inff())", F16: "(-__builtin_inff())", BF16: "(-__builtin_inff())",
                "int": "(-2147483647 - 1)",
                "unsigned int": "0u", "bool": "false"}[ct]
    if kind == "min":
        return {"float": "__builtin_inff()", F16: "__builtin_inff()", BF16: "__builtin_inff()",
                "int": "2147483647",
                "unsigned int": "0xFFFFFFFFu", "bool": "true"}[ct]
    return {"or": "false", "and": "true"}[kind]


@rule("reduce_sum")
def _rule_reduce_sum(env, cursor, eqn):
    _emit_reduce(env, cursor, eqn, _reduce_init(eqn, "sum"), lambda a, x: f"{a} + {x}")


@rule("reduce_max")
def _rule_reduce_max(env, cursor, eqn):
    f = ctype_of(eqn.outvars[0].aval.dtype) in FLOAT_CTYPES
    _emit_reduce(env, cursor, eqn, _reduce_init(eqn, "max"),
                 (lambda a, x: f"ph_fmax({a}, {x})") if f else (lambda a, x: f"(({x} > {a}) ? {x} : {a})"))


@rule("reduce_min")
def _rule_reduce_min(env, cursor, eqn):
    f = ctype_of(eqn.outvars[0].aval.dtype) in FLOAT_CTYPES
    _emit_reduce(env, cursor, eqn, _reduce_init(eqn, "min"),
                 (lambda a, x: f"ph_fmin({a}, {x})") if f else (lambda a, x: f"(({x} < {a}) ? {x} : {a})"))


@rule("reduce_or")
def _rule_reduce_or(env, cursor, eqn):
    _emit_reduce(env, cursor, eqn, "false", lambda a, x: f"({a} || {x})")


@rule("reduce_and")
def _rule_reduce_and(env, cursor, eqn):
    _emit_reduce(env, cursor, eqn, "true", lambda a, x: f"({a} && {x})")


# ---------------------------------------------------------------------------
# control flow


def _declare_carries(env: Environment, cursor: Cursor, invars: list[Any], outvars: list[Var]) -> list[CVal]:
    carries = []
    for iv, ov in zip(invars, outvars):
        src = env.val(iv)
        if isinstance(ov.aval, KeyAval) or src.size != 1 or math.prod(ov.aval.shape) != 1:
            dst = declare(env, cursor, ov)
            cursor.copy(dst, src, dst.size)
        else:
            dst = declare(env, cursor, ov, init=src.at("0"))
        carries.append(dst)
    return carries


def copy_back_carries(cursor: Cursor, outs: list[CVal], carries: list[CVal], predicate: str | None = None,
                      guards: list | None = None) -> None:
    """Simultaneous carry update: read every new value into a temporary,
    then write all carries (reference: `src/palladium/emit/rules.py:741-809`;
    the Metal `volatile` workaround is not needed here). With `predicate`,
    a carry takes its new value only where the predicate holds. `guards`
    (one entry per carry, from `select_guards`) narrows that further: a
    carry whose new value is `p ? x : carry` takes x where the predicate
    and p hold, one select where two would otherwise be emitted."""
    guards = guards or [None] * len(carries)
    updates = [(o, c, g) for o, c, g in zip(outs, carries, guards) if o.expr != c.expr]
    staged = []
    for out, carry, g in updates:
        if carry.size == 1:
            t = cursor.fresh("_cb")
            when = predicate
            if g is not None and predicate is not None:
                out, cond = g
                when = cursor.fresh("_cg")
                cursor.emit(f"const bool {when} = ({predicate}) && ({cond});")
            cursor.emit(f"const {carry.ctype} {t} = {out.at('0')};")
            staged.append((carry, t, None, when))
        else:
            t = cursor.fresh("_cb")
            cursor.emit(f"{carry.ctype} {t}[{carry.size}];")
            tv = CVal(t, carry.shape, carry.ctype)
            cursor.copy(tv, out, carry.size)
            staged.append((carry, t, tv, predicate))
    for carry, t, tv, when in staged:
        if when is not None:
            if tv is None:
                cursor.emit(f"{carry.at('0')} = {when} ? {t} : {carry.at('0')};")
            else:
                with cursor.loop(carry.size) as i:
                    cursor.emit(f"{carry.at(i)} = {when} ? {tv.at(i)} : {carry.at(i)};")
        elif tv is None:
            cursor.emit(f"{carry.at('0')} = {t};")
        else:
            cursor.copy(carry, tv, carry.size)


def select_guards(env: Environment, body: Any, nconsts: int) -> list:
    """Per carry of a while body: (x, "p") when the carry's next value is
    `select_n(p, carry, x)`, (x, "!p") for `select_n(p, x, carry)`, else
    None; p a scalar boolean, the C expressions as bound after the body was
    emitted."""
    body = getattr(body, "jaxpr", body)
    producer = {ov: e for e in body.eqns for ov in e.outvars}
    out = []
    for k, ov in enumerate(body.outvars):
        c = body.invars[nconsts + k]
        e = producer.get(ov) if isinstance(ov, Var) else None
        g = None
        if (e is not None and e.primitive.name == "select_n" and len(e.invars) == 3 and isinstance(e.invars[0], Var)
                and np.dtype(e.invars[0].aval.dtype) == np.bool_ and math.prod(e.invars[0].aval.shape) == 1
                and math.prod(c.aval.shape) == 1):
            p = env.val(e.invars[0]).at("0")
            if e.invars[1] is c and e.invars[2] is not c:
                g = (env.val(e.invars[2]), p)
            elif e.invars[2] is c and e.invars[1] is not c:
                g = (env.val(e.invars[1]), f"!({p})")
        out.append(g)
    return out


@rule("scan")
def _rule_scan(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """`fori_loop` / pure-carry `scan` -> a counted for-loop; consts pass
    through, carries become mutable locals (reference:
    `src/palladium/emit/rules.py:679-714`)."""
    length = int(eqn.params["length"])
    body = eqn.params["jaxpr"]
    body_j = getattr(body, "jaxpr", body)
    if eqn.params.get("reverse", False):
        raise EmitError("no reverse-mode scan support, use lax.fori_loop")
    num_carry = len(eqn.outvars)
    num_consts = len(eqn.invars) - num_carry
    if len(body_j.outvars) != num_carry:
        raise EmitError("lax.scan with stacked ys not supported, use lax.fori_loop")
    for ov, bv in zip(eqn.outvars, body_j.outvars):
        if tuple(ov.aval.shape) != tuple(getattr(bv, "aval").shape):
            raise EmitError("lax.scan with stacked ys not supported, use lax.fori_loop")
    for iv, bv in zip(eqn.invars, body_j.invars):
        if tuple(getattr(iv.aval, "shape", ())) != tuple(getattr(bv.aval, "shape", ())):
            raise EmitError("lax.scan with scanned xs not supported, use lax.fori_loop")
    consts = [env.val(v) for v in eqn.invars[:num_consts]]
    carries = _declare_carries(env, cursor, eqn.invars[num_consts:], eqn.outvars)
    unroll = eqn.params.get("unroll", 1)
    if isinstance(unroll, bool):
        unroll = length if unroll else 1
    idx = cursor.fresh("_s")
    if int(unroll) > 1:
        cursor.emit(f"#pragma unroll {int(unroll)}")
    with cursor.block(f"for (int {idx} = 0; {idx} < {length}; ++{idx})"):
        outs = emit_jaxpr(env, cursor, body_j, consts + carries)
        copy_back_carries(cursor, outs, carries)


def _predicable(jaxpr: Any) -> bool:
    """A loop body that may run on lanes whose loop has already ended:
    no ref access (an index built from a finished lane's carries could
    leave its block; a store must not happen), no nested while (its trip
    count could depend on those carries). Pure arithmetic (integer
    division included: ph_idiv/ph_irem are defined for every input and do
    not trap), counted loops, conds and RNG qualify."""
    j = getattr(jaxpr, "jaxpr", jaxpr)
    for e in j.eqns:
        name = e.primitive.name
        if name in ("get", "swap", "while", "lane_index", "lane_reduce"):
            return False
        for v in e.params.values():
            for sub in (v if isinstance(v, tuple) else (v,)):
                if hasattr(getattr(sub, "jaxpr", sub), "eqns") and not _predicable(sub):
                    return False
    return True


@rule("while")
def _rule_while(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """`while_loop` -> `while (true) { cond; if (!p) break; body; }`. Each
    lane iterates independently; the wavefront retires when its last lane
    exits (reference: `src/palladium/emit/rules.py:812-844`).

    With one program instance per lane and a body that may safely run on a
    finished lane (`_predicable`), the loop is emitted predicated instead:
    the wavefront leaves when no lane's condition holds (`__any`), the body
    runs on every lane without exec-mask branching, and each carry keeps
    its old value where the condition is false. Results are identical (a
    finished lane's carries never change again, so its condition stays
    false); the loop avoids the per-iteration mask bookkeeping of the
    divergent form, about 11 % on the adaptive BS3 kernel."""
    cn = int(eqn.params["cond_nconsts"])
    bn = int(eqn.params["body_nconsts"])
    cj = eqn.params["cond_jaxpr"]
    bj = eqn.params["body_jaxpr"]
    if getattr(cj, "consts", None) or getattr(bj, "consts", None):
        raise EmitError("while with jaxpr consts is unsupported")
    if getattr(env, "compact", None) is eqn:
        from palladium_amd.emit.compact import emit_compacting_while

        emit_compacting_while(env, cursor, eqn, emit_jaxpr, _declare_carries, copy_back_carries)
        return
    cond_consts = [env.val(v) for v in eqn.invars[:cn]]
    body_consts = [env.val(v) for v in eqn.invars[cn : cn + bn]]
    carries = _declare_carries(env, cursor, eqn.invars[cn + bn :], eqn.outvars)
    predicated = getattr(env, "lanes", 1) == 1 and _predicable(bj)
    # A predicated loop runs several iterations per pass of its machine loop,
    # each with its own exit test (a break in any of them leaves the loop),
    # as the compacting form does.
    unroll = 1
    if predicated:
        from palladium_amd.emit.compact import epoch_unroll

        unroll = epoch_unroll(getattr(env, "math_mode", None), bj)
    with cursor.block("while (true)"):
        if unroll > 1:
            cursor.emit(f"// {unroll} iterations per pass")
        for _ in range(unroll):
            (pred,) = emit_jaxpr(env, cursor, getattr(cj, "jaxpr", cj), cond_consts + carries)
            p = pred.at("0")
            if predicated:
                # Evaluate once: the body may overwrite what the condition read.
                live = cursor.fresh("_live")
                cursor.emit(f"const bool {live} = {p};")
                with cursor.block(f"if (!__any({live}))"):
                    cursor.emit("break;")
            else:
                with cursor.block(f"if (!({p}))"):
                    cursor.emit("break;")
            outs = emit_jaxpr(env, cursor, getattr(bj, "jaxpr", bj), body_consts + carries)
            if predicated:
                copy_back_carries(cursor, outs, carries, predicate=live, guards=select_guards(env, bj, bn))
            else:
                copy_back_carries(cursor, outs, carries)


@rule("cond")
def _rule_cond(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """`cond`/`switch` -> if / else-if / else over the clamped index
    (reference: `src/palladium/emit/rules.py:847-878`)."""
    branches = eqn.params["branches"]
    index = env.val(eqn.invars[0])
    ops = [env.val(v) for v in eqn.invars[1:]]
    outs = [declare(env, cursor, ov) for ov in eqn.outvars]
    n = len(branches)
    for i, br in enumerate(branches):
        if getattr(br, "consts", None):
            raise EmitError("cond with jaxpr consts is unsupported")
        if n == 1:
            header = "if (true)"
        elif i == 0:
            header = f"if ({index.at('0')} <= 0)"
        elif i < n - 1:
            header = f"else if ({index.at('0')} == {i})"
        else:
            header = "else"
        with cursor.block(header):
            vals = emit_jaxpr(env, cursor, getattr(br, "jaxpr", br), list(ops))
            for o, v in zip(outs, vals):
                cursor.copy(o, v, o.size)


# ---------------------------------------------------------------------------
# iota and the lane-parallel primitives


@rule("iota")
def _rule_iota(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """`lax.broadcasted_iota`: index along `dimension` as the value."""
    out = eqn.outvars[0]
    shape = tuple(int(d) for d in out.aval.shape)
    dim = int(eqn.params["dimension"])
    ct = ctype_of(out.aval.dtype)
    if math.prod(shape) == 1:
        declare(env, cursor, out, init=f"({ct})0")
        return
    dst = declare(env, cursor, out)

    def body(idx_vars: list[str], flat: str) -> None:
        via = "(float)" if ct == BF16 else ""
        cursor.emit(f"{dst.at(flat)} = ({ct}){via}{idx_vars[dim]};")

    _emit_elementwise_loops(cursor, dst, body)


@rule("lane_index")
def _rule_lane_index(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """This lane's row within its instance's block (lane-parallel mode)."""
    env.bind(eqn.outvars[0], CVal(getattr(env, "lane_expr", "_lane"), (), "int"))


_WAVE = 64


@rule("lane_reduce")
def _rule_lane_reduce(env: Environment, cursor: Cursor, eqn: JaxprEqn) -> None:
    """Reduce one scalar per lane over the instance's lanes; every lane gets
    the result. Wavefront butterfly with `__shfl_xor`, then (instances wider
    than one wavefront) partials through LDS, combined in a fixed order."""
    kind = eqn.params["kind"]
    lanes = int(eqn.params["lanes"])
    src = env.val(eqn.invars[0])
    out = eqn.outvars[0]
    ct = ctype_of(out.aval.dtype)
    is_bool = ct == "bool"
    # Shuffles move 32-bit values: bools travel as int, float16 as float
    # (a float16 sum is then accumulated in float32 and rounded once).
    wt = "int" if is_bool else (F32 if ct in (F16, BF16) else ct)
    isf = ct in FLOAT_CTYPES
    comb = {
        "sum": lambda a, b: f"({a} + {b})",
        "max": (lambda a, b: f"ph_fmax({a}, {b})") if isf else (lambda a, b: f"(({a} > {b}) ? {a} : {b})"),
        "min": (lambda a, b: f"ph_fmin({a}, {b})") if isf else (lambda a, b: f"(({a} < {b}) ? {a} : {b})"),
        "or": lambda a, b: f"({a} | {b})",
        "and": lambda a, b: f"({a} & {b})",
    }[kind]
    acc = cursor.fresh("_lr")
    cursor.emit(f"{wt} {acc} = ({wt})({src.at('0')});")
    off = _WAVE // 2
    while off >= 1:
        cursor.emit(f"{acc} = {comb(acc, f'__shfl_xor({acc}, {off}, {_WAVE})')};")
        off //= 2
    if lanes > _WAVE:
        nw = lanes // _WAVE
        sh = cursor.fresh("_lds")
        cursor.emit(f"__shared__ {wt} {sh}[{nw}];")
        cursor.emit(f"if ((_lane & {_WAVE - 1}) == 0) {sh}[_lane / {_WAVE}] = {acc};")
        cursor.emit("__syncthreads();")
        cursor.emit(f"{acc} = {sh}[0];")
        for w in range(1, nw):
            cursor.emit(f"{acc} = {comb(acc, f'{sh}[{w}]')};")
        cursor.emit("__syncthreads();")
    declare(env, cursor, out, init=f"({ct})({acc})" if not is_bool else f"({acc} != 0)")
