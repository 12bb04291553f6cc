"""Lane-parallel lowering of blocked kernels.

When every program instance works on a block of B trajectories along the
leading dim (`BlockSpec((B,), lambda i: (i,))`, B a multiple of 64), running
one instance per lane would put B-element arrays in each lane's registers.
On CDNA4 the natural mapping is the one Pallas intends: the block's leading
dim goes across B lanes (one or more full wavefronts), each lane holding its
own row. This pass rewrites the kernel jaxpr into that per-lane form before
emission:

- a value whose shape carries the lane dim (status L) becomes its per-lane
  row (shape[1:]); values without it (status U: program ids, scalars, keys,
  per-instance reductions) are computed identically by every lane;
- a full-block access `x_ref[...]` / `x_ref[:, j]` on a lane operand indexes
  dim 0 with the lane id; a store of a uniform value to a non-lane location
  is done by lane 0 only;
- `iota` along the lane dim is the lane id;
- a reduction over the lane dim becomes a cross-lane reduction
  (`lane_reduce_*`: wavefront shuffles, then LDS across the instance's waves).

Control flow stays uniform within an instance (loop conditions and switch
indices have no lane dim), so every lane of an instance takes the same path
and the cross-lane reductions are reached by all of them.

If any equation falls outside these forms, `lane_transform` returns None and
the kernel is emitted in the one-lane-per-instance model unchanged.
"""

from __future__ import annotations

import dataclasses
import math
from typing import Any

from palladium_amd.ir import (
    ClosedJaxpr,
    IndexerTree,
    Jaxpr,
    JaxprEqn,
    KeyAval,
    Literal,
    NDIndexer,
    RefAval,
    ShapedArray,
    Slice,
    Var,
    _Leaf,
    primitive,
)
from palladium_amd.trace import KernelSpec

L, U = "L", "U"

_ELEMENTWISE = set(
    "add sub mul div rem min max pow neg abs sign exp exp2 log log2 log1p expm1 sin cos tan tanh sqrt rsqrt floor "
    "ceil round logistic atan2 lt le gt ge eq ne and or xor not shift_right_logical shift_right_arithmetic "
    "shift_left clamp select_n integer_pow convert_element_type bitcast_convert_type threefry2x32".split()
)
_REDUCE = {"reduce_sum": "sum", "reduce_max": "max", "reduce_min": "min", "reduce_or": "or", "reduce_and": "and"}


class _Bail(Exception):
    pass


@dataclasses.dataclass(frozen=True)
class LanePlan:
    """`rows`: when the lane operands' last block runs past their arrays
    (a ragged tail, e.g. N = 100,000 in blocks of 256), the number of valid
    rows; lanes past it load a clamped row and skip their stores."""

    lanes: int
    jaxpr: Jaxpr
    lane_operands: tuple[int, ...]
    rows: int | None = None


def _depends_on_grid(info) -> bool:
    imj = info.index_map_jaxpr.jaxpr
    return bool(imj.invars) and not all(isinstance(o, Literal) for o in imj.outvars)


def _lane_count(spec: KernelSpec) -> tuple[int, tuple[int, ...]] | None:
    operands = list(spec.inputs) + list(spec.outputs)
    cands = [(k, info.block_shape[0]) for k, info in enumerate(operands)
             if info.block_shape and _depends_on_grid(info) and info.block_shape[0] > 1
             and len(info.block_shape) == len(info.array_shape)]
    if not cands:
        # No lane-blocked operand: a kernel may still build its rows itself
        # (`iota` over a leading dim of B, e.g. B paths per instance that are
        # reduced before the store).
        b = _iota_rows(spec.jaxpr)
        if b is None:
            return None
        return (b, ()) if b % 64 == 0 and b <= 1024 else None
    b = max(c for _, c in cands)
    if b % 64 or b > 1024:
        return None
    lane_ops = tuple(k for k, c in cands if c == b)
    return b, lane_ops


def _iota_rows(j: Jaxpr) -> int | None:
    best = None
    for e in j.eqns:
        if e.primitive.name == "iota" and int(e.params["dimension"]) == 0:
            n = int(tuple(e.params["shape"])[0])
            if n > 1:
                best = max(best or 0, n)
        for v in e.params.values():
            subs = v if isinstance(v, tuple) else (v,)
            for sj in subs:
                inner = getattr(sj, "jaxpr", None)
                if isinstance(inner, Jaxpr):
                    r = _iota_rows(inner)
                    if r:
                        best = max(best or 0, r)
    return best


class _Pass:
    def __init__(self, b: int):
        self.b = b
        self.lane_var: Var | None = None

    # -- helpers -----------------------------------------------------------
    def per_lane(self, aval: Any, st: str) -> Any:
        if st == U or isinstance(aval, (KeyAval, RefAval)):
            return aval
        return ShapedArray(tuple(aval.shape[1:]), aval.dtype, aval.weak_type)

    def status_of_shape(self, aval: Any) -> bool:
        return not isinstance(aval, (KeyAval, RefAval)) and len(aval.shape) >= 1 and aval.shape[0] == self.b

    def lane(self, eqns: list[JaxprEqn]) -> Var:
        v = Var(ShapedArray((), "int32"))
        eqns.append(JaxprEqn([], [v], primitive("lane_index"), {"lanes": self.b}))
        return v

    # -- jaxpr walk ------------------------------------------------------------
    def jaxpr(self, j: Jaxpr, in_status: list[str], ref_lane: dict[Any, bool]) -> tuple[Jaxpr, list[str]]:
        env: dict[Any, Any] = {}
        st: dict[Any, str] = {}
        new_invars = []
        for v, s in zip(j.invars, in_status):
            nv = Var(self.per_lane(v.aval, s))
            env[v] = nv
            st[v] = s
            if v in ref_lane:
                ref_lane[nv] = ref_lane[v]
            new_invars.append(nv)
        eqns: list[JaxprEqn] = []

        def a(x: Any) -> Any:
            return x if isinstance(x, Literal) else env[x]

        def s_of(x: Any) -> str:
            return U if isinstance(x, Literal) else st[x]

        for e in j.eqns:
            self.eqn(e, env, st, eqns, a, s_of, ref_lane)
        outs = [a(o) for o in j.outvars]
        return Jaxpr([], new_invars, outs, eqns), [s_of(o) for o in j.outvars]

    def eqn(self, e: JaxprEqn, env, st, eqns, a, s_of, ref_lane) -> None:
        name = e.primitive.name
        ins_st = [s_of(x) for x in e.invars]

        def out(status: str, params: dict | None = None, invars: list | None = None, prim: str | None = None) -> None:
            nouts = []
            for ov in e.outvars:
                if status == L and not self.status_of_shape(ov.aval):
                    raise _Bail(f"{name}: lane value without the lane dim")
                nv = Var(self.per_lane(ov.aval, status))
                env[ov] = nv
                st[ov] = status
                nouts.append(nv)
            eqns.append(JaxprEqn(invars if invars is not None else [a(x) for x in e.invars], nouts,
                                 primitive(prim or name), params if params is not None else dict(e.params)))

        if name in _ELEMENTWISE:
            if L in ins_st:
                for x, s in zip(e.invars, ins_st):
                    if s == U and not isinstance(x, Literal) and self.status_of_shape(x.aval):
                        raise _Bail("uniform operand with the lane dim in a lane op")
                    if s == U and not isinstance(x, Literal) and x.aval.shape and len(x.aval.shape) >= len(e.outvars[0].aval.shape):
                        raise _Bail("uniform operand of full rank in a lane op")
                out(L)
            else:
                out(U)
            return
        if name in ("get", "swap"):
            ref = e.invars[0]
            is_lane_ref = ref_lane.get(env[ref], False)
            start = 1 if name == "get" else 2
            tree = e.params["tree"]
            idx = tree.unflatten(e.invars[start:])
            if not is_lane_ref:
                if name == "swap" and s_of(e.invars[1]) == L:
                    raise _Bail("lane value stored to a non-lane ref")
                params = dict(e.params)
                if name == "swap":
                    params["lane0_only"] = True
                out(U, params=params)
                return
            if not idx:
                indices = [Slice(0, n, 1) for n in env[ref].aval.shape]
            else:
                indices = list(idx[0].indices)
            first = indices[0]
            if not (isinstance(first, Slice) and isinstance(first.start, int) and first.start == 0 and first.size == self.b):
                if name == "swap" and s_of(e.invars[1]) == L:
                    raise _Bail("lane value stored to a single row")
                params = dict(e.params)
                if name == "swap":
                    params["lane0_only"] = True
                out(U, params=params)
                return
            lane = self.lane(eqns)
            leaves: list[Any] = [lane]
            tmpl: list[Any] = [_Leaf(0)]
            for ix in indices[1:]:
                if isinstance(ix, Slice):
                    if isinstance(ix.start, (int,)):
                        tmpl.append(ix)
                    else:
                        leaves.append(a(ix.start))
                        tmpl.append(Slice(_Leaf(len(leaves) - 1), ix.size, ix.stride))
                else:
                    if s_of(ix) == L:
                        raise _Bail("lane-varying ref index")
                    leaves.append(a(ix))
                    tmpl.append(_Leaf(len(leaves) - 1))
            new_tree = IndexerTree(NDIndexer(tuple(tmpl), tuple(env[ref].aval.shape)), len(leaves))
            if name == "get":
                out(L, params={"tree": new_tree, "lane_row": True}, invars=[env[ref], *leaves])
            else:
                val = e.invars[1]
                vnew = a(val)
                out(L, params={"tree": new_tree, "lane_row": True}, invars=[env[ref], vnew, *leaves])
            return
        if name == "iota":
            dim = int(e.params["dimension"])
            shape = tuple(e.params["shape"])
            if shape and shape[0] == self.b:
                if dim == 0:
                    lane = self.lane(eqns)
                    nv = Var(self.per_lane(e.outvars[0].aval, L))
                    env[e.outvars[0]] = nv
                    st[e.outvars[0]] = L
                    if nv.aval.shape:
                        eqns.append(JaxprEqn([lane], [nv], primitive("broadcast_in_dim"),
                                             {"shape": nv.aval.shape, "broadcast_dimensions": (), "sharding": None}))
                    else:
                        eqns.append(JaxprEqn([lane], [nv], primitive("convert_element_type"),
                                             {"new_dtype": nv.aval.dtype, "weak_type": False}))
                    return
                out(L, params={**e.params, "shape": shape[1:], "dimension": dim - 1})
                return
            out(U)
            return
        if name == "broadcast_in_dim":
            shape = tuple(e.params["shape"])
            bd = tuple(e.params["broadcast_dimensions"])
            src = e.invars[0]
            if ins_st[0] == L:
                if not bd or bd[0] != 0:
                    raise _Bail("lane dim moved by broadcast")
                out(L, params={**e.params, "shape": shape[1:], "broadcast_dimensions": tuple(d - 1 for d in bd[1:])})
                return
            if shape and shape[0] == self.b:
                # Uniform -> every lane holds the broadcast row.
                sshape = () if isinstance(src, Literal) else tuple(src.aval.shape)
                if 0 in bd and sshape[bd.index(0)] != 1:
                    raise _Bail("uniform value with the lane dim")
                keep = [(k, d) for k, d in enumerate(bd) if d != 0]
                if len(keep) != len(bd):
                    raise _Bail("size-1 source dim mapped onto the lane dim")
                out(L, params={**e.params, "shape": shape[1:], "broadcast_dimensions": tuple(d - 1 for _, d in keep)})
                return
            out(U)
            return
        if name in ("reshape", "squeeze", "expand_dims"):
            if ins_st[0] == L:
                old, new = e.invars[0].aval.shape, e.outvars[0].aval.shape
                if not (old and new and old[0] == self.b and new[0] == self.b):
                    raise _Bail("reshape moves the lane dim")
                out(L, params={**e.params, "new_sizes": tuple(new[1:])})
                return
            out(U)
            return
        if name == "transpose":
            if ins_st[0] == L:
                perm = tuple(e.params["permutation"])
                if perm[0] != 0:
                    raise _Bail("transpose moves the lane dim")
                out(L, params={"permutation": tuple(p - 1 for p in perm[1:])})
                return
            out(U)
            return
        if name == "dot_general":
            (lc, rc), (lb, rb) = e.params["dimension_numbers"]
            if ins_st[1] == L or tuple(lb) or tuple(rb):
                raise _Bail("dot_general with a lane rhs or batch dims")
            if ins_st[0] == U:
                out(U)
                return
            lcd = [int(d) for d in lc]
            if 0 in lcd:
                raise _Bail("dot_general contracts over the lane dim")
            out(L, params={**e.params, "dimension_numbers": ((tuple(d - 1 for d in lcd), tuple(rc)), ((), ()))})
            return
        if name in _REDUCE:
            axes = tuple(int(x) for x in e.params["axes"])
            if ins_st[0] == U:
                out(U)
                return
            if 0 not in axes:
                out(L, params={**e.params, "axes": tuple(x - 1 for x in axes)})
                return
            rest = tuple(x - 1 for x in axes if x != 0)
            src = a(e.invars[0])
            if rest:
                mid = Var(ShapedArray(tuple(s for k, s in enumerate(src.aval.shape) if k not in rest), src.aval.dtype))
                eqns.append(JaxprEqn([src], [mid], primitive(name), {**e.params, "axes": rest}))
                src = mid
            if src.aval.shape:
                raise _Bail("cross-lane reduction of a non-scalar row")
            out(U, params={"kind": _REDUCE[name], "lanes": self.b}, invars=[src], prim="lane_reduce")
            return
        if name in ("program_id", "num_programs", "random_wrap", "random_unwrap", "random_fold_in", "random_bits"):
            if L in ins_st:
                raise _Bail(f"{name} of a lane value")
            out(U)
            return
        if name in ("pjit", "jit", "closed_call", "core_call", "custom_jvp_call", "custom_vjp_call"):
            inner = e.params.get("jaxpr") or e.params.get("call_jaxpr")
            body = getattr(inner, "jaxpr", inner)
            nb, outs_st = self.jaxpr(body, ins_st[-len(body.invars):], dict(ref_lane))
            self._bind_outs(e, env, st, eqns, outs_st, "pjit", {"jaxpr": ClosedJaxpr(nb, [])},
                            [a(x) for x in e.invars][-len(body.invars):])
            return
        if name == "scan":
            body = getattr(e.params["jaxpr"], "jaxpr", e.params["jaxpr"])
            nc = len(e.outvars)
            nconst = len(e.invars) - nc
            carry_st = ins_st[nconst:]
            for _ in range(len(carry_st) + 1):
                nb, outs_st = self.jaxpr(body, ins_st[:nconst] + carry_st, dict(ref_lane))
                merged = [L if L in (c, o) else U for c, o in zip(carry_st, outs_st)]
                if merged == carry_st:
                    break
                carry_st = merged
            for x, s0, s1 in zip(e.invars[nconst:], ins_st[nconst:], carry_st):
                if s0 != s1:
                    raise _Bail("uniform loop init promoted to a lane carry")
            self._bind_outs(e, env, st, eqns, carry_st, "scan", {**e.params, "jaxpr": ClosedJaxpr(nb, [])},
                            [a(x) for x in e.invars])
            return
        if name == "while":
            cn, bn = int(e.params["cond_nconsts"]), int(e.params["body_nconsts"])
            cj = getattr(e.params["cond_jaxpr"], "jaxpr", e.params["cond_jaxpr"])
            bj = getattr(e.params["body_jaxpr"], "jaxpr", e.params["body_jaxpr"])
            carry_st = ins_st[cn + bn:]
            for _ in range(len(carry_st) + 1):
                nb, outs_st = self.jaxpr(bj, ins_st[cn:cn + bn] + carry_st, dict(ref_lane))
                merged = [L if L in (c, o) else U for c, o in zip(carry_st, outs_st)]
                if merged == carry_st:
                    break
                carry_st = merged
            for s0, s1 in zip(ins_st[cn + bn:], carry_st):
                if s0 != s1:
                    raise _Bail("uniform loop init promoted to a lane carry")
            ncj, (pst,) = self.jaxpr(cj, ins_st[:cn] + carry_st, dict(ref_lane))
            if pst == L:
                raise _Bail("while condition varies across lanes")
            self._bind_outs(e, env, st, eqns, carry_st, "while",
                            {**e.params, "cond_jaxpr": ClosedJaxpr(ncj, []), "body_jaxpr": ClosedJaxpr(nb, [])},
                            [a(x) for x in e.invars])
            return
        if name == "cond":
            if ins_st[0] == L:
                raise _Bail("cond index varies across lanes")
            branches = e.params["branches"]
            results = [self.jaxpr(getattr(br, "jaxpr", br), ins_st[1:], dict(ref_lane)) for br in branches]
            outs_st = [L if any(r[1][k] == L for r in results) else U for k in range(len(e.outvars))]
            for r in results:
                if r[1] != outs_st:
                    raise _Bail("cond branches disagree on lane status")
            self._bind_outs(e, env, st, eqns, outs_st, "cond",
                            {**e.params, "branches": tuple(ClosedJaxpr(r[0], []) for r in results)},
                            [a(x) for x in e.invars])
            return
        raise _Bail(f"no lane rule for {name}")

    def _bind_outs(self, e, env, st, eqns, outs_st, prim, params, invars) -> None:
        nouts = []
        for ov, s in zip(e.outvars, outs_st):
            nv = Var(self.per_lane(ov.aval, s))
            env[ov] = nv
            st[ov] = s
            nouts.append(nv)
        eqns.append(JaxprEqn(invars, nouts, primitive(prim), params))


def lane_transform(spec: KernelSpec) -> LanePlan | None:
    """Per-lane rewrite of `spec.jaxpr`, or None when the kernel is not in
    lane-separable form."""
    found = _lane_count(spec)
    if found is None:
        return None
    b, lane_ops = found
    p = _Pass(b)
    ref_lane: dict[Any, bool] = {}
    for k, v in enumerate(spec.jaxpr.invars):
        ref_lane[v] = k in lane_ops
    try:
        nj, _ = p.jaxpr(spec.jaxpr, [U] * len(spec.jaxpr.invars), ref_lane)
    except _Bail:
        return None
    rows = _ragged_rows(spec, b, lane_ops, nj)
    if rows is False:
        return None
    return LanePlan(b, nj, lane_ops, rows)


def _uses(j: Jaxpr, names: set[str]) -> bool:
    for e in j.eqns:
        if e.primitive.name in names:
            return True
        for v in e.params.values():
            for sub in (v if isinstance(v, tuple) else (v,)):
                inner = getattr(sub, "jaxpr", sub)
                if isinstance(inner, Jaxpr) and _uses(inner, names):
                    return True
    return False


def _ragged_rows(spec: KernelSpec, b: int, lane_ops: tuple[int, ...], nj: Jaxpr) -> int | None | bool:
    """None when every lane block lies inside its array; the valid row
    count R when the last block of a 1-D grid runs past it (all lane
    operands of R rows, block i at rows [i*b, i*b + b), no cross-lane
    reduction, so rows are independent); False when blocks run past the
    arrays in any other way (not lowered)."""
    from palladium_amd.interpret import _grid_pids, eval_index_map

    operands = list(spec.inputs) + list(spec.outputs)
    if not lane_ops or not any(b * spec.num_programs > operands[k].array_shape[0] for k in lane_ops):
        return None
    if len(spec.grid) != 1:
        return False
    rows = {operands[k].array_shape[0] for k in lane_ops}
    if len(rows) != 1:
        return False
    (r,) = rows
    g = spec.grid[0]
    if not (g - 1) * b < r <= g * b:
        return False
    pids = _grid_pids(tuple(spec.grid))
    for k in lane_ops:
        if not (eval_index_map(operands[k], pids, spec.num_programs)[0] == pids[0]).all():
            return False
    if _uses(nj, {"lane_reduce"}):
        return False
    return r


def lanes_of(spec: KernelSpec) -> int:
    plan = lane_transform(spec)
    return plan.lanes if plan else 1


def workgroup_for(lanes: int, block: int | None) -> int:
    """Workgroup size for a lane plan: one instance per workgroup above 64
    lanes (cross-lane reductions then synchronise the whole workgroup);
    with 64 lanes, several single-wave instances share a workgroup."""
    if lanes > 64:
        return lanes
    b = block or 256
    return max(64, b - b % 64)


def flat_threads(spec: KernelSpec, lanes: int) -> int:
    return math.prod(spec.grid) * lanes
