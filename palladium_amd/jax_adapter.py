"""Trace a real `jax.experimental.pallas.pallas_call` into palladium_amd's IR.

Only used where JAX is importable (it is not in the build container, so this
module is exercised on machines with jax installed). It follows the
reference tracer (`src/palladium/trace.py:117-177`): `jax.make_jaxpr`, find
the single `pallas_call` equation, reject scalar prefetch, read the grid and
block mappings; then it converts the kernel jaxpr and the index-map jaxprs
into `palladium_amd.ir` objects (same attribute names), mapping JAX avals to
ShapedArray / RefAval / KeyAval and JAX's get/swap indexer treedefs to
IndexerTree-compatible wrappers.
"""

from __future__ import annotations

from typing import Any

import numpy as np

from palladium_amd import ir
from palladium_amd.dtypes import is_bf16, to_float
from palladium_amd.errors import TraceError
from palladium_amd.trace import BlockInfo, KernelSpec

__all__ = ["convert_jaxpr", "trace_jax"]


def _aval(a: Any) -> ir.ShapedArray:
    dtype = getattr(a, "dtype", None)
    name = type(a).__name__
    if "Ref" in name:
        inner = getattr(a, "inner_aval", a)
        return ir.RefAval(tuple(inner.shape), inner.dtype)
    if dtype is not None and "key" in str(dtype):
        return ir.KeyAval(tuple(a.shape))
    return ir.ShapedArray(tuple(a.shape), np.dtype(dtype), bool(getattr(a, "weak_type", False)))


class _JaxTree:
    """Wraps a JAX indexer treedef; unflatten returns palladium_amd NDIndexers."""

    def __init__(self, treedef: Any):
        self.treedef = treedef

    def unflatten(self, leaves: list[Any]) -> tuple[ir.NDIndexer, ...]:
        import jax.experimental.pallas as pl

        out = self.treedef.unflatten(list(leaves))
        res = []
        for idx in out:
            indices = []
            for i in idx.indices:
                if isinstance(i, pl.Slice):
                    indices.append(ir.Slice(i.start, int(i.size), int(i.stride)))
                else:
                    indices.append(i)
            res.append(ir.NDIndexer(tuple(indices), tuple(int(s) for s in idx.shape)))
        return tuple(res)


class _Converter:
    def __init__(self) -> None:
        self.vars: dict[Any, ir.Var] = {}

    def atom(self, a: Any) -> Any:
        from jax.extend.core import Literal

        if isinstance(a, Literal):
            val = np.asarray(a.val)
            if is_bf16(val.dtype):  # an ml_dtypes (or surrogate) bfloat16 scalar
                return ir.Literal(float(to_float(val).reshape(())), _aval(a.aval))
            return ir.Literal(val.item(), _aval(a.aval))
        v = self.vars.get(a)
        if v is None:
            v = self.vars[a] = ir.Var(_aval(a.aval))
        return v

    def params(self, eqn: Any) -> dict[str, Any]:
        p = dict(eqn.params)
        for k, v in list(p.items()):
            if hasattr(v, "jaxpr") and hasattr(v, "consts"):
                if v.consts:
                    raise TraceError(f"{eqn.primitive.name}: closed-over constants are not supported")
                p[k] = ir.ClosedJaxpr(self.jaxpr(v.jaxpr), [])
            elif k == "branches":
                p[k] = tuple(ir.ClosedJaxpr(self.jaxpr(b.jaxpr), []) for b in v)
            elif k == "tree":
                p[k] = _JaxTree(v)
            elif k in ("jaxpr", "call_jaxpr") and hasattr(v, "eqns"):
                p[k] = self.jaxpr(v)
        return p

    def jaxpr(self, j: Any) -> ir.Jaxpr:
        if j.constvars:
            raise TraceError(
                f"the kernel captures {len(j.constvars)} array(s) from its enclosing scope; "
                "a kernel may close over Python scalars, and arrays must be passed in as operands"
            )
        invars = [self.atom(v) for v in j.invars]
        eqns = []
        for e in j.eqns:
            ins = [self.atom(a) for a in e.invars]
            outs = [self.atom(o) for o in e.outvars]
            eqns.append(ir.JaxprEqn(ins, outs, ir.primitive(e.primitive.name), self.params(e)))
        return ir.Jaxpr([], invars, [self.atom(o) for o in j.outvars], eqns)


def convert_jaxpr(j: Any) -> ir.Jaxpr:
    return _Converter().jaxpr(j)


def _block_dim(dim: Any) -> int | None:
    import jax.experimental.pallas as pl

    if isinstance(dim, (int, np.integer)):
        return int(dim)
    if dim is None or isinstance(dim, getattr(pl, "Squeezed", ())):
        return None
    if isinstance(dim, getattr(pl, "Blocked", ())):
        return int(dim.block_size)
    raise TraceError(
        f"unsupported block dim type {type(dim).__name__}: only int, pl.Blocked, and pl.Squeezed "
        "dims are lowered (pl.Element, pl.Indirect, and pl.BoundedSlice indexing is unimplemented)"
    )


def trace_jax(pallas_fn: Any, *example_args: Any) -> KernelSpec:
    import jax

    closed = jax.make_jaxpr(pallas_fn)(*example_args)
    eqns = [e for e in closed.jaxpr.eqns if e.primitive.name == "pallas_call"]
    if not eqns:
        raise TraceError("no pallas_call equation found; pass the callable returned by pl.pallas_call")
    if len(eqns) > 1:
        raise TraceError(f"found {len(eqns)} pallas_call equations; trace them separately")
    params = dict(eqns[0].params)
    gm = params["grid_mapping"]
    if gm.num_index_operands:
        raise TraceError("PrefetchScalarGridSpec is not supported")
    kj = params["jaxpr"]
    kj = getattr(kj, "jaxpr", kj)
    n_in, n_out = gm.num_inputs, gm.num_outputs
    conv = _Converter()

    def infos(mappings) -> tuple[BlockInfo, ...]:
        out = []
        for bm in mappings:
            dims = [_block_dim(d) for d in bm.block_shape]
            imj = bm.index_map_jaxpr
            out.append(BlockInfo(
                block_shape=tuple(d for d in dims if d is not None),
                array_shape=tuple(bm.array_aval.shape),
                dtype=np.dtype(bm.array_aval.dtype),
                index_map_jaxpr=ir.ClosedJaxpr(_Converter().jaxpr(imj.jaxpr), []),
                full_block_shape=tuple(1 if d is None else d for d in dims),
            ))
        return tuple(out)

    mappings = list(gm.block_mappings)
    grid = tuple(int(g) for g in gm.grid) or (1,)
    nsi = params.get("name_and_src_info")  # newer JAX: NameAndSrcInfo(name=...)
    name = params.get("name") or getattr(nsi, "name", None) or "palladium_kernel"
    return KernelSpec(
        name=name if str(name).isidentifier() else "palladium_kernel",
        jaxpr=conv.jaxpr(kj),
        grid=grid,
        inputs=infos(mappings[:n_in]),
        outputs=infos(mappings[n_in : n_in + n_out]),
        raw_params={"grid": grid},
    )
