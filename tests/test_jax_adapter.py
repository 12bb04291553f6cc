"""`jax_adapter.convert_jaxpr` without JAX: kernel jaxprs traced by the
native frontend are re-expressed as duck-typed stand-ins for JAX's objects
(`jax.extend.core.Literal`, `AbstractRef` avals, `key<fry>` dtypes, closed
jaxprs in params, indexer treedefs producing `pl.Slice`/NDIndexer), the
adapter converts them back, and the emitted HIP must be identical to the
native path's. A faithful adapter loses nothing on the way."""

import dataclasses
import sys
import types

import numpy as np
import pytest

from palladium_amd import dtypes, ir
from palladium_amd.emit import emit_hip
from palladium_amd.frontend import random
from palladium_amd.trace import trace


class FakeShaped:
    def __init__(self, shape, dtype, weak_type=False):
        self.shape, self.dtype, self.weak_type = tuple(shape), np.dtype(dtype), weak_type


class AbstractRef:
    def __init__(self, inner):
        self.inner_aval = inner
        self.shape, self.dtype = inner.shape, inner.dtype


class FakeKeyDtype:
    def __str__(self):
        return "key<fry>"


class FakeKey:
    def __init__(self, shape):
        self.shape, self.dtype = tuple(shape), FakeKeyDtype()


class FakeVar:
    def __init__(self, aval):
        self.aval = aval


class FakeLiteral:
    def __init__(self, val, aval):
        self.val, self.aval = val, aval


class FakePrim:
    def __init__(self, name):
        self.name = name


@dataclasses.dataclass
class FakeEqn:
    invars: list
    outvars: list
    primitive: FakePrim
    params: dict


@dataclasses.dataclass
class FakeJaxpr:
    constvars: list
    invars: list
    outvars: list
    eqns: list


@dataclasses.dataclass
class FakeClosed:
    jaxpr: FakeJaxpr
    consts: list


@dataclasses.dataclass
class FakeSlice:
    start: object
    size: int
    stride: int = 1


@dataclasses.dataclass
class FakeNDIndexer:
    indices: tuple
    shape: tuple


class FakeTreedef:
    """Plays JAX's indexer treedef: unflatten gives pl.Slice-based indexers."""

    def __init__(self, tree):
        self.tree = tree

    def unflatten(self, leaves):
        out = []
        for idx in self.tree.unflatten(leaves):
            ind = tuple(FakeSlice(i.start, i.size, i.stride) if isinstance(i, ir.Slice) else i for i in idx.indices)
            out.append(FakeNDIndexer(ind, idx.shape))
        return tuple(out)


def _fake_aval(a):
    if isinstance(a, ir.RefAval):
        return AbstractRef(FakeShaped(a.shape, a.dtype))
    if isinstance(a, ir.KeyAval):
        return FakeKey(a.shape)
    return FakeShaped(a.shape, a.dtype, a.weak_type)


class _Jaxify:
    def __init__(self):
        self.vars = {}

    def atom(self, x):
        if isinstance(x, ir.Literal):
            if dtypes.is_bf16(x.aval.dtype):  # JAX holds bf16 literals as ml_dtypes scalars
                return FakeLiteral(dtypes.from_float(np.float32(x.val)).reshape(()), _fake_aval(x.aval))
            return FakeLiteral(np.asarray(x.val, dtype=x.aval.dtype), _fake_aval(x.aval))
        if x not in self.vars:
            self.vars[x] = FakeVar(_fake_aval(x.aval))
        return self.vars[x]

    def params(self, p):
        out = {}
        for k, v in p.items():
            if isinstance(v, ir.ClosedJaxpr):
                out[k] = FakeClosed(self.jaxpr(v.jaxpr), [])
            elif isinstance(v, ir.Jaxpr):
                out[k] = self.jaxpr(v)
            elif k == "branches":
                out[k] = tuple(FakeClosed(self.jaxpr(b.jaxpr), []) for b in v)
            elif k == "tree":
                out[k] = FakeTreedef(v)
            else:
                out[k] = v
        return out

    def jaxpr(self, j):
        return FakeJaxpr([], [self.atom(v) for v in j.invars], [self.atom(v) for v in j.outvars],
                         [FakeEqn([self.atom(a) for a in e.invars], [self.atom(o) for o in e.outvars],
                                  FakePrim(e.primitive.name), self.params(e.params)) for e in j.eqns])


@pytest.fixture
def fake_jax(monkeypatch):
    jax = types.ModuleType("jax")
    extend = types.ModuleType("jax.extend")
    core = types.ModuleType("jax.extend.core")
    core.Literal = FakeLiteral
    experimental = types.ModuleType("jax.experimental")
    pallas = types.ModuleType("jax.experimental.pallas")
    pallas.Slice = FakeSlice
    jax.extend, extend.core, jax.experimental, experimental.pallas = extend, core, experimental, pallas
    for name, mod in (("jax", jax), ("jax.extend", extend), ("jax.extend.core", core),
                      ("jax.experimental", experimental), ("jax.experimental.pallas", pallas)):
        monkeypatch.setitem(sys.modules, name, mod)


def _specs():
    from fuzz_vec import make_call, make_inputs
    from palladium_amd.workloads import (
        BS3_CFG, GBM_CFG, bs3_inputs, bs3_vdp_call, gbm_call, gray_scott_call, gray_scott_initial,
        lv_inputs, lv_rk4_call,
    )

    yield "lv_rk4", trace(lv_rk4_call(64, 0.01, 10, track_max=True)._staged, *lv_inputs(64, 0))
    yield "bs3_vdp", trace(bs3_vdp_call(64, BS3_CFG)._staged, *bs3_inputs(64))
    yield "gbm", trace(gbm_call(GBM_CFG, n_paths=64)._staged, random.key(42))
    yield "gray_scott", trace(gray_scott_call(size=64)._staged, *gray_scott_initial(64))
    yield "fuzz_vec_lanes", trace(make_call(3, rows=128, lanes=True)._staged, *make_inputs(3, rows=128))
    yield "fuzz_vec_instance", trace(make_call(4, rows=128)._staged, *make_inputs(4, rows=128))
    for dt, tag in ((dtypes.bfloat16, "bf16"), (np.float16, "f16")):
        yield f"fuzz_vec_lanes_{tag}", trace(make_call(5, rows=128, lanes=True, dtype=dt)._staged,
                                              *make_inputs(5, rows=128, dtype=dt))
        yield f"fuzz_vec_instance_{tag}", trace(make_call(6, rows=128, dtype=dt)._staged, *make_inputs(6, rows=128, dtype=dt))


@pytest.mark.parametrize("name,spec", list(_specs()), ids=lambda x: x if isinstance(x, str) else "")
def test_converted_jaxpr_emits_identical_hip(fake_jax, name, spec):
    from palladium_amd.jax_adapter import convert_jaxpr

    converted = convert_jaxpr(_Jaxify().jaxpr(spec.jaxpr))
    again = dataclasses.replace(spec, jaxpr=converted)
    for mode in ("safe", "fast"):
        assert emit_hip(again, math_mode=mode) == emit_hip(spec, math_mode=mode), name


def test_captured_constants_are_rejected(fake_jax):
    from palladium_amd.errors import TraceError
    from palladium_amd.jax_adapter import convert_jaxpr

    j = FakeJaxpr([FakeVar(FakeShaped((4,), np.float32))], [], [], [])
    with pytest.raises(TraceError, match="captures 1 array"):
        convert_jaxpr(j)
