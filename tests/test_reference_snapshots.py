"""The reference's three other golden kernels (tests/test_msl_snapshots.py:
34-110 of the reference: conditional_loop, blocked_saxpy, copy_2d), pinned
by structure rather than text: our frontend must stage the same ops in the
same order, and our emitter must give every operand the same per-instance
offset (grid axis x stride) and block size, as the reference's blessed
Metal output. tests/golden/reference_snapshots.json holds those facts,
extracted from the Metal files by tests/golden/make_snapshot_structure.py."""

import json
import re
from pathlib import Path

import numpy as np
import pytest

from palladium_amd.emit import emit_hip
from palladium_amd.ir import Literal
from test_hip_snapshots import _blocked_saxpy, _conditional_loop, _copy_2d

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_snapshots.json").read_text())
BUILDERS = {"conditional_loop": _conditional_loop, "blocked_saxpy": _blocked_saxpy, "copy_2d": _copy_2d}


def _ops(jaxpr, names):
    """[primitive, operands...] of the float-valued eqns, operands
    normalised as the fixture does; loop-index bookkeeping and ref
    reads/writes are not ops."""
    ops = []
    for e in jaxpr.eqns:
        name = e.primitive.name
        if name == "get":
            names[e.outvars[0]] = names[e.invars[0]]
            continue
        if name in ("swap", "scan"):
            continue
        if np.dtype(e.outvars[0].aval.dtype).kind in "iu":
            continue

        def norm(a):
            if isinstance(a, Literal):
                return repr(float(a.val))
            return names[a]

        ops.append([name] + [norm(a) for a in e.invars])
        names[e.outvars[0]] = f"e{len(ops) - 1}"
    return ops


def _offsets(src):
    out = {}
    for m in re.finditer(r"(?:const )?float\* __restrict__ (arg\d+) = arg\d+_base(?: \+ (.+))?;", src):
        arg, expr = m.groups()
        terms = []
        if expr:
            for t in expr.split("+"):
                tm = re.match(r"\s*\(int\)\(_pid(\d)\) \* (\d+)\s*$", t)
                assert tm, f"unrecognised offset term {t!r}"
                terms.append([int(tm.group(1)), int(tm.group(2))])
        out[arg] = terms
    return out


@pytest.mark.parametrize("name", sorted(BUILDERS))
def test_offsets_match_reference(name):
    src = emit_hip(BUILDERS[name](), math_mode="safe")
    assert _offsets(src) == GOLDEN[name]["offsets"]


def test_conditional_loop_ops_and_trips():
    spec = _conditional_loop()
    g = GOLDEN["conditional_loop"]
    (scan,) = [e for e in spec.jaxpr.eqns if e.primitive.name == "scan"]
    assert scan.params["length"] == g["loop_trips"]
    body = scan.params["jaxpr"].jaxpr
    nc = scan.params["num_consts"]
    assert nc == 1  # r, read once before the loop as in the reference
    names = {body.invars[0]: "in1", body.invars[-1]: "carry"}
    assert _ops(body, names) == g["ops"]
    assert all(b.block_shape == (g["elements"],) for b in spec.inputs + spec.outputs)
    # the const is the second operand's block, the carry starts as the first's
    top = {e.outvars[0]: e.invars[0] for e in spec.jaxpr.eqns if e.primitive.name == "get"}
    refs = spec.jaxpr.invars
    assert top[scan.invars[0]] is refs[1]
    assert top[scan.invars[-1]] is refs[0]


def test_blocked_saxpy_ops_and_block():
    spec = _blocked_saxpy()
    g = GOLDEN["blocked_saxpy"]
    names = {spec.jaxpr.invars[0]: "in0", spec.jaxpr.invars[1]: "in1"}
    assert _ops(spec.jaxpr, names) == g["ops"]
    assert all(b.block_shape == (g["elements"],) for b in spec.inputs + spec.outputs)


def test_copy_2d_copies_every_element_once():
    spec = _copy_2d()
    g = GOLDEN["copy_2d"]
    assert _ops(spec.jaxpr, {spec.jaxpr.invars[0]: "in0"}) == g["ops"] == []
    assert int(np.prod(spec.inputs[0].block_shape)) == g["elements"]
    src = emit_hip(spec, math_mode="safe")
    src_arg, dst_arg = g["copy"]
    assert re.search(rf"{dst_arg}\[_i\d+\] = {src_arg}\[_i\d+\];", src)
    assert re.search(rf"< {g['elements']};", src)
