"""Every element-wise primitive on a grid of special values, device
against interpreter under SAFE (tests/edge_cases.py): 625 float pairs
through 27 outputs, 256 int32 pairs through 21."""

import numpy as np
import pytest

import edge_cases as ec

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", ["float", "int"])
def test_edge_values_match_interpreter(kind):
    pairs = ec.float_pairs() if kind == "float" else ec.int_pairs()
    n, args = ec.pad64(*pairs)
    names, call = (ec.float_call if kind == "float" else ec.int_call)(args[0].size)
    bad = [name for name, g, w in zip(names, call(*args), call.interpret(*args)) if not ec.same(g[:n], w[:n])]
    assert not bad, bad


def test_transcendentals_on_special_values():
    """exp/log/pow/trig on the same grid under SAFE: special results
    (NaN, signed infinities and zeros, domain errors) equal the
    interpreter's, finite ones within 4 float32 ulps (device libm against
    NumPy's)."""
    n, args = ec.pad64(*ec.float_pairs())
    names, call = ec.transcendental_call(args[0].size)
    bad = [name for name, g, w in zip(names, call(*args), call.interpret(*args)) if not ec.close(g[:n], w[:n])]
    assert not bad, bad
