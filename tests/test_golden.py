"""The committed golden fixtures (tests/golden/, written by make_fixtures.py)
against the oracle, the NumPy interpreter and the mathematics (CPU)."""

import dataclasses
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from oracle.ref64 import lv_rk4_f64
from palladium_amd.frontend import random
from palladium_amd.workloads import (
    BS3_CFG,
    GBM_CFG,
    GS_CFG,
    LV_CFG0,
    gbm_call,
    gray_scott_call,
    lv_inputs,
    lv_rk4_call,
)

GOLDEN = Path(__file__).parent / "golden"


def _npz(name):
    with np.load(GOLDEN / name) as z:
        return {k: z[k] for k in z.files}


def _hex(xs):
    return [int(x, 16) for x in xs]


def test_threefry_kats_and_bits():
    doc = json.loads((GOLDEN / "threefry_kat.json").read_text())
    for kat in doc["kats"]:
        assert list(oracle.threefry2x32(*_hex(kat["key"]), *_hex(kat["ctr"]))) == _hex(kat["out"])
    rb = doc["random_bits"]
    np.testing.assert_array_equal(oracle.random_bits(tuple(rb["key"]), rb["n"]), np.array(_hex(rb["bits"]), np.uint32))
    # bits[i] = x0 ^ x1 of threefry(key, (0, i)): restated from the definition.
    for i, b in enumerate(_hex(rb["bits"])):
        x0, x1 = oracle.threefry2x32(*rb["key"], 0, i)
        assert b == x0 ^ x1
    fi = doc["fold_in"]
    assert list(oracle.fold_in(tuple(fi["key"]), fi["data"])) == _hex(fi["out"])
    assert list(oracle.threefry2x32(*fi["key"], 0, fi["data"])) == _hex(fi["out"])
    for case in doc["bits_to_uniform"]:
        b = int(case["bits"], 16)
        u = float(oracle.bits_to_uniform(b))
        assert u == case["u"]
        # The top 23 bits as a mantissa in [1, 2), minus one: exactly (b >> 9) / 2**23.
        assert u == (b >> 9) / 2.0**23
        assert 0.0 <= u < 1.0


def test_lv_fixture():
    z = _npz("lv_rk4_small.npz")
    args = lv_inputs(z["x"].size, LV_CFG0.seed)
    np.testing.assert_array_equal(np.stack(args), z["inputs"])
    x, y, ymax = oracle.lv_rk4(*args, float(z["dt"]), int(z["steps"]), track_max=True)
    for got, name in ((x, "x"), (y, "y"), (ymax, "ymax")):
        np.testing.assert_array_equal(got, z[name], err_msg=name)
    # fp32 RK4 vs the float64 restatement: integration error only.
    np.testing.assert_allclose(z["x"], z["x64"], rtol=2e-4)
    np.testing.assert_allclose(z["y"], z["y64"], rtol=2e-4)
    assert np.all(z["ymax"] >= np.abs(z["y"]))  # running max over the post-step y values
    # The NumPy interpreter over the traced kernel follows the same op order.
    got = lv_rk4_call(x.size, float(z["dt"]), int(z["steps"]), track_max=True).interpret(*args)
    for g, name in zip(got, ("x", "y", "ymax")):
        np.testing.assert_array_equal(g, z[name], err_msg=name)


def test_lv_df32_fixture():
    z = _npz("lv_rk4_small.npz")
    dt, steps = float(z["dt"]), int(z["steps"])
    got = oracle.lv_rk4_df32(*z["inputs"], dt, steps)
    np.testing.assert_array_equal(np.stack(got), z["df32"])
    # The df32 kernel integrates with float32 step constants (dt, 0.5f*dt,
    # dt/6.0f), so its float64 counterpart uses those; df32 tracks it far
    # closer than fp32 does.
    d32 = np.float32(dt)
    consts = (float(np.float32(0.5) * d32), float(d32), float(d32 / np.float32(6.0)))
    x64, y64 = lv_rk4_f64(*z["inputs"], dt, steps, consts=consts)
    xh, xl, yh, yl = (v.astype(np.float64) for v in z["df32"])
    err_df = max(np.max(np.abs(xh + xl - x64) / np.abs(x64)), np.max(np.abs(yh + yl - y64) / np.abs(y64)))
    err_f32 = np.max(np.abs(z["x"] - x64) / np.abs(x64))
    assert err_df < 1e-9
    assert err_f32 > 1e3 * err_df


def test_bs3_fixture():
    z = _npz("bs3_small.npz")
    got = oracle.bs3_vdp(z["x0"], z["v0"], z["mu"], BS3_CFG)
    for g, name in zip(got, ("t", "x", "v", "accepted", "rejected")):
        np.testing.assert_array_equal(g, z[name], err_msg=name)
    assert np.all(z["t"] == np.float32(BS3_CFG.t1))
    assert np.all(z["accepted"] > 0) and z["accepted"].std() > 0
    # Stiffer oscillators (larger mu) need more steps on average.
    order = np.argsort(z["mu"])
    lo, hi = order[: len(order) // 4], order[-len(order) // 4 :]
    assert z["accepted"][hi].mean() > z["accepted"][lo].mean()


def test_gray_scott_fixture():
    z = _npz("gray_scott_64.npz")
    u, v = oracle.gray_scott(z["u0"], z["v0"], GS_CFG, int(z["steps"]))
    np.testing.assert_array_equal(u, z["u"])
    np.testing.assert_array_equal(v, z["v"])
    call = gray_scott_call(size=z["u0"].shape[0])
    u, v = z["u0"], z["v0"]
    for _ in range(int(z["steps"])):
        u, v = call.interpret(u, v)
    np.testing.assert_array_equal(u, z["u"])
    np.testing.assert_array_equal(v, z["v"])
    # Periodic boundary: shifting the initial condition shifts the result.
    su, sv = oracle.gray_scott(np.roll(z["u0"], (5, -3), (0, 1)), np.roll(z["v0"], (5, -3), (0, 1)), GS_CFG,
                               int(z["steps"]))
    np.testing.assert_array_equal(su, np.roll(z["u"], (5, -3), (0, 1)))
    np.testing.assert_array_equal(sv, np.roll(z["v"], (5, -3), (0, 1)))


def test_gbm_fixture():
    z = _npz("gbm_small.npz")
    cfg = dataclasses.replace(GBM_CFG, n_steps=int(z["n_steps"]))
    # libm transcendentals: the same machine reproduces the fixture exactly,
    # another glibc may differ in the last ulp.
    np.testing.assert_allclose(oracle.gbm(cfg, z["payoff"].size), z["payoff"], rtol=1e-5, atol=1e-4)
    got = gbm_call(cfg, n_paths=z["payoff"].size).interpret(random.key(cfg.seed))
    np.testing.assert_allclose(got, z["payoff"], rtol=1e-4, atol=1e-3)
    assert np.all(z["payoff"] >= 0)


@pytest.mark.parametrize("op", ["sum", "prod"])
def test_df32_fixture_is_exact(op):
    doc = json.loads((GOLDEN / "df32_ops.json").read_text())
    a = np.array([c["a"] for c in doc["cases"]], np.float32)
    b = np.array([c["b"] for c in doc["cases"]], np.float32)
    zero = np.zeros_like(a)
    hi, lo = (oracle.df32_add if op == "sum" else oracle.df32_mul)(a, zero, b, zero)
    want = np.array([c[op] for c in doc["cases"]], np.float32)
    np.testing.assert_array_equal(hi, want[:, 0])
    np.testing.assert_array_equal(lo, want[:, 1])
    # A sum or product of two floats is exact in float64, and the double-word
    # result must represent it exactly, with |lo| <= ulp(hi)/2.
    exact = np.array([c[f"{op}_exact"] for c in doc["cases"]])
    np.testing.assert_array_equal(hi.astype(np.float64) + lo.astype(np.float64), exact)
    assert np.all(np.abs(lo) <= np.spacing(np.abs(hi)) / 2)
