"""The GPU path against the committed golden fixtures (tests/golden/).

SAFE math keeps the traced IEEE op order, so LV, BS3 (states and step
counts), Gray-Scott and the Threefry bits must match the fixtures bit for
bit; GBM payoffs pass through transcendentals and are held to a tolerance."""

import dataclasses
import json
from pathlib import Path

import numpy as np
import pytest

import palladium_amd as pa
from palladium_amd.frontend import pl, random
from palladium_amd.df32 import lv_rk4_df32
from palladium_amd.workloads import (
    BS3_CFG,
    GBM_CFG,
    bs3_vdp_call,
    gbm_call,
    gray_scott_call,
    gray_scott_run,
    lv_rk4_call,
)

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).parent / "golden"


def _npz(name):
    with np.load(GOLDEN / name) as z:
        return {k: z[k] for k in z.files}


def _hex(xs):
    return np.array([int(x, 16) for x in xs], np.uint32)


def test_threefry_kats_on_device():
    doc = json.loads((GOLDEN / "threefry_kat.json").read_text())
    kats = doc["kats"]
    n = len(kats)

    def kernel(k_ref, c_ref, o0_ref, o1_ref):
        o0_ref[0], o1_ref[0] = random.threefry2x32_p(k_ref[0], k_ref[1], c_ref[0], c_ref[1])

    f = pa.hip_call(kernel, grid=(n,), in_specs=[pl.BlockSpec((2,), lambda i: (i,))] * 2,
                    out_specs=(pl.BlockSpec((1,), lambda i: (i,)),) * 2,
                    out_shape=(pl.ShapeDtypeStruct((n,), np.uint32),) * 2)
    keys = np.concatenate([_hex(k["key"]) for k in kats])
    ctrs = np.concatenate([_hex(k["ctr"]) for k in kats])
    o0, o1 = f(keys, ctrs)
    want = np.stack([_hex(k["out"]) for k in kats])
    np.testing.assert_array_equal(o0, want[:, 0])
    np.testing.assert_array_equal(o1, want[:, 1])


def test_random_bits_fixture_on_device():
    doc = json.loads((GOLDEN / "threefry_kat.json").read_text())
    rb = doc["random_bits"]

    def kernel(k_ref, bits_ref, fold_ref):
        key = random.wrap_key_data(k_ref[...])
        bits_ref[...] = random.bits(key, (rb["n"],))
        fold_ref[...] = random.key_data(random.fold_in(key, doc["fold_in"]["data"]))

    f = pa.hip_call(kernel, out_shape=(pl.ShapeDtypeStruct((rb["n"],), np.uint32),
                                       pl.ShapeDtypeStruct((2,), np.uint32)), math_mode="safe")
    bits, folded = f(np.array(rb["key"], np.uint32))
    np.testing.assert_array_equal(bits, _hex(rb["bits"]))
    np.testing.assert_array_equal(folded, _hex(doc["fold_in"]["out"]))


@pytest.mark.parametrize("block", [1, 64])
def test_lv_fixture_on_device(block):
    z = _npz("lv_rk4_small.npz")
    n = z["x"].size
    f = lv_rk4_call(n, float(z["dt"]), int(z["steps"]), track_max=True, block=block, math_mode="safe")
    got = f(*z["inputs"])
    for g, name in zip(got, ("x", "y", "ymax")):
        np.testing.assert_array_equal(g, z[name], err_msg=name)


def test_bs3_fixture_on_device():
    z = _npz("bs3_small.npz")
    got = bs3_vdp_call(z["x0"].size, BS3_CFG, math_mode="safe")(z["x0"], z["v0"], z["mu"])
    for g, name in zip(got, ("t", "x", "v", "accepted", "rejected")):
        np.testing.assert_array_equal(g, z[name], err_msg=name)


def test_gray_scott_fixture_on_device():
    z = _npz("gray_scott_64.npz")
    call = gray_scott_call(size=z["u0"].shape[0], math_mode="safe")
    u, v, _ = gray_scott_run(call, z["u0"], z["v0"], int(z["steps"]))
    np.testing.assert_array_equal(u, z["u"])
    np.testing.assert_array_equal(v, z["v"])


def test_gbm_fixture_on_device():
    z = _npz("gbm_small.npz")
    cfg = dataclasses.replace(GBM_CFG, n_steps=int(z["n_steps"]))
    got = gbm_call(cfg, n_paths=z["payoff"].size, math_mode="safe")(random.key(cfg.seed))
    np.testing.assert_allclose(got, z["payoff"], rtol=2e-5, atol=2e-4)


def test_df32_lv_fixture_on_device():
    z = _npz("lv_rk4_small.npz")
    got = lv_rk4_df32(*z["inputs"], float(z["dt"]), int(z["steps"]))
    np.testing.assert_array_equal(np.stack(got), z["df32"])
