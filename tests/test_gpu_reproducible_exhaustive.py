"""The REPRODUCIBLE float functions on every one of the 2^32 float inputs:
the device's ph_dexpf, ph_dlogf, ph_dtrig (sine and cosine), ph_dtanhf,
ph_dlog2f and ph_dexp2f against their C restatements in oracle/oracle.c,
bit for bit (any NaN matching any NaN), and the double logs inside the two
deterministic pows (SAFE's ph_pow_log, REPRODUCIBLE's ph_rpow_log). The host side takes one to two
minutes on 16 cores, so the test runs only with PALLADIUM_EXHAUSTIVE=1; the
regular suite samples the same functions (tests/test_gpu_reproducible.py)."""

import os

import numpy as np
import pytest

import oracle
from palladium_amd import runtime as rt
from palladium_amd.emit.prelude import PRELUDE

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(os.environ.get("PALLADIUM_EXHAUSTIVE") != "1",
                                 reason="2^32 inputs: set PALLADIUM_EXHAUSTIVE=1")]

NAMES = ("dexpf", "dlogf", "dsinf", "dcosf", "dtanhf", "dlog2f", "dexp2f")

SRC = PRELUDE + r"""
extern "C" __global__ void __launch_bounds__(256)
every_float(float* __restrict__ o0, float* __restrict__ o1, float* __restrict__ o2, float* __restrict__ o3,
            float* __restrict__ o4, float* __restrict__ o5, float* __restrict__ o6,
            double* __restrict__ d0, double* __restrict__ d1, unsigned int base)
{
    const unsigned int i = blockIdx.x * 256u + threadIdx.x;
    const float x = __uint_as_float(base + i);
    o0[i] = ph_dexpf(x);
    o1[i] = ph_dlogf(x);
    o2[i] = ph_dtrig(x, 0);
    o3[i] = ph_dtrig(x, 1);
    o4[i] = ph_dtanhf(x);
    o5[i] = ph_dlog2f(x);
    o6[i] = ph_dexp2f(x);
    d0[i] = ph_pow_log(x);
    d1[i] = ph_rpow_log(x);
}
"""


def test_every_float_input():
    chunk = 1 << 26
    k = rt.Kernel(SRC, "every_float", "reproducible")
    outs = [rt.Buffer.empty((chunk,), np.float32) for _ in NAMES]
    logs = [rt.Buffer.empty((chunk,), np.float64) for _ in range(2)]
    bad = {n: 0 for n in NAMES}
    first = {}
    for c in range((1 << 32) // chunk):
        base = c * chunk
        rt.run(k, (chunk // 256,), outs + logs, [np.uint32(base)])
        x = np.arange(base, base + chunk, dtype=np.uint64).astype(np.uint32).view(np.float32)
        for name, ob in zip(NAMES, outs):
            got = ob.to_numpy()
            want = getattr(oracle, name)(x)
            diff = (got.view(np.uint32) != want.view(np.uint32)) & ~(np.isnan(got) & np.isnan(want))
            nb = int(diff.sum())
            if nb:
                bad[name] += nb
                first.setdefault(name, hex(int(x.view(np.uint32)[np.flatnonzero(diff)[0]])))
        for name, ob, ref in (("pow_log", logs[0], oracle.pow_log), ("rpow_log", logs[1], oracle.rpow_log_many)):
            got = ob.to_numpy()
            want = ref(x)
            diff = (got.view(np.uint64) != want.view(np.uint64)) & ~(np.isnan(got) & np.isnan(want))
            nb = int(diff.sum())
            if nb:
                bad[name] = bad.get(name, 0) + nb
                first.setdefault(name, hex(int(x.view(np.uint32)[np.flatnonzero(diff)[0]])))
        print(f"[exhaustive] chunk {c + 1}/{(1 << 32) // chunk} done, mismatches so far {sum(bad.values())}", flush=True)
    assert sum(bad.values()) == 0, f"mismatches {bad}, first inputs {first}"
