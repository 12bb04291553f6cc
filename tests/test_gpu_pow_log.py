"""The deterministic pow's base-only part, `ph_pow_log` (SAFE prelude), on
the GPU against the C oracle's `oracle_pow_log`, bit for bit, for every
float mantissa: the device takes the reciprocal of m + 1 by Newton steps
from the hardware float reciprocal, the oracle by a division, and both must
give RN(1 / (m + 1)) for each of the 2^23 mantissas (x in [0.5, 1) reaches
every m the reduction produces), plus subnormals, powers of two, special
values and a random sample over the whole float range; and the whole SAFE
`ph_pow` (the direct 2^z path for positive finite bases with z in
[-151, 129], the C99 special cases in a branch) against `oracle_pow`."""

import numpy as np
import pytest

import oracle
from palladium_amd import runtime as rt
from palladium_amd.emit.prelude import PRELUDE

pytestmark = pytest.mark.gpu

SRC = PRELUDE + r"""
extern "C" __global__ void __launch_bounds__(256)
pow_log_all(const float* __restrict__ x, double* __restrict__ out, unsigned int n)
{
    const unsigned int i = blockIdx.x * 256u + threadIdx.x;
    if (i < n) out[i] = ph_pow_log(x[i]);
}
"""


def _device(x: np.ndarray) -> np.ndarray:
    k = rt.Kernel(SRC, "pow_log_all", "safe")
    xb = rt.Buffer.from_numpy(np.ascontiguousarray(x, np.float32))
    ob = rt.Buffer.empty((x.size,), np.float64)
    rt.run(k, x.size, [xb, ob], [np.uint32(x.size)])
    return ob.to_numpy()


def test_every_mantissa():
    bits = np.arange(0x3F000000, 0x3F800000, dtype=np.uint32)      # [0.5, 1): all 2^23 mantissas
    x = bits.view(np.float32)
    print(f"[pow_log] {x.size} mantissas", flush=True)
    got, want = _device(x), oracle.pow_log(x)
    bad = np.flatnonzero(got.view(np.uint64) != want.view(np.uint64))
    assert bad.size == 0, f"{bad.size} mismatches, first at x={x[bad[0]]!r}: {got[bad[0]]!r} != {want[bad[0]]!r}"


def test_special_and_scattered_bases():
    r = np.random.default_rng(11)
    x = np.concatenate([
        r.integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 2.0, 0.5, 1e-45, -1e-45, 1.17549435e-38,
                  3.4028235e38, 0.70710677, 0.7071068, 1.4142135, 1.4142137], np.float32),
        np.ldexp(np.float32(1.0), np.arange(-149, 128)).astype(np.float32),
    ])
    got, want = _device(x), oracle.pow_log(x)
    np.testing.assert_array_equal(got.view(np.uint64), want.view(np.uint64))


POW_SRC = PRELUDE + r"""
extern "C" __global__ void __launch_bounds__(256)
pow_all(const float* __restrict__ x, const float* __restrict__ y, float* __restrict__ out, unsigned int n)
{
    const unsigned int i = blockIdx.x * 256u + threadIdx.x;
    if (i < n) out[i] = ph_pow(x[i], y[i]);
}
"""


def test_safe_pow_against_the_oracle():
    r = np.random.default_rng(12)
    n = 1 << 20
    special = np.array([0.0, -0.0, 1.0, -1.0, 2.0, 0.5, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1.17549435e-38,
                        3.4028235e38, 16777216.0, 16777217.0, 3.0, -3.0, 0.25, 1e10, 1e-10, 129.0, -151.0,
                        150.0, -150.0, 128.0, -149.0], np.float32)
    base = np.concatenate([
        r.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32),
        (10.0 ** r.uniform(-9, 9, n)).astype(np.float32),
        np.full(4096, 2.0, np.float32), np.full(4096, 0.5, np.float32),
        np.repeat(special, special.size),
    ])
    expo = np.concatenate([
        r.uniform(-4, 4, n).astype(np.float32),
        r.uniform(-1, 1, n).astype(np.float32),
        # z = y log2 x right at and around the direct path's limits
        (np.float32(129.0) + np.arange(-2048, 2048, dtype=np.float32) * np.float32(2.0 ** -12)),
        (np.float32(151.0) + np.arange(-2048, 2048, dtype=np.float32) * np.float32(2.0 ** -12)),
        np.tile(special, special.size),
    ])
    print(f"[pow] SAFE ph_pow over {base.size} pairs", flush=True)
    k = rt.Kernel(POW_SRC, "pow_all", "safe")
    xb = rt.Buffer.from_numpy(base)
    yb = rt.Buffer.from_numpy(expo)
    ob = rt.Buffer.empty((base.size,), np.float32)
    rt.run(k, base.size, [xb, yb, ob], [np.uint32(base.size)])
    got, want = ob.to_numpy(), oracle.pow_many(base, expo)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    bad = np.flatnonzero(~same)
    assert bad.size == 0, f"{bad.size} mismatches, e.g. pow({base[bad[0]]!r}, {expo[bad[0]]!r}) = {got[bad[0]]!r} != {want[bad[0]]!r}"
