"""The deterministic pow's base-only part, `ph_pow_log` (SAFE prelude), on
the GPU against the C oracle's `oracle_pow_log`, bit for bit, for every
float mantissa: the device takes the reciprocal of m + 1 by Newton steps
from the hardware float reciprocal, the oracle by a division, and both must
give RN(1 / (m + 1)) for each of the 2^23 mantissas (x in [0.5, 1) reaches
every m the reduction produces), plus subnormals, powers of two, special
values and a random sample over the whole float range."""

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
