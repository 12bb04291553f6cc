"""df32 (double-float) arithmetic for HIP kernels, and the df32 RK4 LV kernel.

The reference reaches compensated arithmetic through metal-runtime's df32
prelude and a hand-written kernel (`examples/05_df32_precision.py:27-80,
155`), because the jnp frontend has no df32 dtype. This module is that
prelude for gfx950, written from the published algorithms:

- TwoSum (Knuth) and Fast2Sum (Dekker) for exact sums,
- TwoProd via FMA for exact products,
- DWPlusDW ("AccurateDWPlusDW", Alg. 6) and DWTimesDW (FMA-based, Alg. 12)
  of Joldes, Muller & Popescu, ACM TOMS 44(2), 2017.

A df32 value is `hi + lo`, |lo| <= ulp(hi)/2. Kernels using it must compile
under SAFE math: contraction or reassociation would cancel the error terms.
`lv_rk4_df32` runs the RK4 Lotka-Volterra ensemble with every operation in
df32, one trajectory per lane, and returns both words of the result.
"""

from __future__ import annotations

import numpy as np

from palladium_amd import runtime as rt

DF32_PRELUDE = r"""
struct df32 { float hi, lo; };

__device__ __forceinline__ df32 df_fast2sum(float a, float b) {
    float s = a + b;
    float z = s - a;
    df32 r; r.hi = s; r.lo = b - z; return r;
}
__device__ __forceinline__ df32 df_twosum(float a, float b) {
    float s = a + b;
    float ap = s - b;
    float bp = s - ap;
    float da = a - ap;
    float db = b - bp;
    df32 r; r.hi = s; r.lo = da + db; return r;
}
__device__ __forceinline__ df32 df_from_float(float a) { df32 r; r.hi = a; r.lo = 0.0f; return r; }
__device__ __forceinline__ float df_to_float(df32 a) { return a.hi + a.lo; }
__device__ __forceinline__ df32 df_add(df32 x, df32 y) {
    df32 s = df_twosum(x.hi, y.hi);
    df32 t = df_twosum(x.lo, y.lo);
    float c = s.lo + t.hi;
    df32 v = df_fast2sum(s.hi, c);
    float w = t.lo + v.lo;
    return df_fast2sum(v.hi, w);
}
__device__ __forceinline__ df32 df_neg(df32 a) { df32 r; r.hi = -a.hi; r.lo = -a.lo; return r; }
__device__ __forceinline__ df32 df_sub(df32 x, df32 y) { return df_add(x, df_neg(y)); }
__device__ __forceinline__ df32 df_mul(df32 x, df32 y) {
    float ch = x.hi * y.hi;
    float cl1 = __builtin_fmaf(x.hi, y.hi, -ch);
    float tl0 = x.lo * y.lo;
    float tl1 = __builtin_fmaf(x.hi, y.lo, tl0);
    float cl2 = __builtin_fmaf(x.lo, y.hi, tl1);
    float cl3 = cl1 + cl2;
    return df_fast2sum(ch, cl3);
}
__device__ __forceinline__ df32 operator+(df32 a, df32 b) { return df_add(a, b); }
__device__ __forceinline__ df32 operator-(df32 a, df32 b) { return df_sub(a, b); }
__device__ __forceinline__ df32 operator*(df32 a, df32 b) { return df_mul(a, b); }
"""

LV_DF32_SOURCE = DF32_PRELUDE + r"""
struct LVState { df32 x, y; };

__device__ __forceinline__ LVState lv_rhs(LVState s, df32 a, df32 b, df32 c, df32 d) {
    df32 xy = s.x * s.y;
    LVState r; r.x = a * s.x - b * xy; r.y = c * xy - d * s.y; return r;
}
__device__ __forceinline__ LVState lv_adv(LVState s, LVState k, df32 h) {
    LVState r; r.x = s.x + h * k.x; r.y = s.y + h * k.y; return r;
}

extern "C" __global__ void __launch_bounds__(256)
lv_rk4_df32(const float* __restrict__ x0, const float* __restrict__ y0,
            const float* __restrict__ a_, const float* __restrict__ b_,
            const float* __restrict__ c_, const float* __restrict__ d_,
            float* __restrict__ xo_hi, float* __restrict__ xo_lo,
            float* __restrict__ yo_hi, float* __restrict__ yo_lo,
            float dt, unsigned int steps, unsigned int n)
{
    const unsigned int i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    df32 a = df_from_float(a_[i]), b = df_from_float(b_[i]);
    df32 c = df_from_float(c_[i]), d = df_from_float(d_[i]);
    df32 half = df_from_float(0.5f * dt), full = df_from_float(dt);
    df32 sixth = df_from_float(dt / 6.0f), two = df_from_float(2.0f);
    LVState s; s.x = df_from_float(x0[i]); s.y = df_from_float(y0[i]);
    for (unsigned int k = 0; k < steps; ++k) {
        LVState k1 = lv_rhs(s, a, b, c, d);
        LVState k2 = lv_rhs(lv_adv(s, k1, half), a, b, c, d);
        LVState k3 = lv_rhs(lv_adv(s, k2, half), a, b, c, d);
        LVState k4 = lv_rhs(lv_adv(s, k3, full), a, b, c, d);
        LVState sum;
        sum.x = k1.x + two * k2.x + two * k3.x + k4.x;
        sum.y = k1.y + two * k2.y + two * k3.y + k4.y;
        s = lv_adv(s, sum, sixth);
    }
    xo_hi[i] = s.x.hi; xo_lo[i] = s.x.lo;
    yo_hi[i] = s.y.hi; yo_lo[i] = s.y.lo;
}
"""

# float32 operations per df32 operation as written above (FMA = 2):
# df_add = 2 TwoSum (6 each) + 2 adds + 2 Fast2Sum (3 each) = 20;
# df_mul = 2 muls + 3 FMAs + 1 add + 1 Fast2Sum = 12.
DF_ADD_FLOPS = 20
DF_MUL_FLOPS = 12
# One RK4 step of lv_rk4_df32: four rhs (5 muls, 2 adds: x*y is shared),
# four stage/final updates (2 muls, 2 adds), the weighted sums (4 muls,
# 6 adds): 32 df_mul + 22 df_add.
LV_DF32_MULS_PER_STEP = 32
LV_DF32_ADDS_PER_STEP = 22
LV_DF32_FLOPS_PER_STEP = LV_DF32_MULS_PER_STEP * DF_MUL_FLOPS + LV_DF32_ADDS_PER_STEP * DF_ADD_FLOPS

_kernel: rt.Kernel | None = None


def lv_kernel() -> rt.Kernel:
    """The df32 LV kernel, compiled under SAFE math."""
    global _kernel
    if _kernel is None:
        _kernel = rt.Kernel(LV_DF32_SOURCE, "lv_rk4_df32", rt.MathMode.SAFE)
    return _kernel


def lv_rk4_df32_device(bufs_in, bufs_out, dt: float, steps: int, n: int, stream=None) -> None:
    """Launch on device buffers: 6 inputs, 4 outputs (x_hi, x_lo, y_hi, y_lo)."""
    blocks = (n + 255) // 256
    lv_kernel().launch((blocks,), (256,), [*bufs_in, *bufs_out, np.float32(dt), np.uint32(steps), np.uint32(n)], stream)


def lv_rk4_df32(x0, y0, a, b, c, d, dt: float, steps: int):
    """NumPy in/out: returns (x_hi, x_lo, y_hi, y_lo)."""
    host = [np.ascontiguousarray(v, np.float32) for v in (x0, y0, a, b, c, d)]
    n = host[0].size
    ins = [rt.Buffer.from_numpy(h) for h in host]
    outs = [rt.Buffer.empty((n,), np.float32) for _ in range(4)]
    stream = rt.Stream()
    lv_rk4_df32_device(ins, outs, dt, steps, n, stream)
    return tuple(o.to_numpy(stream) for o in outs)
