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
/* x * c for a float c (a df32 whose lo word is +0): DWTimesDW with y.lo = 0
   reduces exactly to this, bit for bit, for nonzero finite operands (the
   dropped terms are x.lo * 0 and fma(x.hi, 0, that), signed zeros only). */
__device__ __forceinline__ df32 df_mul_f(df32 x, float c) {
    float ch = x.hi * c;
    float cl1 = __builtin_fmaf(x.hi, c, -ch);
    float cl2 = x.lo * c;
    float cl3 = cl1 + cl2;
    return df_fast2sum(ch, cl3);
}
/* 2 * x is exact in both words (barring overflow), and equals
   DWTimesDW(x, 2) bit for bit. */
__device__ __forceinline__ df32 df_twice(df32 x) { df32 r; r.hi = 2.0f * x.hi; r.lo = 2.0f * x.lo; return r; }
__device__ __forceinline__ df32 operator+(df32 a, df32 b) { return df_add(a, b); }
__device__ __forceinline__ df32 operator-(df32 a, df32 b) { return df_sub(a, b); }
__device__ __forceinline__ df32 operator*(df32 a, df32 b) { return df_mul(a, b); }
"""

LV_DF32_SOURCE = DF32_PRELUDE + r"""
struct LVState { df32 x, y; };

/* The parameters and step sizes are floats (df32 with lo = 0): their
   products use df_mul_f, which equals the general df_mul on them exactly. */
__device__ __forceinline__ LVState lv_rhs(LVState s, float a, float b, float c, float d) {
    df32 xy = s.x * s.y;
    LVState r; r.x = df_mul_f(s.x, a) - df_mul_f(xy, b); r.y = df_mul_f(xy, c) - df_mul_f(s.y, d); return r;
}
__device__ __forceinline__ LVState lv_adv(LVState s, LVState k, float h) {
    LVState r; r.x = s.x + df_mul_f(k.x, h); r.y = s.y + df_mul_f(k.y, h); return r;
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
    const float a = a_[i], b = b_[i], c = c_[i], d = d_[i];
    const float half = 0.5f * dt, full = dt, sixth = dt / 6.0f;
    LVState s; s.x = df_from_float(x0[i]); s.y = df_from_float(y0[i]);
    for (unsigned int k = 0; k < steps; ++k) {
        LVState k1 = lv_rhs(s, a, b, c, d);
        LVState k2 = lv_rhs(lv_adv(s, k1, half), a, b, c, d);
        LVState k3 = lv_rhs(lv_adv(s, k2, half), a, b, c, d);
        LVState k4 = lv_rhs(lv_adv(s, k3, full), a, b, c, d);
        LVState sum;
        sum.x = k1.x + df_twice(k2.x) + df_twice(k3.x) + k4.x;
        sum.y = k1.y + df_twice(k2.y) + df_twice(k3.y) + k4.y;
        s = lv_adv(s, sum, sixth);
    }
    xo_hi[i] = s.x.hi; xo_lo[i] = s.x.lo;
    yo_hi[i] = s.y.hi; yo_lo[i] = s.y.lo;
}
"""

# float32 operations per df32 operation as written above (FMA = 2):
# df_add = 2 TwoSum (6 each) + 2 adds + 2 Fast2Sum (3 each) = 20;
# df_mul = 2 muls + 3 FMAs + 1 add + 1 Fast2Sum = 12;
# df_mul_f (df32 x float) = 2 muls + 1 FMA + 1 add + 1 Fast2Sum = 8;
# df_twice = 2 muls.
DF_ADD_FLOPS = 20
DF_MUL_FLOPS = 12
DF_MUL_F_FLOPS = 8
DF_TWICE_FLOPS = 2
# One RK4 step of lv_rk4_df32: four rhs (x*y shared: 1 df_mul + 4 df_mul_f
# + 2 df_add each), four stage/final updates (2 df_mul_f + 2 df_add each),
# the weighted sums (4 df_twice + 6 df_add): 58 df32 operations.
LV_DF32_MULS_PER_STEP = 4
LV_DF32_MUL_FS_PER_STEP = 24
LV_DF32_TWICES_PER_STEP = 4
LV_DF32_ADDS_PER_STEP = 22
LV_DF32_FLOPS_PER_STEP = (LV_DF32_MULS_PER_STEP * DF_MUL_FLOPS + LV_DF32_MUL_FS_PER_STEP * DF_MUL_F_FLOPS
                          + LV_DF32_TWICES_PER_STEP * DF_TWICE_FLOPS + LV_DF32_ADDS_PER_STEP * DF_ADD_FLOPS)

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
