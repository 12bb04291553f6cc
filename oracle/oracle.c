/*
 * CPU oracle for palladium_amd's hot path. TEST INFRASTRUCTURE ONLY: it is
 * loaded by tests/, by __graft_entry__.smoke() and by bench.py's
 * cpu_baseline leg, as the checker, never by the product path.
 *
 * Each function restates, in plain C with IEEE single precision and no
 * contraction (built with -ffp-contract=off), the algorithm the reference
 * runs for that kernel, citing the reference file:line it follows. The
 * parity pinning of each function is listed in oracle/README.md.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------------
 * RK4 Lotka-Volterra, op for op as the reference's staged kernel body:
 * tests/golden/rk4_lotka_volterra.metal:55-293 (examples/01_ode_ensembles.py
 * :72-103). h2 = f32(0.5*dt), h = f32(dt), h6 = f32(dt/6) are the constants
 * Python folds before JAX sees them.
 * ---------------------------------------------------------------------- */
static inline void lv_rhs(float a, float b, float c, float d, float x, float y,
                          float *fx, float *fy) {
  float ax = a * x;
  float bx = b * x;
  float bxy = bx * y;
  *fx = ax - bxy;
  float cx = c * x;
  float cxy = cx * y;
  float dy = d * y;
  *fy = cxy - dy;
}

void oracle_lv_rk4(long n, const float *x0, const float *y0, const float *a,
                   const float *b, const float *c, const float *d, double dt,
                   long steps, float *xo, float *yo, float *ymax) {
  const float h2 = (float)(0.5 * dt);
  const float h = (float)dt;
  const float h6 = (float)(dt / 6.0);
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) {
    float x = x0[i], y = y0[i];
    const float ai = a[i], bi = b[i], ci = c[i], di = d[i];
    float m = fabsf(y);
    for (long s = 0; s < steps; ++s) {
      float k1x, k1y, k2x, k2y, k3x, k3y, k4x, k4y;
      lv_rhs(ai, bi, ci, di, x, y, &k1x, &k1y);
      float t1 = h2 * k1x, t2 = h2 * k1y;
      lv_rhs(ai, bi, ci, di, x + t1, y + t2, &k2x, &k2y);
      t1 = h2 * k2x; t2 = h2 * k2y;
      lv_rhs(ai, bi, ci, di, x + t1, y + t2, &k3x, &k3y);
      t1 = h * k3x; t2 = h * k3y;
      lv_rhs(ai, bi, ci, di, x + t1, y + t2, &k4x, &k4y);
      float sx = k1x + 2.0f * k2x;
      sx = sx + 2.0f * k3x;
      sx = sx + k4x;
      float nx = x + h6 * sx;
      float sy = k1y + 2.0f * k2y;
      sy = sy + 2.0f * k3y;
      sy = sy + k4y;
      float ny = y + h6 * sy;
      x = nx;
      y = ny;
      m = fmaxf(m, fabsf(y));
    }
    xo[i] = x;
    yo[i] = y;
    if (ymax) ymax[i] = m;
  }
}

/* ------------------------------------------------------------------------
 * Threefry-2x32-20 (Salmon, Moraes, Dror, Shaw, SC'11), as emitted by the
 * reference (src/palladium/emit/rules.py:121-165): rotation sets
 * (13,15,26,6) and (17,29,16,24), ks2 = k0 ^ k1 ^ 0x1BD11BDA, key injection
 * with round counter after every 4 rounds.
 * ---------------------------------------------------------------------- */
static inline uint32_t rotl(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

void oracle_threefry2x32(uint32_t k0, uint32_t k1, uint32_t c0, uint32_t c1,
                         uint32_t *o0, uint32_t *o1) {
  static const int R[8] = {13, 15, 26, 6, 17, 29, 16, 24};
  uint32_t ks[3] = {k0, k1, k0 ^ k1 ^ 0x1BD11BDAu};
  uint32_t x0 = c0 + ks[0], x1 = c1 + ks[1];
  for (int g = 0; g < 5; ++g) {
    for (int r = 0; r < 4; ++r) {
      x0 += x1;
      x1 = rotl(x1, R[(g & 1) * 4 + r]);
      x1 ^= x0;
    }
    x0 += ks[(g + 1) % 3];
    x1 += ks[(g + 2) % 3] + (uint32_t)(g + 1);
  }
  *o0 = x0;
  *o1 = x1;
}

/* jax.random.bits(key, (n,)): element i hashes counter (0, i), returns
 * x0 ^ x1 (src/palladium/emit/rules.py:168-185). */
void oracle_random_bits(uint32_t k0, uint32_t k1, long n, uint32_t *out) {
  for (long i = 0; i < n; ++i) {
    uint32_t a, b;
    oracle_threefry2x32(k0, k1, 0u, (uint32_t)i, &a, &b);
    out[i] = a ^ b;
  }
}

/* jax.random.fold_in: new key = threefry(key, (0, data))
 * (src/palladium/emit/rules.py:188-201). */
void oracle_fold_in(uint32_t k0, uint32_t k1, uint32_t data, uint32_t *n0, uint32_t *n1) {
  oracle_threefry2x32(k0, k1, 0u, data, n0, n1);
}

/* jax.random.uniform's float conversion of one uint32
 * (tests/test_10_random_bits.py:42-54): (bits >> 9) | 0x3F800000 as a float
 * in [1,2), minus 1, times (max-min), plus min, clamped below by min. */
float oracle_bits_to_uniform(uint32_t bits, float lo, float hi) {
  uint32_t fb = (bits >> 9) | 0x3F800000u;
  float f;
  memcpy(&f, &fb, 4);
  f = f - 1.0f;
  f = f * (hi - lo);
  f = f + lo;
  return fmaxf(lo, f);
}
