/*
 * CPU oracle for palladium_amd's hot path. TEST INFRASTRUCTURE ONLY: it is
 * loaded by tests/, by __graft_entry__.smoke() and by bench.py's
 * cpu_baseline leg, as the checker, never by the product path.
 *
 * Each function restates, in plain C with IEEE single precision and no
 * contraction (built with -ffp-contract=off), the algorithm the reference
 * runs for that kernel, citing the reference file:line it follows. What
 * pins each function (known answers, float64 restatements, invariants) is
 * tested in tests/test_oracle.py, tests/test_oracle_sensitivity.py,
 * tests/test_golden.py and (the REPRODUCIBLE-mode restatements)
 * tests/test_reproducible.py.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <string.h>

/* Threads the OpenMP loops below use (the CPU baselines time 1 and all). */
void oracle_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int oracle_max_threads(void) { return omp_get_max_threads(); }

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

/* ------------------------------------------------------------------------
 * GBM Monte Carlo, one path per call index (examples/03_sde_montecarlo.py:
 * 97-119 restated with the configured counter layout): per step one
 * Threefry block over counter (path, step) gives two uint32; each becomes
 * a uniform through JAX's conversion; u1 is floored at 1e-7; Box-Muller
 * z = sqrt(-2 ln u1) cos(2 pi u2); s <- s * exp(drift + vol z).
 * Op order matches palladium_amd.workloads.gbm_kernel.
 * ---------------------------------------------------------------------- */
void oracle_gbm(long n_paths, long first_path, long n_steps, uint32_t k0, uint32_t k1,
                float s0, float strike, float drift, float vol, float two_pi,
                float *payoff) {
#pragma omp parallel for schedule(static)
  for (long p = 0; p < n_paths; ++p) {
    uint32_t path = (uint32_t)(first_path + p);
    float s = s0;
    for (long i = 0; i < n_steps; ++i) {
      uint32_t b0, b1;
      oracle_threefry2x32(k0, k1, path, (uint32_t)i, &b0, &b1);
      float u1 = oracle_bits_to_uniform(b0, 0.0f, 1.0f);
      u1 = fmaxf(u1, 1e-7f);
      float u2 = oracle_bits_to_uniform(b1, 0.0f, 1.0f);
      float l = logf(u1);
      float r = sqrtf(-2.0f * l);
      float c = cosf(two_pi * u2);
      float z = r * c;
      float e = expf(drift + vol * z);
      s = s * e;
    }
    float d = s - strike;
    payoff[p] = fmaxf(d, 0.0f);
  }
}

/* ------------------------------------------------------------------------
 * Deterministic pow, the same sequence as the SAFE-mode device ph_pow
 * (palladium_amd/emit/prelude.py): double-precision log2 via the atanh
 * series (coefficients carrying 2/ln 2) and 2^z via z = k + r reduction and a
 * degree-10 polynomial in r, all in IEEE double with explicit fma. Pinned
 * against libm pow in tests (correctly rounded on every sampled argument).
 * ---------------------------------------------------------------------- */
static double ph_log2_pos(double x) {
  int e;
  double m = frexp(x, &e);
  if (m < 0.70710678118654752440) { m = m * 2.0; e = e - 1; }
  /* (m - 1) times the correctly rounded reciprocal of m + 1: the device
     reaches the same reciprocal by Newton steps (emit/prelude.py). */
  double t = (m - 1.0) * (1.0 / (m + 1.0));
  double t2 = t * t;
  /* sum_{k=0..7} 2 t2^k / ((2k+1) ln 2) by Horner's rule (one constant per
     FMA, so no constant needs a register move first). |t| <= 0.1716, so the
     first omitted term is below 1.3e-13 of the sum. */
  double p = fma(0.19235933878519512, t2, 0.22195308321368667);
  p = fma(p, t2, 0.2623081892525388);
  p = fma(p, t2, 0.3205988979753252);
  p = fma(p, t2, 0.4121985831111324);
  p = fma(p, t2, 0.5770780163555853);
  p = fma(p, t2, 0.9617966939259756);
  p = fma(p, t2, 2.8853900817779268);
  return fma(t, p, (double)e);
}

static double ph_exp2_dbl(double z) {
  double kd = rint(z);
  double r = z - kd; /* exact */
  /* sum_{n=0..10} (ln 2)^n r^n / n! by Horner's rule. |r ln 2| <= 0.347,
     so the first omitted term is below 2.2e-13. */
  double p = fma(7.054911620801123e-09, r, 1.01780860092397e-07);
  p = fma(p, r, 1.321548679014431e-06);
  p = fma(p, r, 1.5252733804059841e-05);
  p = fma(p, r, 0.0001540353039338161);
  p = fma(p, r, 0.0013333558146428443);
  p = fma(p, r, 0.009618129107628477);
  p = fma(p, r, 0.05550410866482158);
  p = fma(p, r, 0.24022650695910072);
  p = fma(p, r, 0.6931471805599453);
  p = fma(p, r, 1.0);
  return ldexp(p, (int)kd);
}

/* ph_pow's base-only part (palladium_amd/emit/prelude.py:ph_pow_log):
   log2 |x| for a finite nonzero x, 0 otherwise. */
double oracle_pow_log(float x) {
  float ax = fabsf(x);
  return ph_log2_pos((double)((ax > 0.0f && ax < INFINITY) ? ax : 1.0f));
}

void oracle_pow_log_many(long n, const float *x, double *out) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) out[i] = oracle_pow_log(x[i]);
}

float oracle_pow(float x, float y) {
  if (y == 0.0f || x == 1.0f) return 1.0f;
  if (x != x || y != y) return x + y;
  float ax = fabsf(x);
  float ay = fabsf(y);
  int y_int = (ay < 16777216.0f) ? (truncf(y) == y) : 1;
  int y_odd = y_int && (ay < 16777216.0f) && (fmodf(ay, 2.0f) == 1.0f);
  if (x < 0.0f && !y_int && ax != INFINITY) return NAN;
  if (ay == INFINITY) {
    if (ax == 1.0f) return 1.0f;
    return ((ax > 1.0f) == (y > 0.0f)) ? INFINITY : 0.0f;
  }
  float sign = (signbit(x) && y_odd) ? -1.0f : 1.0f; /* -0 too: pow(-0, 3) = -0 */
  if (ax == 0.0f) return (y < 0.0f) ? sign * INFINITY : sign * 0.0f;
  if (ax == INFINITY) return (y < 0.0f) ? sign * 0.0f : sign * INFINITY;
  double z = (double)y * ph_log2_pos((double)ax);
  if (z > 129.0) return sign * INFINITY;
  if (z < -151.0) return sign * 0.0f;
  return sign * (float)ph_exp2_dbl(z);
}

void oracle_pow_many(long n, const float *x, const float *y, float *out) {
  for (long i = 0; i < n; ++i) out[i] = oracle_pow(x[i], y[i]);
}

/* ------------------------------------------------------------------------
 * Adaptive Bogacki-Shampine 3(2) with FSAL and a PI step controller on Van
 * der Pol, one trajectory per index, as tests/test_08_adaptive.py:76-122
 * (tableau, error norm, controller, dt clamp) but iterating while t < T1
 * (bounded by max_attempts). Op order matches
 * palladium_amd.workloads.bs3_vdp_kernel, statement for statement.
 * ---------------------------------------------------------------------- */
static inline void vdp_rhs(float mu, float x, float v, float *fx, float *fv) {
  float x2 = x * x;
  float a = 1.0f - x2;
  float b = mu * a;
  float c = b * v;
  *fx = v;
  *fv = c - x;
}

void oracle_bs3_vdp(long n, const float *x0, const float *v0, const float *mu_in,
                    float t1, float dt0, float rtol, float atol, long max_attempts,
                    float *to, float *xo, float *vo, int32_t *acc_out,
                    int32_t *rej_out) {
  const float coeff1 = (float)((0.3 + 0.4) / 3.0);
  const float coeff2 = (float)(-0.4 / 3.0);
  const float b1 = (float)(2.0 / 9.0), b2 = (float)(1.0 / 3.0), b3 = (float)(4.0 / 9.0);
  const float e1 = (float)(7.0 / 24.0), e2 = 0.25f, e3 = (float)(1.0 / 3.0), e4 = 0.125f;
#pragma omp parallel for schedule(dynamic, 64)
  for (long i = 0; i < n; ++i) {
    const float mu = mu_in[i];
    float x = x0[i], v = v0[i];
    float t = 0.0f, dt = dt0, prev = 1.0f;
    float k1x, k1v;
    vdp_rhs(mu, x, v, &k1x, &k1v);
    int32_t acc = 0, rej = 0, it = 0;
    while (t < t1 && it < max_attempts) {
      float rem = t1 - t;
      dt = fminf(dt, rem);
      float h = 0.5f * dt;
      float xa = x + h * k1x, va = v + h * k1v;
      float k2x, k2v;
      vdp_rhs(mu, xa, va, &k2x, &k2v);
      h = 0.75f * dt;
      xa = x + h * k2x; va = v + h * k2v;
      float k3x, k3v;
      vdp_rhs(mu, xa, va, &k3x, &k3v);
      float sx = b1 * k1x; sx = sx + b2 * k2x; sx = sx + b3 * k3x;
      float x3 = x + dt * sx;
      float sv = b1 * k1v; sv = sv + b2 * k2v; sv = sv + b3 * k3v;
      float v3 = v + dt * sv;
      float k4x, k4v;
      vdp_rhs(mu, x3, v3, &k4x, &k4v);
      float qx = e1 * k1x; qx = qx + e2 * k2x; qx = qx + e3 * k3x; qx = qx + e4 * k4x;
      float x2 = x + dt * qx;
      float qv = e1 * k1v; qv = qv + e2 * k2v; qv = qv + e3 * k3v; qv = qv + e4 * k4v;
      float v2 = v + dt * qv;
      float ex = x3 - x2, ev = v3 - v2;
      float nx = fabsf(ex) / (atol + rtol * fabsf(x3));
      float nv = fabsf(ev) / (atol + rtol * fabsf(v3));
      float err = fmaxf(nx, nv);
      int accept = err <= 1.0f;
      float tn = t + dt;
      float t2 = accept ? tn : t;
      float xn = accept ? x3 : x;
      float vn = accept ? v3 : v;
      float kx = accept ? k4x : k1x;
      float kv = accept ? k4v : k1v;
      err = fmaxf(err, 1e-9f);
      float inv = 1.0f / err;
      float f = 0.9f * oracle_pow(inv, coeff1);
      f = f * oracle_pow(prev, coeff2);
      float pn = accept ? inv : prev;
      float cl = fminf(10.0f, fmaxf(0.2f, f));
      dt = dt * cl;
      acc = acc + (accept ? 1 : 0);
      rej = rej + (accept ? 0 : 1);
      it = it + 1;
      t = t2; x = xn; v = vn; k1x = kx; k1v = kv; prev = pn;
    }
    to[i] = t; xo[i] = x; vo[i] = v; acc_out[i] = acc; rej_out[i] = rej;
  }
}

/* ------------------------------------------------------------------------
 * REPRODUCIBLE math mode (palladium_amd/emit/prelude.py, PH_MATH_MODE 3):
 * division a / b is a * RN(1/b); pow is the fast deterministic power below.
 * The device reaches RN(1/b) by a Newton step from the hardware estimate
 * (IEEE division where the result is not a normal number); the host divides
 * (the device sequence is checked against the IEEE quotient on every
 * float).
 * ---------------------------------------------------------------------- */
float oracle_rdiv(float a, float b) { return a * (1.0f / b); }

/* log2 x for a positive normal float x from its bits: x = m 2^e with m in
   [m0, 2 m0), m0 = 0x1.6a09e6p-1 (the float just above sqrt(1/2)),
   t = (m - 1) r with r ~ 1/(m + 1) from the quadratic R and two Newton
   steps, log2 m = t P(t^2) with P of degree 4, log2 x = e + t P by one fma
   (coefficients: oracle/gen_rpow_coeffs.py). */
double oracle_rpow_log(float x) {
  uint32_t bits;
  memcpy(&bits, &x, 4);
  uint32_t ix = bits - 0x3f3504f3u;
  int e = (int32_t)ix >> 23;
  uint32_t mb = (ix & 0x007fffffu) + 0x3f3504f3u;
  float m;
  memcpy(&m, &mb, 4);
  double dm = (double)m;
  double d = dm + 1.0;
  double r = fma(d, 0.116862893757792, -0.722444125812821);
  r = fma(r, d, 1.4777559273698688);
  double q = fma(-d, r, 1.0);
  r = fma(r, q, r);
  q = fma(-d, r, 1.0);
  r = fma(r, q, r);
  double t = (dm - 1.0) * r;
  double s = t * t;
  double p = fma(s, 0.3407120415619086, 0.41167376623771057);
  p = fma(p, s, 0.5770835660048659);
  p = fma(p, s, 0.9617966734515485);
  p = fma(p, s, 2.885390081789987);
  return fma(t, p, (double)e);
}

void oracle_rpow_log_many(long n, const float *x, double *out) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) out[i] = oracle_rpow_log(x[i]);
}

/* 2^z, z = k + r with |r| <= 1/2: Q(r) of degree 7 as two Horner halves
   joined by one fma with r^4, then scaled by 2^k. */
static double oracle_rexp2(double z) {
  double kd = rint(z);
  double r = z - kd;
  double r2 = r * r;
  double lo = fma(r, 0.055504109063258665, 0.24022651213498092);
  double hi = fma(r, 1.5303700711365693e-05, 0.00015469729214118296);
  lo = fma(lo, r, 0.6931471805568324);
  hi = fma(hi, r, 0.0013333478473685416);
  double r4 = r2 * r2;
  lo = fma(lo, r, 0.9999999999595618);
  hi = fma(hi, r, 0.009618025613318034);
  return ldexp(fma(hi, r4, lo), (int)kd);
}

/* x^y given lg = oracle_rpow_log(x): 2^(y lg) rounded once to float for a
   positive normal x and |y| < 8192; oracle_pow (with the C99 special
   cases) for every other operand. */
float oracle_rpow_with_log(float x, float y, double lg) {
  int normal_x = x >= 0x1p-126f && x <= 0x1.fffffep127f;
  if (!normal_x || !(fabsf(y) < 8192.0f)) return oracle_pow(x, y);
  return (float)oracle_rexp2((double)y * lg);
}

float oracle_rpow(float x, float y) { return oracle_rpow_with_log(x, y, oracle_rpow_log(x)); }

void oracle_rpow_many(long n, const float *x, const float *y, float *out) {
  for (long i = 0; i < n; ++i) out[i] = oracle_rpow(x[i], y[i]);
}

/* The REPRODUCIBLE mode's float log2 and exp2 (device: ph_dlog2f,
   ph_dexp2f): the double log2 and 2^z above, each rounded once to float.
   log2: NaN for NaN and negative x, -inf for +-0, +inf for +inf,
   log2(x 2^24) - 24 for a subnormal x. exp2: NaN for NaN, +inf or +0 for
   |x| >= 2^20. */
float oracle_dlog2f(float x) {
  if (x != x) return x;
  if (x < 0.0f) return NAN;
  if (x == 0.0f) return -INFINITY;
  if (x == INFINITY) return x;
  if (x < 0x1p-126f) return (float)(oracle_rpow_log(x * 0x1p24f) - 24.0);
  return (float)oracle_rpow_log(x);
}

float oracle_dexp2f(float x) {
  if (x != x) return x;
  if (!(fabsf(x) < 0x1p20f)) return x > 0.0f ? INFINITY : 0.0f;
  return (float)oracle_rexp2((double)x);
}

void oracle_dlog2f_many(long n, const float *x, float *out) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) out[i] = oracle_dlog2f(x[i]);
}

void oracle_dexp2f_many(long n, const float *x, float *out) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) out[i] = oracle_dexp2f(x[i]);
}

/* The REPRODUCIBLE mode's float exp, log, sin and cos (device: ph_dexpf,
   ph_dlogf, ph_dtrig in palladium_amd/emit/prelude.py).
   exp: 2^(x log2 e), the product rounded to double; NaN for NaN, +inf or
   +0 for |x| >= 2^19. log: the double log2 times ln 2; special operands as
   oracle_dlog2f. sin/cos: x = k pi/2 + r, k = rint(x 2/pi) and
   r = fma(-k, PIO2_LO, fma(-k, PIO2_HI, x)) for |x| < 2^20 (PIO2_HI carries
   33 bits, so the inner FMA is exact); beyond, the exact reduction
   x 2/pi mod 4 from a 96-bit window of the bits of 2/pi (x = M 2^e), kept
   to 2^-62; sin r = r S(r^2), cos r = C(r^2) (degree 5, from
   oracle/gen_rpow_coeffs.py) and the quadrant picks +-sin r or +-cos r;
   NaN for infinities and NaN. */
float oracle_dexpf(float x) {
  if (x != x) return x;
  if (!(fabsf(x) < 0x1p19f)) return x > 0.0f ? INFINITY : 0.0f;
  return (float)oracle_rexp2((double)x * 1.4426950408889634);
}

float oracle_dlogf(float x) {
  if (x != x) return x;
  if (x < 0.0f) return NAN;
  if (x == 0.0f) return -INFINITY;
  if (x == INFINITY) return x;
  if (x < 0x1p-126f) return (float)((oracle_rpow_log(x * 0x1p24f) - 24.0) * 0.6931471805599453);
  return (float)(oracle_rpow_log(x) * 0.6931471805599453);
}

static float dtrig_poly(double r, int q) {
  double s = r * r;
  double ps = fma(s, -2.47565580235085e-08, 2.7555271883000814e-06);
  double pc = fma(s, -2.717342886965949e-07, 2.47989287418407e-05);
  ps = fma(ps, s, -0.0001984126329834066);
  pc = fma(pc, s, -0.0013888880393711728);
  ps = fma(ps, s, 0.008333333323878053);
  pc = fma(pc, s, 0.04166666654390994);
  ps = fma(ps, s, -0.16666666666616684);
  pc = fma(pc, s, -0.4999999999935111);
  ps = fma(ps, s, 0.9999999999999957);
  pc = fma(pc, s, 0.9999999999999444);
  double v = (q & 1) ? pc : r * ps;
  return (float)((q & 2) ? -v : v);
}

static const uint32_t two_over_pi[7] = {0xA2F9836Eu, 0x4E441529u, 0xFC2757D1u, 0xF534DDC0u,
                                        0xDB629599u, 0x3C439041u, 0xFE5163ABu};

static float dtrig(float x, int off) {
  if (!(fabsf(x) < INFINITY)) return NAN;
  if (fabsf(x) < 0x1p20f) {
    double xd = (double)x;
    double k = rint(xd * 0.6366197723675814);
    double r = fma(-k, 0x1.921fb544p+0, xd);
    r = fma(-k, 0x1.0b4611a626331p-34, r);
    return dtrig_poly(r, (int)k + off);
  }
  uint32_t b;
  memcpy(&b, &x, 4);
  int e = (int)((b >> 23) & 0xffu) - 150;
  unsigned __int128 m = (b & 0x7fffffu) | 0x800000u;
  int i0 = e >= 2 ? e - 1 : 1;
  int j = (i0 - 1) >> 5, sh = (i0 - 1) & 31;
  unsigned __int128 w = ((unsigned __int128)two_over_pi[j] << 96) | ((unsigned __int128)two_over_pi[j + 1] << 64) |
                        ((unsigned __int128)two_over_pi[j + 2] << 32) | two_over_pi[j + 3];
  w = (w << sh) >> 32;
  int n = 97 - e + i0;
  unsigned __int128 p = (m * w) & ((((unsigned __int128)1) << n) - 1);
  int q = (int)(p >> (n - 2)) & 3;
  long long f = (long long)((uint64_t)(p >> (n - 64)) & ((1ull << 62) - 1));
  if (f >= (1ll << 61)) { f -= (1ll << 62); q += 1; }
  double r = (double)f * 0x1.921fb54442d18p-62;
  if (b >> 31) { r = -r; q = -q; }
  return dtrig_poly(r, q + off);
}

float oracle_dsinf(float x) { return dtrig(x, 0); }
float oracle_dcosf(float x) { return dtrig(x, 1); }

/* The REPRODUCIBLE mode's float tanh (device: ph_dtanhf): a = |x|; a T(a^2)
   below 1/2 (T of degree 7), else 1 - 2 / (e + 1) with e = 2^(2 log2(e)
   min(a, 10)) on the 2^z core and a double division; rounded once to float,
   the sign of x, NaN passed through. */
float oracle_dtanhf(float x) {
  if (x != x) return x;
  double a = fabs((double)x);
  double s = a * a;
  double p = fma(s, -0.0009849941049264166, 0.003415370282047567);
  p = fma(p, s, -0.008827257095239422);
  p = fma(p, s, 0.021865363235290286);
  p = fma(p, s, -0.053967994875471936);
  p = fma(p, s, 0.13333332529982497);
  p = fma(p, s, -0.33333333323808056);
  p = fma(p, s, 0.9999999999998141);
  double e = oracle_rexp2(fmin(a, 10.0) * 2.8853900817779268);
  double t = a < 0.5 ? a * p : 1.0 - 2.0 / (e + 1.0);
  return copysignf((float)t, x);
}

void oracle_dtanhf_many(long n, const float *x, float *out) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) out[i] = oracle_dtanhf(x[i]);
}

void oracle_dexpf_many(long n, const float *x, float *out) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) out[i] = oracle_dexpf(x[i]);
}
void oracle_dlogf_many(long n, const float *x, float *out) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) out[i] = oracle_dlogf(x[i]);
}
void oracle_dsinf_many(long n, const float *x, float *out) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) out[i] = oracle_dsinf(x[i]);
}
void oracle_dcosf_many(long n, const float *x, float *out) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) out[i] = oracle_dcosf(x[i]);
}

/* ------------------------------------------------------------------------
 * GBM Monte Carlo under the REPRODUCIBLE mode: the program FAST's rewrites
 * and the contraction pass make of palladium_amd.workloads.gbm_kernel's
 * step (the redundant clamp of each uniform at 0 dropped, drift + vol z as
 * one fmaf), with exp, log and cos the deterministic forms above and sqrtf
 * correctly rounded, statement for statement. Same counters, conversion
 * and layout as oracle_gbm.
 * ---------------------------------------------------------------------- */
void oracle_gbm_r(long n_paths, long first_path, long n_steps, uint32_t k0, uint32_t k1,
                  float s0, float strike, float drift, float vol, float two_pi,
                  float *payoff) {
#pragma omp parallel for schedule(static)
  for (long p = 0; p < n_paths; ++p) {
    uint32_t path = (uint32_t)(first_path + p);
    float s = s0;
    for (long i = 0; i < n_steps; ++i) {
      uint32_t b0, b1, f0, f1;
      oracle_threefry2x32(k0, k1, path, (uint32_t)i, &b0, &b1);
      f0 = (b0 >> 9) | 0x3f800000u;
      f1 = (b1 >> 9) | 0x3f800000u;
      float u1, u2;
      memcpy(&u1, &f0, 4);
      memcpy(&u2, &f1, 4);
      u1 = fmaxf(fmaf(u1 - 1.0f, 1.0f, 0.0f), 1e-7f);
      u2 = fmaf(u2 - 1.0f, 1.0f, 0.0f);
      float l = oracle_dlogf(u1);
      float r = sqrtf(-2.0f * l);
      float c = oracle_dcosf(two_pi * u2);
      float z = r * c;
      float e = oracle_dexpf(fmaf(vol, z, drift));
      s = s * e;
    }
    payoff[p] = fmaxf(s - strike, 0.0f);
  }
}

/* ------------------------------------------------------------------------
 * RK4 Lotka-Volterra under the REPRODUCIBLE mode: the program FAST's
 * rewrites make of the traced step (palladium_amd/emit/optimize.py:
 * factor_common_products, reuse_affine_shifts), with fmaf wherever the
 * product contraction fuses a single-use product into its add or
 * subtract. Per step, with h2 = f32(dt/2), h = f32(dt), h6 = f32(dt/6):
 *   A = a - b y, C = c x - d          (the rhs as x A, y C)
 *   stage k: the shifted state's A' = A - (b h_k) k_y, C' = C + (c h_k) k_x
 *   k4 fused into the weighted sums, x' = x + h6 ((k1 + 2 k2) + 2 k3 + k4)
 * statement for statement as the rewritten jaxpr.
 * ---------------------------------------------------------------------- */
void oracle_lv_rk4_r(long n, const float *x0, const float *y0, const float *a,
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
      float A = fmaf(-bi, y, ai);
      float k1x = x * A;
      float C = fmaf(ci, x, -di);
      float k1y = y * C;
      float xa = fmaf(h2, k1x, x);
      float ya = fmaf(h2, k1y, y);
      float A2 = fmaf(-(bi * h2), k1y, A);
      float k2x = xa * A2;
      float C2 = fmaf(ci * h2, k1x, C);
      float k2y = ya * C2;
      float xb = fmaf(h2, k2x, x);
      float yb = fmaf(h2, k2y, y);
      float A3 = fmaf(-(bi * h2), k2y, A);
      float k3x = xb * A3;
      float C3 = fmaf(ci * h2, k2x, C);
      float k3y = yb * C3;
      float xc = fmaf(h, k3x, x);
      float yc = fmaf(h, k3y, y);
      float A4 = fmaf(-(bi * h), k3y, A);
      float C4 = fmaf(ci * h, k3x, C);
      float sx = fmaf(2.0f, k2x, k1x);
      sx = fmaf(2.0f, k3x, sx);
      sx = fmaf(xc, A4, sx);
      float nx = fmaf(h6, sx, x);
      float sy = fmaf(2.0f, k2y, k1y);
      sy = fmaf(2.0f, k3y, sy);
      sy = fmaf(yc, C4, sy);
      float ny = fmaf(h6, sy, y);
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
 * The adaptive BS3(2)+PI Van der Pol loop of oracle_bs3_vdp under the
 * REPRODUCIBLE mode: the same statements, with fmaf wherever the emitter's
 * product contraction (palladium_amd/emit/optimize.py:contract_products)
 * fuses a single-use product into its add or subtract, both error-norm
 * divisions as a * RN(1/b), and the controller as FAST's power-law rewrite
 * makes it (power_laws_to_exp2, carry_logs): the factor is
 * 2^(log2 0.9 - c1 log2 err + c2 L) with L the carried log2 of
 * prev_inv_err, in the deterministic float log2 and exp2. Fused sites, in
 * the kernel's order:
 *   stage states      x + h k         -> fmaf(h, k, x)
 *   right-hand side   1 - x*x         -> fmaf(-x, x, 1)
 *                     (mu a) v - x    -> fmaf(mu a, v, -x)
 *   weighted sums     p1 + c2 k2      -> fmaf(c2, k2, p1), and so on
 *   updates           x + dt s        -> fmaf(dt, s, x)
 *   tolerance         atol + rtol|y|  -> fmaf(rtol, |y|, atol)
 *   controller        log2 0.9 - c1 le, then + c2 L -> two fmaf
 * ---------------------------------------------------------------------- */
static inline void vdp_rhs_r(float mu, float x, float v, float *fx, float *fv) {
  float a = fmaf(-x, x, 1.0f);
  float b = mu * a;
  *fx = v;
  *fv = fmaf(b, v, -x);
}

void oracle_bs3_vdp_r(long n, const float *x0, const float *v0, const float *mu_in,
                      float t1, float dt0, float rtol, float atol, long max_attempts,
                      float *to, float *xo, float *vo, int32_t *acc_out, int32_t *rej_out) {
  const float coeff1 = (float)((0.3 + 0.4) / 3.0);
  const float coeff2 = (float)(-0.4 / 3.0);
  const float log2_09 = -0x1.374d6ap-3f; /* f32(log2(f32(0.9))), as the rewrite folds it */
  const float b1 = (float)(2.0 / 9.0), b2 = (float)(1.0 / 3.0), b3 = (float)(4.0 / 9.0);
  const float e1 = (float)(7.0 / 24.0), e2 = 0.25f, e3 = (float)(1.0 / 3.0), e4 = 0.125f;
#pragma omp parallel for schedule(dynamic, 64)
  for (long i = 0; i < n; ++i) {
    const float mu = mu_in[i];
    float x = x0[i], v = v0[i];
    float t = 0.0f, dt = dt0;
    float prev_log = oracle_dlog2f(1.0f);
    float k1x, k1v;
    vdp_rhs_r(mu, x, v, &k1x, &k1v);
    int32_t acc = 0, rej = 0, it = 0;
    while (t < t1 && it < max_attempts) {
      float rem = t1 - t;
      dt = fminf(dt, rem);
      float h = 0.5f * dt;
      float xa = fmaf(h, k1x, x), va = fmaf(h, k1v, v);
      float k2x, k2v;
      vdp_rhs_r(mu, xa, va, &k2x, &k2v);
      h = 0.75f * dt;
      xa = fmaf(h, k2x, x);
      va = fmaf(h, k2v, v);
      float k3x, k3v;
      vdp_rhs_r(mu, xa, va, &k3x, &k3v);
      float sx = b1 * k1x; sx = fmaf(b2, k2x, sx); sx = fmaf(b3, k3x, sx);
      float x3 = fmaf(dt, sx, x);
      float sv = b1 * k1v; sv = fmaf(b2, k2v, sv); sv = fmaf(b3, k3v, sv);
      float v3 = fmaf(dt, sv, v);
      float k4x, k4v;
      vdp_rhs_r(mu, x3, v3, &k4x, &k4v);
      float qx = e1 * k1x; qx = fmaf(e2, k2x, qx); qx = fmaf(e3, k3x, qx); qx = fmaf(e4, k4x, qx);
      float x2 = fmaf(dt, qx, x);
      float qv = e1 * k1v; qv = fmaf(e2, k2v, qv); qv = fmaf(e3, k3v, qv); qv = fmaf(e4, k4v, qv);
      float v2 = fmaf(dt, qv, v);
      float ex = x3 - x2, ev = v3 - v2;
      float nx = oracle_rdiv(fabsf(ex), fmaf(rtol, fabsf(x3), atol));
      float nv = oracle_rdiv(fabsf(ev), fmaf(rtol, fabsf(v3), atol));
      float err = fmaxf(nx, nv);
      int accept = err <= 1.0f;
      float tn = t + dt;
      float t2 = accept ? tn : t;
      float xn = accept ? x3 : x;
      float vn = accept ? v3 : v;
      float kx = accept ? k4x : k1x;
      float kv = accept ? k4v : k1v;
      err = fmaxf(err, 1e-9f);
      /* 0.9 (1/err)^c1 prev^c2 as 2^(log2 0.9 - c1 log2 err + c2 log2 prev),
         the carry held as its log2 */
      float le = oracle_dlog2f(err);
      float z = fmaf(-coeff1, le, log2_09);
      z = fmaf(coeff2, prev_log, z);
      float f = oracle_dexp2f(z);
      float pln = accept ? -le : prev_log;
      float cl = fminf(10.0f, fmaxf(0.2f, f));
      dt = dt * cl;
      acc = acc + (accept ? 1 : 0);
      rej = rej + (accept ? 0 : 1);
      it = it + 1;
      t = t2; x = xn; v = vn; k1x = kx; k1v = kv; prev_log = pln;
    }
    to[i] = t; xo[i] = x; vo[i] = v; acc_out[i] = acc; rej_out[i] = rej;
  }
}

/* ------------------------------------------------------------------------
 * One Gray-Scott explicit Euler step on an n x n periodic grid, one cell per
 * index, as examples/04_reaction_diffusion.py:61-74: five-point Laplacian
 * ((((u[ip,j] + u[im,j]) + u[i,jp]) + u[i,jm]) - 4u), uvv = (u v) v,
 * u' = u + dt((Du lap_u - uvv) + F(1-u)), v' = v + dt((Dv lap_v + uvv) - (F+k) v).
 * ---------------------------------------------------------------------- */
void oracle_gray_scott_step(long n, const float *u, const float *v, float du, float dv,
                            float f, float fk, float dt, float *uo, float *vo) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) {
    long ip = (i == n - 1) ? 0 : i + 1;
    long im = (i == 0) ? n - 1 : i - 1;
    for (long j = 0; j < n; ++j) {
      long jp = (j == n - 1) ? 0 : j + 1;
      long jm = (j == 0) ? n - 1 : j - 1;
      float uc = u[i * n + j], vc = v[i * n + j];
      float lu = u[ip * n + j] + u[im * n + j];
      lu = lu + u[i * n + jp];
      lu = lu + u[i * n + jm];
      lu = lu - 4.0f * uc;
      float lv = v[ip * n + j] + v[im * n + j];
      lv = lv + v[i * n + jp];
      lv = lv + v[i * n + jm];
      lv = lv - 4.0f * vc;
      float uv = uc * vc;
      float uvv = uv * vc;
      float a = du * lu;
      a = a - uvv;
      float b = 1.0f - uc;
      b = f * b;
      a = a + b;
      uo[i * n + j] = uc + dt * a;
      float c = dv * lv;
      c = c + uvv;
      float d = fk * vc;
      c = c - d;
      vo[i * n + j] = vc + dt * c;
    }
  }
}

void oracle_gray_scott(long n, long steps, float *u, float *v, float *tmp_u, float *tmp_v,
                       float du, float dv, float f, float fk, float dt) {
  for (long s = 0; s < steps; ++s) {
    oracle_gray_scott_step(n, u, v, du, dv, f, fk, dt, tmp_u, tmp_v);
    memcpy(u, tmp_u, sizeof(float) * n * n);
    memcpy(v, tmp_v, sizeof(float) * n * n);
  }
}

/* ------------------------------------------------------------------------
 * df32 (double-float) arithmetic: a value is hi + lo with |lo| <= ulp(hi)/2.
 * Algorithms: TwoSum (Knuth), Fast2Sum (Dekker), TwoProd via FMA, and the
 * double-word operations of Joldes, Muller & Popescu, "Tight and rigorous
 * error bounds for basic building blocks of double-word arithmetic",
 * ACM TOMS 44(2), 2017: DWPlusDW (Alg. 6, "AccurateDWPlusDW") and
 * DWTimesDW (Alg. 12, FMA-based). The device prelude
 * (palladium_amd/df32.py) performs the same sequence.
 * Used by the df32 RK4 LV kernel (examples/05_df32_precision.py:27-80).
 * ---------------------------------------------------------------------- */
typedef struct { float hi, lo; } df32;

static inline df32 df_fast2sum(float a, float b) {
  float s = a + b;
  float z = s - a;
  df32 r = {s, b - z};
  return r;
}
static inline df32 df_twosum(float a, float b) {
  float s = a + b;
  float ap = s - b;
  float bp = s - ap;
  float da = a - ap;
  float db = b - bp;
  df32 r = {s, da + db};
  return r;
}
static inline df32 df_from_float(float a) { df32 r = {a, 0.0f}; return r; }
static inline float df_to_float(df32 a) { return a.hi + a.lo; }
static inline df32 df_add(df32 x, df32 y) {
  df32 s = df_twosum(x.hi, y.hi);
  df32 t = df_twosum(x.lo, y.lo);
  float c = s.lo + t.hi;
  df32 v = df_fast2sum(s.hi, c);
  float w = t.lo + v.lo;
  return df_fast2sum(v.hi, w);
}
static inline df32 df_neg(df32 a) { df32 r = {-a.hi, -a.lo}; return r; }
static inline df32 df_sub(df32 x, df32 y) { return df_add(x, df_neg(y)); }
static inline df32 df_mul(df32 x, df32 y) {
  float ch = x.hi * y.hi;
  float cl1 = fmaf(x.hi, y.hi, -ch);
  float tl0 = x.lo * y.lo;
  float tl1 = fmaf(x.hi, y.lo, tl0);
  float cl2 = fmaf(x.lo, y.hi, tl1);
  float cl3 = cl1 + cl2;
  return df_fast2sum(ch, cl3);
}

void oracle_df32_add(long n, const float *ah, const float *al, const float *bh, const float *bl,
                     float *oh, float *ol) {
  for (long i = 0; i < n; ++i) {
    df32 a = {ah[i], al[i]}, b = {bh[i], bl[i]};
    df32 r = df_add(a, b);
    oh[i] = r.hi; ol[i] = r.lo;
  }
}

void oracle_df32_mul(long n, const float *ah, const float *al, const float *bh, const float *bl,
                     float *oh, float *ol) {
  for (long i = 0; i < n; ++i) {
    df32 a = {ah[i], al[i]}, b = {bh[i], bl[i]};
    df32 r = df_mul(a, b);
    oh[i] = r.hi; ol[i] = r.lo;
  }
}

static inline void df_lv_rhs(df32 a, df32 b, df32 c, df32 d, df32 x, df32 y, df32 *fx, df32 *fy) {
  df32 xy = df_mul(x, y);
  *fx = df_sub(df_mul(a, x), df_mul(b, xy));
  *fy = df_sub(df_mul(c, xy), df_mul(d, y));
}

static inline df32 df_adv(df32 s, df32 k, df32 h) { return df_add(s, df_mul(h, k)); }

/* RK4 LV in df32, as examples/05_df32_precision.py:27-80 (the rhs groups
 * x*y once; stage constants 0.5*dt, dt, dt/6 and 2 enter as df32 of their
 * fp32 values). Outputs both words. */
void oracle_lv_rk4_df32(long n, const float *x0, const float *y0, const float *a_,
                        const float *b_, const float *c_, const float *d_, float dt,
                        long steps, float *xo_hi, float *xo_lo, float *yo_hi, float *yo_lo) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) {
    df32 a = df_from_float(a_[i]), b = df_from_float(b_[i]);
    df32 c = df_from_float(c_[i]), d = df_from_float(d_[i]);
    df32 half = df_from_float(0.5f * dt), full = df_from_float(dt);
    df32 sixth = df_from_float(dt / 6.0f), two = df_from_float(2.0f);
    df32 x = df_from_float(x0[i]), y = df_from_float(y0[i]);
    for (long s = 0; s < steps; ++s) {
      df32 k1x, k1y, k2x, k2y, k3x, k3y, k4x, k4y;
      df_lv_rhs(a, b, c, d, x, y, &k1x, &k1y);
      df_lv_rhs(a, b, c, d, df_adv(x, k1x, half), df_adv(y, k1y, half), &k2x, &k2y);
      df_lv_rhs(a, b, c, d, df_adv(x, k2x, half), df_adv(y, k2y, half), &k3x, &k3y);
      df_lv_rhs(a, b, c, d, df_adv(x, k3x, full), df_adv(y, k3y, full), &k4x, &k4y);
      df32 sx = df_add(df_add(df_add(k1x, df_mul(two, k2x)), df_mul(two, k3x)), k4x);
      df32 sy = df_add(df_add(df_add(k1y, df_mul(two, k2y)), df_mul(two, k3y)), k4y);
      x = df_adv(x, sx, sixth);
      y = df_adv(y, sy, sixth);
    }
    xo_hi[i] = x.hi; xo_lo[i] = x.lo; yo_hi[i] = y.hi; yo_lo[i] = y.lo;
  }
}
