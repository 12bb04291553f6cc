"""Device-side helpers prepended to every emitted kernel.

- `ph_threefry2x32`: Threefry-2x32 with 20 rounds (Salmon et al., SC'11),
  the generator behind `jax.random` and the reference's emitted RNG
  (`src/palladium/emit/rules.py:121-165`): rotations (13,15,26,6) /
  (17,29,16,24), key schedule k0, k1, k0^k1^0x1BD11BDA with a round
  counter added every four rounds.
- `ph_pow`: under SAFE math (`PH_MATH_MODE == 0`) a deterministic power
  function built only from IEEE double add/mul/div/fma, so a host build of
  the same sequence returns bit-identical results; this is what makes
  adaptive accept/reject decisions reproducible on the CPU. Under RELAXED
  it is the device `powf`; under FAST, 2^(y log2 x) on the hardware base-2
  transcendentals for positive normal bases (powf otherwise).
  Method, in base 2: x = m * 2^e with m in [sqrt(1/2), sqrt(2));
  log2 m = (2/ln 2) atanh(t), t = (m-1) RN(1/(m+1)), as an odd series in t;
  2^z by z = k + r, |r| <= 1/2, and a degree-10 polynomial in r; both
  carried in double, so the float result is the double value rounded once
  (correctly rounded on every sampled argument).
- `ph_rrcp`/`ph_rdiv`/`ph_rpow` (REPRODUCIBLE, `PH_MATH_MODE == 3`): the
  reciprocal correctly rounded from the hardware estimate by one Newton
  step (IEEE division, in a branch, for the divisors whose reciprocal is
  not a normal number), `a / b` as `a * RN(1/b)`, and a fast deterministic power:
  for a positive normal base and |y| < 8192, log2 x from the float's bits
  (x = m 2^e, m in [sqrt(1/2), sqrt(2)), t = (m-1)/(m+1) by a quadratic
  start and two Newton steps, a degree-4 polynomial in t^2) and 2^z
  (z = k + r, a degree-7 polynomial in r), in double; any other operand takes the SAFE `ph_pow` in a branch that a
  wavefront enters only when one of its lanes needs it. `ph_dlog2f` and
  `ph_dexp2f`, what the power-law rewrite's log2 and exp2 become in this
  mode, are the same double log2 and 2^z rounded once to float.
- `ph_exp2`/`ph_log2`: under FAST the hardware base-2 exponential and
  logarithm; libm otherwise.
- `ph_sin`/`ph_cos`: under FAST the hardware sine/cosine (the reference's
  FAST contract allows approximate transcendentals); libm-accurate under
  SAFE and RELAXED. Under REPRODUCIBLE, `ph_exp`, `ph_log`, `ph_sin`,
  `ph_cos`, `ph_tanh`, `ph_exp2` and `ph_log2` are deterministic double-core
  forms (`ph_dexpf`, `ph_dlogf`, `ph_dtrig`, `ph_dtanhf`, `ph_dexp2f`,
  `ph_dlog2f`) that
  `palladium_amd.exact` and `oracle/oracle.c` restate bit for bit.
- `ph_fmin`/`ph_fmax`: NaN-suppressing min/max (C fminf/fmaxf), the
  reference's lowering of `min`/`max` (`src/palladium/emit/core.py:574-575`).
"""

PRELUDE = r"""
#ifndef PH_MATH_MODE
#define PH_MATH_MODE 2
#endif

__device__ __forceinline__ unsigned int ph_rotl32(unsigned int x, unsigned int r) {
    return (x << r) | (x >> (32u - r));
}

__device__ __forceinline__ void ph_threefry2x32(unsigned int k0, unsigned int k1,
                                                unsigned int c0, unsigned int c1,
                                                unsigned int* o0, unsigned int* o1) {
    const unsigned int k2 = k0 ^ k1 ^ 0x1BD11BDAu;
    unsigned int x0 = c0 + k0;
    unsigned int x1 = c1 + k1;
#define PH_TF_ROUND(r) x0 += x1; x1 = ph_rotl32(x1, r); x1 ^= x0;
    PH_TF_ROUND(13)
    /* Optimisation barrier (an empty asm that emits no instruction): without
       it LLVM re-associates each key injection into the following rounds'
       adds and keeps injected and un-injected copies of the state live,
       about 30% more VALU work per block (fold_in chains twice that). After
       the first round rather than before it, so a counter word that is
       uniform (a scalar) needs no copy into a vector register first. */
    asm volatile("" : "+v"(x0), "+v"(x1));
    PH_TF_ROUND(15) PH_TF_ROUND(26) PH_TF_ROUND(6)
    x0 += k1; x1 += k2 + 1u;
    PH_TF_ROUND(17) PH_TF_ROUND(29) PH_TF_ROUND(16) PH_TF_ROUND(24)
    x0 += k2; x1 += k0 + 2u;
    PH_TF_ROUND(13) PH_TF_ROUND(15) PH_TF_ROUND(26) PH_TF_ROUND(6)
    x0 += k0; x1 += k1 + 3u;
    PH_TF_ROUND(17) PH_TF_ROUND(29) PH_TF_ROUND(16) PH_TF_ROUND(24)
    x0 += k1; x1 += k2 + 4u;
    PH_TF_ROUND(13) PH_TF_ROUND(15) PH_TF_ROUND(26) PH_TF_ROUND(6)
    x0 += k2; x1 += k0 + 5u;
#undef PH_TF_ROUND
    *o0 = x0;
    *o1 = x1;
}

#if PH_MATH_MODE == 2
/* FAST: hardware sine/cosine (v_sin_f32/v_cos_f32 take revolutions, so
   cos(2*pi*u) needs no range reduction after reassociation). */
__device__ __forceinline__ float ph_sin(float x) { return __builtin_amdgcn_sinf(x * 0.15915494309189535f); }
__device__ __forceinline__ float ph_cos(float x) { return __builtin_amdgcn_cosf(x * 0.15915494309189535f); }
__device__ __forceinline__ float ph_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }
/* v_exp_f32 / v_log_f32: 2^x and log2(x), 1 ulp, subnormals flushed. */
__device__ __forceinline__ float ph_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float ph_log2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float ph_log(float x) { return logf(x); }
__device__ __forceinline__ float ph_tanh(float x) { return tanhf(x); }
#elif PH_MATH_MODE != 3
__device__ __forceinline__ float ph_exp2(float x) { return exp2f(x); }
__device__ __forceinline__ float ph_log2(float x) { return log2f(x); }
__device__ __forceinline__ float ph_sin(float x) { return sinf(x); }
__device__ __forceinline__ float ph_cos(float x) { return cosf(x); }
__device__ __forceinline__ float ph_exp(float x) { return expf(x); }
__device__ __forceinline__ float ph_log(float x) { return logf(x); }
__device__ __forceinline__ float ph_tanh(float x) { return tanhf(x); }
#endif

/* Integer division and float->integer conversion with every input defined,
   as XLA's elemental emitter defines them: x / 0 = -1 (all ones unsigned),
   x % 0 = x, INT_MIN / -1 = INT_MIN, INT_MIN % -1 = 0; conversions
   saturate and send NaN to 0. (C leaves all of these undefined.) */
__device__ __forceinline__ int ph_idiv(int a, int b) {
    return b == 0 ? -1 : (b == -1 ? (int)(0u - (unsigned int)a) : a / b);
}
__device__ __forceinline__ int ph_irem(int a, int b) { return (b == 0) ? a : (b == -1 ? 0 : a % b); }
__device__ __forceinline__ unsigned int ph_udiv(unsigned int a, unsigned int b) { return b == 0u ? 0xFFFFFFFFu : a / b; }
__device__ __forceinline__ unsigned int ph_urem(unsigned int a, unsigned int b) { return b == 0u ? a : a % b; }
__device__ __forceinline__ int ph_f2i(float x) {
    return x != x ? 0 : (x >= 2147483648.0f ? 2147483647 : (x <= -2147483648.0f ? (-2147483647 - 1) : (int)x));
}
__device__ __forceinline__ unsigned int ph_f2u(float x) {
    return x != x ? 0u : (x >= 4294967296.0f ? 0xFFFFFFFFu : (x <= 0.0f ? 0u : (unsigned int)x));
}
__device__ __forceinline__ int ph_iabs(int a) { return a < 0 ? (int)(0u - (unsigned int)a) : a; }

/* expm1 with C99's expm1(-0) = -0 (the device library returns +0). */
__device__ __forceinline__ float ph_expm1(float x) { return x == 0.0f ? x : expm1f(x); }

__device__ __forceinline__ float ph_fmin(float a, float b) { return fminf(a, b); }
__device__ __forceinline__ float ph_fmax(float a, float b) { return fmaxf(a, b); }

#if PH_MATH_MODE == 0 || PH_MATH_MODE == 3
/* The wavefront mask of lanes whose x is in one of the classes `mask`
   selects (v_cmp_class bits: 0 sNaN, 1 qNaN, 2 -inf, 3 -normal, 4 -subnormal,
   5 -0, 6 +0, 7 +subnormal, 8 +normal, 9 +inf), as a scalar: written straight
   into a scalar register pair, so testing it costs one vector compare and
   a scalar branch (through a bool and a ballot the compiler spends a
   select and a second compare). Inactive lanes read 0. */
__device__ __forceinline__ unsigned long long ph_class_mask(float x, unsigned int mask) {
    unsigned long long m;
    __asm__ volatile("v_cmp_class_f32_e64 %0, %1, %2" : "=s"(m) : "v"(x), "s"(mask));
    return m;
}

/* a * b + c, correctly rounded (one v_fma_f64), with the constant c read
   from scalar registers. Written out because the compiler otherwise keeps
   polynomial coefficients in vector registers and copies each into the
   accumulator of a v_fmac_f64 first: two instructions per term. */
__device__ __forceinline__ double ph_fma_k(double a, double b, double c) {
    double r;
    asm("v_fma_f64 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(c));
    return r;
}

/* log2 of a positive finite double: x = m 2^e with m in [sqrt(1/2), sqrt(2)),
   log2 m = (2 / ln 2) atanh(t), t = (m - 1) RN(1 / (m + 1)), as an odd series in t
   whose coefficients carry the 2 / ln 2; log2 x = e + t P(t^2), one FMA. */
__device__ __forceinline__ double ph_log2_core(double m, int e);

__device__ __forceinline__ double ph_log2_pos(double x) {
    int e;
    double m = frexp(x, &e);          /* x = m 2^e, m in [0.5, 1) */
    if (m < 0.70710678118654752440) { m = m * 2.0; e = e - 1; }
    return ph_log2_core(m, e);
}

/* log2(m 2^e) for m in [sqrt(1/2), sqrt(2)) with at most 24 significant bits. */
__device__ __forceinline__ double ph_log2_core(double m, int e) {
    /* t = (m - 1) RN(1 / (m + 1)), the reciprocal without a division. m is a
       float, so d = m + 1 in [1.707, 2.414) has at most 25 significant bits.
       From the hardware float reciprocal (relative error below 2^-22) two
       Newton steps r + r (1 - d r), each two correctly rounded FMAs, leave
       r within 2^-88 of 1 / d; 1 / d is never within 2^-79 of a midpoint
       between doubles (1 - d * midpoint is a nonzero integer over 2^79 at
       most), so r is RN(1 / d) exactly, the value the host oracle gets from
       1.0 / d. */
    double d = m + 1.0;
    double r = (double)__builtin_amdgcn_rcpf((float)d);
    double q = fma(-d, r, 1.0);
    r = fma(r, q, r);
    q = fma(-d, r, 1.0);
    r = fma(r, q, r);
    double t = (m - 1.0) * r;
    double t2 = t * t;
    /* sum_{k=0..7} 2 t2^k / ((2k+1) ln 2) by Horner's rule (one constant per
       FMA, so no constant needs a register move first). |t| <= 0.1716, so the
       first omitted term is below 1.3e-13 of the sum. */
    double p = ph_fma_k(t2, 0.19235933878519512, 0.22195308321368667);
    p = ph_fma_k(p, t2, 0.2623081892525388);
    p = ph_fma_k(p, t2, 0.3205988979753252);
    p = ph_fma_k(p, t2, 0.4121985831111324);
    p = ph_fma_k(p, t2, 0.5770780163555853);
    p = ph_fma_k(p, t2, 0.9617966939259756);
    p = ph_fma_k(p, t2, 2.8853900817779268);
    return fma(t, p, (double)e);
}

/* 2^z for |z| <= 151: z = k + r, |r| <= 1/2, 2^r = sum (r ln 2)^n / n!
   with the ln 2 powers folded into the coefficients. */
__device__ __forceinline__ double ph_exp2_dbl(double z) {
    double kd = rint(z);
    double r = z - kd;                /* exact */
    /* sum_{n=0..10} (ln 2)^n r^n / n! by Horner's rule. |r ln 2| <= 0.347,
       so the first omitted term is below 2.2e-13. */
    double p = ph_fma_k(r, 7.054911620801123e-09, 1.01780860092397e-07);
    p = ph_fma_k(p, r, 1.321548679014431e-06);
    p = ph_fma_k(p, r, 1.5252733804059841e-05);
    p = ph_fma_k(p, r, 0.0001540353039338161);
    p = ph_fma_k(p, r, 0.0013333558146428443);
    p = ph_fma_k(p, r, 0.009618129107628477);
    p = ph_fma_k(p, r, 0.05550410866482158);
    p = ph_fma_k(p, r, 0.24022650695910072);
    p = ph_fma_k(p, r, 0.6931471805599453);
    p = ph_fma_k(p, r, 1.0);
    return ldexp(p, (int)kd);
}

/* The part of ph_pow that depends on the base alone: log2 |x| for a
   finite nonzero base (log2 1 = 0 otherwise, which the special cases then
   override). ph_pow(x, y) == ph_pow_with_log(x, y, ph_pow_log(x)) bit for
   bit, so a loop can compute the log of a base once and use it in several
   powers, or carry it with the base. */
__device__ __noinline__ double ph_pow_log_slow(float x) {
    float ax = fabsf(x);
    bool finite_base = ax > 0.0f && ax < __builtin_inff();
    return ph_log2_pos((double)(finite_base ? ax : 1.0f));
}

/* For a normal base the split comes from the float's bits: |x| = m 2^e with
   m in [0x1.6a09e8p-1, 2 * 0x1.6a09e6p-1], the float range frexp's
   m < sqrt(1/2) doubling gives, so m and e, and the log, are the same bits.
   A wavefront holding a zero, subnormal, infinite or NaN base takes the
   frexp form for those lanes in a branch. */
__device__ __forceinline__ double ph_pow_log(float x) {
    unsigned int ix = (__float_as_uint(x) & 0x7fffffffu) - 0x3f3504f4u;
    int e = (int)ix >> 23;
    float m = __uint_as_float((ix & 0x007fffffu) + 0x3f3504f4u);
    double lg = ph_log2_core((double)m, e);
    if (__builtin_expect(ph_class_mask(x, 0x2f7) != 0ull, 0))   /* a lane not -normal, not +normal */
        lg = __builtin_amdgcn_classf(x, 0x2f7) ? ph_pow_log_slow(x) : lg;
    return lg;
}

/* Every operand: the main path on a harmless base for special operands
   and the C99 special cases selected over it, highest priority last. Same
   results as oracle/oracle.c:oracle_pow, which tests them in order. */
__device__ __noinline__ float ph_pow_full(float x, float y, double lg) {
    const float inf = __builtin_inff();
    float ax = fabsf(x);
    float ay = fabsf(y);
    bool small = ay < 16777216.0f;
    bool y_int = small ? (truncf(y) == y) : true;
    /* fmodf(ay, 2) == 1 for an integral ay below 2^24, exactly */
    bool y_odd = y_int && small && (ay - 2.0f * truncf(0.5f * ay) == 1.0f);
    float sign = (__builtin_signbit(x) && y_odd) ? -1.0f : 1.0f; /* -0 too: pow(-0, 3) = -0 */
    double z = (double)y * lg;
    double zc = fmin(fmax(z, -151.0), 129.0);
    float r = sign * (float)ph_exp2_dbl(zc);
    r = (z > 129.0) ? sign * inf : r;
    r = (z < -151.0) ? sign * 0.0f : r;
    r = (ax == inf) ? ((y < 0.0f) ? sign * 0.0f : sign * inf) : r;
    r = (ax == 0.0f) ? ((y < 0.0f) ? sign * inf : sign * 0.0f) : r;
    r = (ay == inf) ? ((ax == 1.0f) ? 1.0f : (((ax > 1.0f) == (y > 0.0f)) ? inf : 0.0f)) : r;
    r = (x < 0.0f && !y_int && ax != inf) ? __builtin_nanf("") : r;
    r = (x != x || y != y) ? x + y : r;
    r = (y == 0.0f || x == 1.0f) ? 1.0f : r;
    return r;
}

/* The wavefront mask of lanes whose double z lies outside [lo, hi] (or is
   NaN), as a scalar, like ph_class_mask. */
__device__ __forceinline__ unsigned long long ph_outside_mask(double z, double lo, double hi) {
    unsigned long long a, b;
    __asm__ volatile("v_cmp_nge_f64_e64 %0, %1, %2" : "=s"(a) : "v"(z), "s"(lo));
    __asm__ volatile("v_cmp_nle_f64_e64 %0, %1, %2" : "=s"(b) : "v"(z), "s"(hi));
    return a | b;
}

/* x^y given lg = ph_pow_log(x). For a positive finite base and
   -151 <= z = y lg <= 129 every special case of ph_pow_full leaves its
   main path's value, 2^z rounded once to float (x = 1 gives z = 0 and 1;
   y = 0 gives z = 0 and 1; a NaN or infinite y makes z NaN or infinite),
   so that value is computed directly, and a wavefront holding any other
   lane (a zero, negative, infinite or NaN base, or z out of that range)
   takes ph_pow_full for those lanes in a branch. Bit for bit ph_pow_full. */
__device__ __forceinline__ float ph_pow_with_log(float x, float y, double lg) {
    double z = (double)y * lg;
    float r = (float)ph_exp2_dbl(z);
    unsigned long long any = ph_class_mask(x, 0x27f) | ph_outside_mask(z, -151.0, 129.0);
    if (__builtin_expect(any != 0ull, 0))
        r = (!(x > 0.0f && x < __builtin_inff()) || !(z >= -151.0 && z <= 129.0)) ? ph_pow_full(x, y, lg) : r;
    return r;
}

__device__ __forceinline__ float ph_pow(float x, float y) { return ph_pow_with_log(x, y, ph_pow_log(x)); }
#endif
#if PH_MATH_MODE == 3
/* RN(1/b) for every float b. The hardware estimate (within 1 ulp) and one
   Newton step y + y (1 - b y), the residual exact in the inner FMA, give
   the correctly rounded reciprocal whenever the result is a normal
   number. Any other result (b zero, subnormal, infinite or NaN, or
   |b| >= 2^126, where 1/b is subnormal) is redone by IEEE division, in a
   branch a wavefront takes only when one of its lanes needs it (the empty
   asm keeps the wavefront mask an opaque scalar: one compare and one
   scalar branch on the common path). Checked against the IEEE quotient on
   every float on the device. */
__device__ __noinline__ float ph_rrcp_slow(float b) { return 1.0f / b; }

__device__ __forceinline__ float ph_rrcp(float b) {
    float y = __builtin_amdgcn_rcpf(b);
    float e = __builtin_fmaf(-b, y, 1.0f);
    y = __builtin_fmaf(e, y, y);
    if (__builtin_expect(ph_class_mask(y, 0x2f7) != 0ull, 0))   /* a lane not -normal, not +normal */
        y = __builtin_amdgcn_classf(y, 0x2f7) ? ph_rrcp_slow(b) : y;
    return y;
}

__device__ __forceinline__ float ph_rdiv(float a, float b) { return a * ph_rrcp(b); }

/* log2 x for a positive normal float x; any other x gives a finite or NaN
   value that ph_rpow_with_log never uses. The exponent split works on the
   bits: x = m 2^e with m in [m0, 2 m0), m0 = 0x1.6a09e6p-1 (the float just
   above sqrt(1/2)); t = (m - 1) r with r ~ 1/(m + 1) from a quadratic start
   (relative error 2^-9.6) and two Newton steps (2^-38); log2 m = t P(t^2)
   with P of degree 4, log2 x = e + t P by one FMA. Every step is a
   correctly rounded double operation, so the host repeats it exactly.
   Coefficients: oracle/gen_rpow_coeffs.py. */
__device__ __forceinline__ double ph_rpow_log(float x) {
    unsigned int ix = __float_as_uint(x) - 0x3f3504f3u;
    int e = (int)ix >> 23;
    float m = __uint_as_float((ix & 0x007fffffu) + 0x3f3504f3u);
    double dm = (double)m;
    double d = dm + 1.0;
    double r = ph_fma_k(d, 0.116862893757792, -0.722444125812821);
    r = ph_fma_k(r, d, 1.4777559273698688);
    double q = fma(-d, r, 1.0);
    r = fma(r, q, r);
    q = fma(-d, r, 1.0);
    r = fma(r, q, r);
    double t = (dm - 1.0) * r;
    double s = t * t;
    double p = ph_fma_k(s, 0.3407120415619086, 0.41167376623771057);
    p = ph_fma_k(p, s, 0.5770835660048659);
    p = ph_fma_k(p, s, 0.9617966734515485);
    p = ph_fma_k(p, s, 2.885390081789987);
    return fma(t, p, (double)e);
}

/* 2^z for |z| < 2^21: z = k + r, |r| <= 1/2, Q(r) of degree 7 as two
   Horner halves (degrees 0-3 and 4-7, independent chains) joined by one
   FMA with r^4. */
__device__ __forceinline__ double ph_rexp2(double z) {
    double kd = __builtin_rint(z);
    double r = z - kd;
    double r2 = r * r;
    double lo = ph_fma_k(r, 0.055504109063258665, 0.24022651213498092);
    double hi = ph_fma_k(r, 1.5303700711365693e-05, 0.00015469729214118296);
    lo = ph_fma_k(lo, r, 0.6931471805568324);
    hi = ph_fma_k(hi, r, 0.0013333478473685416);
    double r4 = r2 * r2;
    lo = ph_fma_k(lo, r, 0.9999999999595618);
    hi = ph_fma_k(hi, r, 0.009618025613318034);
    return __builtin_ldexp(fma(hi, r4, lo), (int)kd);
}

__device__ __noinline__ float ph_rpow_slow(float x, float y) { return ph_pow(x, y); }

/* x^y given lg = ph_rpow_log(x). For a positive normal x and |y| < 8192,
   |z| = |y lg| < 2^20 and 2^z rounded once to float (ldexp in double keeps
   overflow to inf and underflow to subnormals and zero exact until then).
   Any other operand (zero, subnormal, negative, infinite or NaN x; large,
   infinite or NaN y) takes the SAFE pow with its C99 special cases, in a
   branch taken only by wavefronts holding such a lane. */
__device__ __forceinline__ float ph_rpow_with_log(float x, float y, double lg) {
    float r = (float)ph_rexp2((double)y * lg);
    bool wide_y = !(__builtin_fabsf(y) < 8192.0f);   /* folds away for a literal exponent */
    unsigned long long any = ph_class_mask(x, 0x2ff) | __builtin_amdgcn_ballot_w64(wide_y);
    if (__builtin_expect(any != 0ull, 0))
        r = (__builtin_amdgcn_classf(x, 0x2ff) || wide_y) ? ph_rpow_slow(x, y) : r;
    return r;
}

__device__ __forceinline__ float ph_rpow(float x, float y) { return ph_rpow_with_log(x, y, ph_rpow_log(x)); }

/* The wavefront mask of lanes where |x| < limit fails (|x| >= limit or x
   NaN), as a scalar, like ph_class_mask. */
__device__ __forceinline__ unsigned long long ph_wide_mask(float x, float limit) {
    unsigned long long m;
    __asm__ volatile("v_cmp_nlt_f32_e64 %0, |%1|, %2" : "=s"(m) : "v"(x), "s"(limit));
    return m;
}

/* Deterministic float log2 and exp2 (what the power-law rewrite's log2 and
   exp2 become under REPRODUCIBLE): the double log2 of ph_rpow_log and the
   double 2^z of ph_rexp2, each rounded once to float. Special operands
   take a branch a wavefront enters only when one of its lanes needs it:
   log2 of NaN is NaN, of a negative number NaN, of +-0 -inf, of +inf +inf,
   of a subnormal x log2(x 2^24) - 24; exp2 of NaN is NaN and of |x| >= 2^20
   +inf or +0. */
__device__ __noinline__ float ph_dlog2f_slow(float x) {
    if (x != x) return x;
    if (x < 0.0f) return __builtin_nanf("");
    if (x == 0.0f) return -__builtin_inff();
    if (x == __builtin_inff()) return x;
    return (float)(ph_rpow_log(x * 0x1p24f) - 24.0);
}

__device__ __forceinline__ float ph_dlog2f(float x) {
    float r = (float)ph_rpow_log(x);
    if (__builtin_expect(ph_class_mask(x, 0x2ff) != 0ull, 0))
        r = __builtin_amdgcn_classf(x, 0x2ff) ? ph_dlog2f_slow(x) : r;
    return r;
}

__device__ __noinline__ float ph_dexp2f_slow(float x) { return x != x ? x : (x > 0.0f ? __builtin_inff() : 0.0f); }

__device__ __forceinline__ float ph_dexp2f(float x) {
    float r = (float)ph_rexp2((double)x);
    if (__builtin_expect(ph_wide_mask(x, 0x1p20f) != 0ull, 0))
        r = !(__builtin_fabsf(x) < 0x1p20f) ? ph_dexp2f_slow(x) : r;
    return r;
}

/* Deterministic float exp and log on the same double cores: e^x as
   2^(x log2 e), the product rounded once to double (error below 2^-46
   absolute in the exponent for |x| < 2^19), and ln x as the double log2
   times ln 2. Special operands as ph_dexp2f (|x| >= 2^19 here) and
   ph_dlog2f. */
__device__ __forceinline__ float ph_dexpf(float x) {
    float r = (float)ph_rexp2((double)x * 1.4426950408889634);
    if (__builtin_expect(ph_wide_mask(x, 0x1p19f) != 0ull, 0))
        r = !(__builtin_fabsf(x) < 0x1p19f) ? ph_dexp2f_slow(x) : r;
    return r;
}

__device__ __noinline__ float ph_dlogf_slow(float x) {
    if (x != x) return x;
    if (x < 0.0f) return __builtin_nanf("");
    if (x == 0.0f) return -__builtin_inff();
    if (x == __builtin_inff()) return x;
    return (float)((ph_rpow_log(x * 0x1p24f) - 24.0) * 0.6931471805599453);
}

__device__ __forceinline__ float ph_dlogf(float x) {
    float r = (float)(ph_rpow_log(x) * 0.6931471805599453);
    if (__builtin_expect(ph_class_mask(x, 0x2ff) != 0ull, 0))
        r = __builtin_amdgcn_classf(x, 0x2ff) ? ph_dlogf_slow(x) : r;
    return r;
}

/* Deterministic float sine and cosine. x = k pi/2 + r with |r| <= pi/4
   (plus rounding); sin r = r S(r^2) and cos r = C(r^2), S and C of degree 5
   in double (relative errors 2^-47.6 and 2^-43.5), and the quadrant
   (k + off) mod 4 picks +-sin r or +-cos r (off = 0 for sine, 1 for cosine),
   rounded once to float. For |x| < 2^20, k = rint(x 2/pi) and
   r = (x - k PIO2_HI) - k PIO2_LO by two FMAs, the first exact (PIO2_HI has
   33 significant bits and k at most 20). Larger finite x take the exact
   reduction of the slow path: x 2/pi mod 4 from a 96-bit window of the
   bits of 2/pi (x = M 2^E, M 24 bits, the product kept to 2^-62 below the
   binary point), in a branch a wavefront enters only when one of its lanes
   needs it; infinities and NaN give NaN. Coefficients:
   oracle/gen_rpow_coeffs.py. */
__device__ __forceinline__ float ph_dtrig_poly(double r, int q) {
    double s = r * r;
    double ps = ph_fma_k(s, -2.47565580235085e-08, 2.7555271883000814e-06);
    double pc = ph_fma_k(s, -2.717342886965949e-07, 2.47989287418407e-05);
    ps = ph_fma_k(ps, s, -0.0001984126329834066);
    pc = ph_fma_k(pc, s, -0.0013888880393711728);
    ps = ph_fma_k(ps, s, 0.008333333323878053);
    pc = ph_fma_k(pc, s, 0.04166666654390994);
    ps = ph_fma_k(ps, s, -0.16666666666616684);
    pc = ph_fma_k(pc, s, -0.4999999999935111);
    ps = ph_fma_k(ps, s, 0.9999999999999957);
    pc = ph_fma_k(pc, s, 0.9999999999999444);
    double v = (q & 1) ? pc : r * ps;
    return (float)((q & 2) ? -v : v);
}

__device__ __constant__ const unsigned int ph_two_over_pi[7] = {
    0xA2F9836Eu, 0x4E441529u, 0xFC2757D1u, 0xF534DDC0u, 0xDB629599u, 0x3C439041u, 0xFE5163ABu};

__device__ __noinline__ float ph_dtrig_slow(float x, int off) {
    if (!(__builtin_fabsf(x) < __builtin_inff())) return __builtin_nanf("");
    unsigned int b = __float_as_uint(x);
    int e = (int)((b >> 23) & 0xffu) - 150;              /* x = M 2^e, e >= -3 here */
    unsigned long long m = (b & 0x7fffffu) | 0x800000u;
    int i0 = e >= 2 ? e - 1 : 1;                         /* first bit of 2/pi that matters mod 4 */
    int j = (i0 - 1) >> 5, sh = (i0 - 1) & 31;
    unsigned __int128 w = ((unsigned __int128)ph_two_over_pi[j] << 96) |
                          ((unsigned __int128)ph_two_over_pi[j + 1] << 64) |
                          ((unsigned __int128)ph_two_over_pi[j + 2] << 32) | ph_two_over_pi[j + 3];
    w = (w << sh) >> 32;                                 /* bits i0 .. i0+95 of 2/pi */
    int n = 97 - e + i0;                                 /* product bits below weight 4 */
    unsigned __int128 p = (m * w) & ((((unsigned __int128)1) << n) - 1);
    int q = (int)(p >> (n - 2)) & 3;
    long long f = (long long)((unsigned long long)(p >> (n - 64)) & ((1ull << 62) - 1));
    if (f >= (1ll << 61)) { f -= (1ll << 62); q += 1; }
    double r = (double)f * 0x1.921fb54442d18p-62;        /* pi/2 2^-62 */
    if (b >> 31) { r = -r; q = -q; }
    return ph_dtrig_poly(r, q + off);
}

__device__ __forceinline__ float ph_dtrig(float x, int off) {
    double xd = (double)x;
    double k = __builtin_rint(xd * 0.6366197723675814);
    double r = fma(-k, 0x1.921fb544p+0, xd);
    r = fma(-k, 0x1.0b4611a626331p-34, r);
    float v = ph_dtrig_poly(r, (int)k + off);
    if (__builtin_expect(ph_wide_mask(x, 0x1p20f) != 0ull, 0))
        v = !(__builtin_fabsf(x) < 0x1p20f) ? ph_dtrig_slow(x, off) : v;
    return v;
}

__device__ __forceinline__ float ph_exp(float x) { return ph_dexpf(x); }
__device__ __forceinline__ float ph_log(float x) { return ph_dlogf(x); }
__device__ __forceinline__ float ph_sin(float x) { return ph_dtrig(x, 0); }
__device__ __forceinline__ float ph_cos(float x) { return ph_dtrig(x, 1); }
__device__ __forceinline__ float ph_exp2(float x) { return ph_dexp2f(x); }
__device__ __forceinline__ float ph_log2(float x) { return ph_dlog2f(x); }

/* Deterministic float tanh: a = |x|; below 1/2, a T(a^2) with T of degree 7
   (relative error 2^-42.3); from 1/2 on, 1 - 2 / (e + 1) with e = e^(2a) on
   the 2^z core (a clamped at 10, where the float result is 1 already) and
   an IEEE double division; rounded once to float, the sign copied from x,
   NaN passed through. */
__device__ __forceinline__ float ph_dtanhf(float x) {
    double a = __builtin_fabs((double)x);
    double s = a * a;
    double p = ph_fma_k(s, -0.0009849941049264166, 0.003415370282047567);
    p = ph_fma_k(p, s, -0.008827257095239422);
    p = ph_fma_k(p, s, 0.021865363235290286);
    p = ph_fma_k(p, s, -0.053967994875471936);
    p = ph_fma_k(p, s, 0.13333332529982497);
    p = ph_fma_k(p, s, -0.33333333323808056);
    p = ph_fma_k(p, s, 0.9999999999998141);
    double e = ph_rexp2(__builtin_fmin(a, 10.0) * 2.8853900817779268);
    double t = a < 0.5 ? a * p : 1.0 - 2.0 / (e + 1.0);
    float r = __builtin_copysignf((float)t, x);
    return x != x ? x : r;
}

__device__ __forceinline__ float ph_tanh(float x) { return ph_dtanhf(x); }
#elif PH_MATH_MODE == 2
/* FAST: x^y = 2^(y log2 x) on the hardware base-2 logarithm and
   exponential (v_log_f32, v_exp_f32) for a positive normal finite base and
   a finite exponent; zero, negative, subnormal and non-finite operands take
   the full powf. */
__device__ __forceinline__ float ph_pow(float x, float y) {
    if (x >= 0x1p-126f && x < __builtin_inff() && __builtin_fabsf(y) < __builtin_inff())
        return __builtin_amdgcn_exp2f(y * __builtin_amdgcn_logf(x));
    return powf(x, y);
}
#elif PH_MATH_MODE == 1
__device__ __forceinline__ float ph_pow(float x, float y) { return powf(x, y); }
#endif
"""
