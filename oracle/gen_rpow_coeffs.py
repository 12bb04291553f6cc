"""Coefficients of the REPRODUCIBLE-mode power function (test
infrastructure: prints the constants that `palladium_amd/emit/prelude.py`
and `oracle/oracle.c` both hard-code; needs mpmath, which only this
generator uses).

    log2 m = t P(t^2),  t = (m - 1) r,  m in [m0, 2 m0),  m0 = 0x1.6a09e6p-1
    r ~ 1/(m + 1): R(m + 1) refined by two Newton steps
    2^r    = Q(r),                              r in [-1/2, 1/2]

    sin r  = r S(r^2), cos r = C(r^2),          |r| <= pi/4 (+1e-6)
    tanh a = a T(a^2),                          0 <= a < 1/2

P has degree 4, R degree 2, Q degree 7, S and C degree 5 and T degree 7, each the Chebyshev interpolant
of its function on its interval (near-minimax), with coefficients rounded
to double. R's relative error is 2^-9.6, so the two Newton steps leave
2^-38. TWO_OVER_PI holds the first 224 fraction bits of 2/pi in 32-bit
words, most significant first (the table of the large-argument sine and
cosine reduction), and PIO2_HI + PIO2_LO splits pi/2 with PIO2_HI carrying
33 significant bits, so k PIO2_HI is exact for |k| < 2^20. Run `python oracle/gen_rpow_coeffs.py` to reprint them with the
measured worst-case errors.
"""

import mpmath as mp

mp.mp.dps = 60
S_MAX = ((mp.sqrt(2) - 1) / (mp.sqrt(2) + 1)) ** 2


def _p_target(s):
    if s == 0:
        return 2 / mp.log(2)
    t = mp.sqrt(s)
    return mp.log((1 + t) / (1 - t), 2) / t


M0 = mp.mpf(float.fromhex("0x1.6a09e6p-1"))


R_TRIG = mp.pi / 4 + mp.mpf("1e-6")


def _s_target(s):
    if s == 0:
        return mp.mpf(1)
    r = mp.sqrt(s)
    return mp.sin(r) / r


def _c_target(s):
    return mp.cos(mp.sqrt(s))


def trig_coefficients():
    """(S, C), low-to-high, as Python floats."""
    sc = mp.chebyfit(_s_target, [0, R_TRIG ** 2], 6)
    cc = mp.chebyfit(_c_target, [0, R_TRIG ** 2], 6)
    return [float(c) for c in reversed(sc)], [float(c) for c in reversed(cc)]


TANH_SPLIT = mp.mpf("0.5")


def _t_target(s):
    if s == 0:
        return mp.mpf(1)
    a = mp.sqrt(s)
    return mp.tanh(a) / a


def tanh_coefficients():
    tc = mp.chebyfit(_t_target, [0, TANH_SPLIT ** 2], 8)
    return [float(c) for c in reversed(tc)]


def tanh_error(samples: int = 4001) -> float:
    T = tanh_coefficients()
    aa = [TANH_SPLIT * mp.mpf(k) / (samples - 1) for k in range(1, samples)]
    return float(max(abs(_poly(T, a * a) * a / mp.tanh(a) - 1) for a in aa))


def two_over_pi_words(n: int = 7):
    with mp.workdps(20 + 10 * n):
        bits = int(mp.floor((2 / mp.pi) * mp.mpf(2) ** (32 * n)))
    return [(bits >> (32 * (n - 1 - i))) & 0xFFFFFFFF for i in range(n)]


def pio2_split():
    hi = mp.floor(mp.pi / 2 * mp.mpf(2) ** 32) / mp.mpf(2) ** 32
    return float(hi), float(mp.pi / 2 - hi)


def trig_errors(samples: int = 4001):
    """Worst relative errors of r S(r^2) against sin r and C(r^2) against cos r."""
    S, C = trig_coefficients()
    rs = [R_TRIG * mp.mpf(k) / (samples - 1) for k in range(1, samples)]
    es = max(abs(_poly(S, r * r) * r / mp.sin(r) - 1) for r in rs)
    ec = max(abs(_poly(C, r * r) / mp.cos(r) - 1) for r in rs)
    return float(es), float(ec)


def coefficients():
    """(P, Q, R), each low-to-high, as Python floats."""
    p, _ = mp.chebyfit(_p_target, [0, S_MAX], 5, error=True)
    q, _ = mp.chebyfit(lambda r: mp.power(2, r), [-0.5, 0.5], 8, error=True)
    r, _ = mp.chebyfit(lambda d: 1 / d, [1 + M0, 1 + 2 * M0], 3, error=True)
    return ([float(c) for c in reversed(p)], [float(c) for c in reversed(q)],
            [float(c) for c in reversed(r)])


def _poly(cs, x):
    acc = mp.mpf(0)
    for c in reversed(cs):
        acc = acc * x + mp.mpf(c)
    return acc


def max_errors(samples: int = 4001):
    """Worst absolute error of t P(t^2) against log2 m over t, and worst
    relative error of Q against 2^r, both with the double coefficients in
    exact arithmetic."""
    P, Q, _ = coefficients()
    tmax = mp.sqrt(S_MAX)
    e_log = max(abs(t * _poly(P, t * t) - mp.log((1 + t) / (1 - t), 2))
                for t in (tmax * (2 * mp.mpf(k) / (samples - 1) - 1) for k in range(samples)))
    e_exp = max(abs(_poly(Q, r) / mp.power(2, r) - 1)
                for r in (mp.mpf(k) / (samples - 1) - mp.mpf(0.5) for k in range(samples)))
    return float(e_log), float(e_exp)


def reciprocal_start_error(samples: int = 4001) -> float:
    _, _, R = coefficients()
    return float(max(abs(_poly(R, d) * d - 1)
                     for d in (1 + M0 + M0 * mp.mpf(k) / (samples - 1) for k in range(samples))))


if __name__ == "__main__":
    P, Q, R = coefficients()
    print("P (t^2, low to high):", ", ".join(repr(c) for c in P))
    print("Q (r, low to high):  ", ", ".join(repr(c) for c in Q))
    print("R (d, low to high):  ", ", ".join(repr(c) for c in R))
    er = reciprocal_start_error()
    print(f"max |R(d) d - 1| = {er:.3g} (2^{float(mp.log(er, 2)):.1f})")
    el, ee = max_errors()
    print(f"max |t P(t^2) - log2 m| = {el:.3g} (2^{float(mp.log(el, 2)):.1f}); "
          f"max |Q(r)/2^r - 1| = {ee:.3g} (2^{float(mp.log(ee, 2)):.1f})")
    S, C = trig_coefficients()
    print("S (r^2, low to high):", ", ".join(repr(c) for c in S))
    print("C (r^2, low to high):", ", ".join(repr(c) for c in C))
    es, ec = trig_errors()
    print(f"max |r S(r^2)/sin r - 1| = 2^{float(mp.log(es, 2)):.1f}; max |C(r^2)/cos r - 1| = 2^{float(mp.log(ec, 2)):.1f}")
    T = tanh_coefficients()
    print("T (a^2, low to high):", ", ".join(repr(c) for c in T))
    print(f"max |a T(a^2)/tanh a - 1| = 2^{float(mp.log(tanh_error(), 2)):.1f}")
    print("TWO_OVER_PI:", ", ".join(f"0x{w:08X}" for w in two_over_pi_words()))
    hi, lo = pio2_split()
    print(f"PIO2_HI = {hi.hex()} ({hi!r}); PIO2_LO = {lo.hex()} ({lo!r})")
