"""Coefficients of the REPRODUCIBLE-mode power function (test
infrastructure: prints the constants that `palladium_amd/emit/prelude.py`
and `oracle/oracle.c` both hard-code; needs mpmath, which only this
generator uses).

    log2 m = t P(t^2),  t = (m - 1) r,  m in [m0, 2 m0),  m0 = 0x1.6a09e6p-1
    r ~ 1/(m + 1): R(m + 1) refined by two Newton steps
    2^r    = Q(r),                              r in [-1/2, 1/2]

P has degree 4, R degree 2 and Q degree 7, each the Chebyshev interpolant
of its function on its interval (near-minimax), with coefficients rounded
to double. R's relative error is 2^-9.6, so the two Newton steps leave
2^-38. Run `python oracle/gen_rpow_coeffs.py` to reprint them with the
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
