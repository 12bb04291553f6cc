"""Write the small golden fixtures under tests/golden/ from the C oracle.

Run from the repo root after `make -C oracle`: `python tests/golden/make_fixtures.py`.
The oracle is pinned independently (Random123 known answers, float64
restatements, invariants; see tests/test_oracle.py); these files freeze its
outputs at small sizes so that the GPU tests, and any later change to the
oracle, are checked against fixed numbers rather than against a program
that could drift with them.

Inputs follow the benchmark configurations' generators
(`palladium_amd.workloads`): LV draws (alpha, beta, gamma, delta, x0, y0)
from `numpy.random.default_rng(seed)`; BS3 draws (mu, x0, v0); Gray-Scott
uses its seeded initial condition; GBM uses key data (0, 42).
"""

from __future__ import annotations

import dataclasses
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from oracle.ref64 import lv_rk4_f64  # noqa: E402
from palladium_amd.workloads import (  # noqa: E402
    BS3_CFG,
    GBM_CFG,
    GS_CFG,
    LV_CFG0,
    bs3_inputs,
    gray_scott_initial,
    lv_inputs,
)

OUT = Path(__file__).resolve().parent

# Random123 known-answer vectors for Threefry-2x32 with 20 rounds
# (kat_vectors of the Random123 distribution; Salmon et al., SC'11).
THREEFRY_KATS = [
    {"key": [0x00000000, 0x00000000], "ctr": [0x00000000, 0x00000000], "out": [0x6B200159, 0x99BA4EFE]},
    {"key": [0xFFFFFFFF, 0xFFFFFFFF], "ctr": [0xFFFFFFFF, 0xFFFFFFFF], "out": [0x1CB996FC, 0xBB002BE7]},
    {"key": [0x13198A2E, 0x03707344], "ctr": [0x243F6A88, 0x85A308D3], "out": [0xC4923A9C, 0x483DF7A0]},
]

LV_N = 64
BS3_N = 64
GS_SIZE = 64
GS_STEPS = 10
GBM_PATHS = 64
GBM_STEPS = 8
DF32_N = 256


def threefry() -> None:
    for kat in THREEFRY_KATS:
        got = oracle.threefry2x32(*kat["key"], *kat["ctr"])
        assert list(got) == kat["out"], (kat, got)
    key = (0, GBM_CFG.seed)
    bits = oracle.random_bits(key, 16)
    folded = oracle.fold_in(key, 7)
    doc = {
        "algorithm": "Threefry-2x32, 20 rounds",
        "kats": [{k: [f"0x{x:08x}" for x in v] for k, v in kat.items()} for kat in THREEFRY_KATS],
        "random_bits": {"key": list(key), "n": 16, "bits": [f"0x{int(b):08x}" for b in bits]},
        "fold_in": {"key": list(key), "data": 7, "out": [f"0x{int(b):08x}" for b in folded]},
        "bits_to_uniform": [
            {"bits": f"0x{b:08x}", "u": float(oracle.bits_to_uniform(b))}
            for b in (0, 1, 0x1FF, 0x200, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF, int(bits[0]))
        ],
    }
    (OUT / "threefry_kat.json").write_text(json.dumps(doc, indent=1) + "\n")


def lv() -> None:
    args = lv_inputs(LV_N, LV_CFG0.seed)
    x, y, ymax = oracle.lv_rk4(*args, LV_CFG0.dt, LV_CFG0.steps, track_max=True)
    x64, y64 = lv_rk4_f64(*args, LV_CFG0.dt, LV_CFG0.steps)
    xh, xl, yh, yl = oracle.lv_rk4_df32(*args, LV_CFG0.dt, LV_CFG0.steps)
    np.savez(OUT / "lv_rk4_small.npz", inputs=np.stack(args), dt=np.float64(LV_CFG0.dt),
             steps=np.int32(LV_CFG0.steps), x=x, y=y, ymax=ymax, x64=x64, y64=y64,
             df32=np.stack([xh, xl, yh, yl]))


def bs3() -> None:
    x0, v0, mu = bs3_inputs(BS3_N, BS3_CFG.seed)
    t, x, v, acc, rej = oracle.bs3_vdp(x0, v0, mu, BS3_CFG)
    np.savez(OUT / "bs3_small.npz", x0=x0, v0=v0, mu=mu, t=t, x=x, v=v, accepted=acc, rejected=rej)


def gray_scott() -> None:
    u0, v0 = gray_scott_initial(GS_SIZE)
    u, v = oracle.gray_scott(u0, v0, GS_CFG, GS_STEPS)
    np.savez(OUT / "gray_scott_64.npz", u0=u0, v0=v0, steps=np.int32(GS_STEPS), u=u, v=v)


def gbm() -> None:
    cfg = dataclasses.replace(GBM_CFG, n_steps=GBM_STEPS)
    payoff = oracle.gbm(cfg, GBM_PATHS)
    np.savez(OUT / "gbm_small.npz", n_steps=np.int32(GBM_STEPS), payoff=payoff)


def df32() -> None:
    rng = np.random.default_rng(11)
    a = (rng.standard_normal(DF32_N) * 10.0 ** rng.integers(-6, 6, DF32_N)).astype(np.float32)
    b = (rng.standard_normal(DF32_N) * 10.0 ** rng.integers(-6, 6, DF32_N)).astype(np.float32)
    b[:16] = -a[:16]  # exact cancellation
    b[16:32] = a[16:32] * np.float32(1 + 2**-20)  # near cancellation
    zero = np.zeros(DF32_N, np.float32)
    sh, sl = oracle.df32_add(a, zero, b, zero)
    ph, pl_ = oracle.df32_mul(a, zero, b, zero)
    cases = []
    for i in range(DF32_N):
        cases.append({
            "a": float(a[i]), "b": float(b[i]),
            "sum_exact": float(np.float64(a[i]) + np.float64(b[i])),
            "sum": [float(sh[i]), float(sl[i])],
            "prod_exact": float(np.float64(a[i]) * np.float64(b[i])),
            "prod": [float(ph[i]), float(pl_[i])],
        })
    (OUT / "df32_ops.json").write_text(json.dumps({"n": DF32_N, "cases": cases}) + "\n")


def main() -> None:
    oracle.build()
    threefry()
    lv()
    bs3()
    gray_scott()
    gbm()
    df32()


if __name__ == "__main__":
    main()
