"""bench.py's accounting helpers (CPU): the replayed lane fraction of the
compacting while loop, the op counts per loop iteration, and the --gpus
guard."""

import subprocess
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from palladium_amd.emit.compact import EPOCH, WORKGROUP  # noqa: E402


def test_compacted_lane_fraction_uniform_work_is_one():
    a = np.full(2 * WORKGROUP, 3 * EPOCH, np.int64)
    assert bench._compacted_lane_fraction(a) == 1.0


def test_compacted_lane_fraction_one_long_lane():
    a = np.full(WORKGROUP, EPOCH, np.int64)
    a[5] = 10 * EPOCH
    # epoch 1: 16 wavefronts; epochs 2-10: one wavefront holding the lone lane
    issued = (16 + 9) * EPOCH * 64
    assert bench._compacted_lane_fraction(a) == a.sum() / issued


def test_compacted_lane_fraction_beats_per_wavefront_maximum():
    rng = np.random.default_rng(0)
    a = rng.integers(1, 3000, 4 * WORKGROUP)
    waves = a.reshape(-1, 64)
    plain = waves.sum() / (waves.max(axis=1).sum() * 64)
    assert bench._compacted_lane_fraction(a) > plain


def test_loop_ops_per_iteration_counts_threefry_blocks():
    from palladium_amd.frontend import random
    from palladium_amd.trace import trace
    from palladium_amd.workloads import GBM_CFG, gbm_call

    spec = trace(gbm_call(GBM_CFG)._staged, random.key(42))
    n = bench.loop_ops_per_iteration(spec, "scan")
    assert n >= bench.THREEFRY_OPS + 10


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       cwd=ROOT, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_fraction_fields_are_found_at_any_depth_and_flagged_over_one():
    res = {"roofline": {"frac": 0.7, "issue": {"frac_of_peak_issue": 1.08, "ratio_to_fma_probe": 1.2}},
           "secondary": {"bs3": {"roofline": {"latency_frac": 0.85, "latency_bound": {"chain_model_ratio": 1.02}}}},
           "list": [{"frac": 1.5}]}
    found = dict(bench.fraction_fields(res))
    assert found == {"roofline.frac": 0.7, "roofline.issue.frac_of_peak_issue": 1.08,
                     "secondary.bs3.roofline.latency_frac": 0.85, "list[0].frac": 1.5}
    over = bench.fractions_over_one(res)
    assert over == ["roofline.issue.frac_of_peak_issue=1.0800", "list[0].frac=1.5000"]


def test_issue_fraction_is_against_the_peak_issue_rate(monkeypatch):
    """A kernel whose instruction mix runs above the pure-FMA probe's
    sustained rate (the probe is clock-limited under a full FMA load) has a
    ratio above 1 to the probe, but its fraction of the published peak issue
    rate stays below 1."""
    from palladium_amd import isa

    monkeypatch.setattr(bench, "valu_costs", lambda: {"sustained_fma_tflops": 121.7, "relative_cost_vs_fma": {}})
    monkeypatch.setattr(isa, "issue_slots", lambda code, costs: (100.0, {"v_add_f32_e32": 100}))
    # 100 slots x 6.6e11 units / 1 s = 6.6e13 slots/s: above the probe's 6.085e13
    r = bench.issue_fraction(b"", 6.6e11, 1000.0)
    assert r["ratio_to_fma_probe"] > 1.0
    assert 0.8 < r["frac_of_peak_issue"] < 1.0
    assert bench.fractions_over_one({"issue": r}) == []


def test_latency_bounds_name_the_issue_floor_a_fraction_and_the_chain_model_a_ratio(monkeypatch):
    from palladium_amd import isa
    from palladium_amd import runtime as rt

    class _Call:
        def bound(self, *a):
            class B:
                hip_source = "// no compaction"

                class spec:
                    name = "k"
            return B()

    monkeypatch.setattr(rt, "compile_code_object", lambda *a, **k: b"")
    monkeypatch.setattr(isa, "loop_model", lambda *a, **k: isa.LoopModel(100, 90, 2, 10, 400.0))
    lat = {"fma_dependent_ns": 4.3, "transcendental_dependent_ns": 5.8, "issue_ns": 2.9, "min_issue_cycles": 5.4}
    lb = bench.bs3_latency_bound(_Call(), (), lat, 1000, 0.35)   # 350 ns per attempt measured
    # the hard floor: 90 vector instructions per attempt at 5.4 cycles, 2.4 GHz
    assert abs(lb["issue_floor_ms"] - 1000 * 90 * 5.4 / 2.4e9 * 1e3) < 1e-12
    assert abs(lb["issue_floor_ms_at_probe_clock"] - 1000 * 100 * 2.9 / 1e6) < 1e-12
    assert lb["latency_frac"] < lb["ratio_to_issue_floor_at_probe_clock"] < 1.0 < lb["chain_model_ratio"]
    assert bench.fractions_over_one(lb) == []
