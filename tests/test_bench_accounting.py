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
