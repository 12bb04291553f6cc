"""Benchmark: RK4 Lotka-Volterra ensemble, N=1,000,000, fp32, on one MI355X.

A "step" is one launch of the emitted kernel over the whole ensemble
(dt=0.005, 4,000 RK4 steps per trajectory, running max|y| carried), with
inputs resident in HBM. `value` is trajectory-steps/s over the timed steps.
The roofline figure is the algorithmic FLOP rate (58 FLOP per
trajectory-step) of the kernel's average launch duration, measured with HIP
events on the stream the kernel runs on, against MI355X's 157.3 TFLOP/s
FP32 vector peak. The CPU baseline is the C oracle (oracle/oracle.c, same
op order) on a bounded sample of the same workload, on the host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload lv]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

FP32_PEAK = 157.3e12
HBM_PEAK = 8.0e12


def _cpu_cores() -> int:
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        return int(env)
    return min(os.cpu_count() or 1, 16)


def bench_lv(steps: int, warmup: int, cpu: bool) -> dict:
    import palladium_amd as pa
    from palladium_amd import runtime as rt
    from palladium_amd.workloads import LV_CFG1, LV_FLOP_PER_STEP, lv_inputs, lv_rk4_call

    cfg = LV_CFG1
    n = cfg.n
    host = lv_inputs(n, cfg.seed)
    call = lv_rk4_call(n, cfg.dt, cfg.steps, track_max=True, math_mode=pa.MathMode.FAST)
    bound = call.bound(*host)
    ins = [rt.Buffer.from_numpy(a) for a in host]
    outs = [rt.Buffer.empty((n,), np.float32) for _ in range(3)]
    stream = bound.stream
    ops = [*ins, *outs]
    print(f"[bench] lv_rk4 n={n} steps/traj={cfg.steps} blocks={bound.geometry.blocks}x{bound.geometry.block}", flush=True)
    for _ in range(warmup):
        bound.launch_device(*ops, stream=stream)
    stream.synchronize()

    evs = [rt.Event() for _ in range(steps + 1)]
    rt.synchronize()
    t0 = time.perf_counter()
    evs[0].record(stream)
    for k in range(steps):
        bound.launch_device(*ops, stream=stream)
        evs[k + 1].record(stream)
    stream.synchronize()
    rt.synchronize()
    wall = time.perf_counter() - t0
    per_launch = [evs[k].elapsed_ms(evs[k + 1]) for k in range(steps)]
    total_ms = evs[0].elapsed_ms(evs[-1])
    ms_per_step = total_ms / steps
    traj_steps = n * cfg.steps
    value = traj_steps / (ms_per_step / 1e3)
    avg_launch_s = float(np.mean(per_launch)) / 1e3
    achieved = LV_FLOP_PER_STEP * traj_steps / avg_launch_s

    x = outs[0].to_numpy()
    if not np.all(np.isfinite(x)):
        raise RuntimeError("non-finite results in the benchmark output")

    result = {
        "metric": "trajectory-steps/sec (RK4 LV N=1e6 fp32) + % of FP32 VALU / HBM roofline",
        "value": value,
        "unit": "trajectory-steps/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy default_rng, seed 1)",
        "config": {
            "workload": "RK4 Lotka-Volterra ensemble, N=1,000,000, dt=0.005, 4,000 steps, max|y| carried (config 1)",
            "n": n,
            "dt": cfg.dt,
            "rk4_steps": cfg.steps,
            "math_mode": "fast",
            "block": bound.geometry.block,
            "wall_s": wall,
        },
        "roofline": {
            "bound": "valu",
            "achieved": achieved / 1e12,
            "peak": FP32_PEAK / 1e12,
            "unit": "TFLOP/s",
            "frac": achieved / FP32_PEAK,
            "traffic": None,
            "flop_per_traj_step": LV_FLOP_PER_STEP,
            "avg_launch_ms": avg_launch_s * 1e3,
        },
    }
    if cpu:
        import oracle

        cores = _cpu_cores()
        os.environ.setdefault("OMP_NUM_THREADS", str(cores))
        n_cpu = int(os.environ.get("PALLADIUM_BENCH_CPU_N", n))
        sample = tuple(a[:n_cpu] for a in host)
        oracle.lv_rk4(*(a[:64] for a in host), cfg.dt, 10, track_max=True)  # load + warm
        t0 = time.perf_counter()
        oracle.lv_rk4(*sample, cfg.dt, cfg.steps, track_max=True)
        dt_cpu = time.perf_counter() - t0
        result["cpu_baseline"] = {
            "value": n_cpu * cfg.steps / dt_cpu,
            "unit": "trajectory-steps/s",
            "cores": cores,
            "kind": "port",
            "sample": f"first {n_cpu} of {n} trajectories of config 1, all {cfg.steps} steps, C oracle (gcc -O2, OpenMP, same op order), {dt_cpu:.2f} s",
        }
    return result


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="lv")
    ap.add_argument("--no-cpu", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        print(
            "bench.py measures one GPU: every hot kernel here is per-trajectory or "
            "per-cell on one MI355X; multi-GPU sharding is a design note only.",
            file=sys.stderr,
        )
        return 2
    rank = int(os.environ.get("RANK", "0"))
    if a.workload == "lv":
        res = bench_lv(a.steps, a.warmup, cpu=not a.no_cpu and rank == 0)
    else:
        raise SystemExit(f"unknown workload {a.workload}")
    if rank == 0:
        print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
