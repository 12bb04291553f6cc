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


def _timed_launches(bound, ops, steps: int, warmup: int):
    from palladium_amd import runtime as rt

    stream = bound.stream
    for _ in range(warmup):
        bound.launch_device(*ops, stream=stream)
    stream.synchronize()
    evs = [rt.Event() for _ in range(steps + 1)]
    evs[0].record(stream)
    for k in range(steps):
        bound.launch_device(*ops, stream=stream)
        evs[k + 1].record(stream)
    stream.synchronize()
    per = [evs[k].elapsed_ms(evs[k + 1]) for k in range(steps)]
    return evs[0].elapsed_ms(evs[-1]) / steps, float(np.mean(per))


def _base(metric: str, value: float, unit: str, steps: int, warmup: int, ms: float, config: dict) -> dict:
    return {
        "metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded)", "config": config,
    }


def bench_gbm(steps: int, warmup: int, cpu: bool) -> dict:
    from palladium_amd import runtime as rt
    from palladium_amd.frontend import random
    from palladium_amd.workloads import GBM_CFG, gbm_call

    cfg = GBM_CFG
    key = random.key(cfg.seed)
    bound = gbm_call(cfg).bound(key)
    ops = [rt.Buffer.from_numpy(key), rt.Buffer.empty((cfg.n_paths,), np.float32)]
    ms, avg = _timed_launches(bound, ops, steps, warmup)
    ps = cfg.n_paths * cfg.n_steps
    res = _base("GBM path-steps/s (4,194,304 paths x 252 steps, Threefry + Box-Muller, fp32)", ps / (ms / 1e3),
                "path-steps/s", steps, warmup, ms,
                {"workload": "GBM Monte Carlo, config 3", "paths": cfg.n_paths, "steps": cfg.n_steps, "math_mode": "fast"})
    res["roofline"] = {"bound": "valu", "achieved": None, "peak": None, "unit": None, "frac": None, "traffic": None,
                       "avg_launch_ms": avg}
    if cpu:
        import oracle

        n_cpu = 65536
        oracle.gbm(cfg, 64)
        t0 = time.perf_counter()
        oracle.gbm(cfg, n_cpu)
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": n_cpu * cfg.n_steps / dt, "unit": "path-steps/s", "cores": _cpu_cores(),
                               "kind": "port", "sample": f"{n_cpu} paths x {cfg.n_steps} steps, C oracle, {dt:.2f} s"}
    return res


def bench_gs(steps: int, warmup: int, cpu: bool) -> dict:
    from palladium_amd.workloads import GS_BYTES_PER_CELL_STEP, GS_CFG, gray_scott_call, gray_scott_initial, gray_scott_run

    cfg = GS_CFG
    u0, v0 = gray_scott_initial(cfg.size)
    call = gray_scott_call(cfg)
    gray_scott_run(call, u0, v0, 10)  # compile + warm
    n_steps = cfg.steps
    _, v, gpu_s = gray_scott_run(call, u0, v0, n_steps, graph=True)
    cells = cfg.size * cfg.size
    ms = gpu_s * 1e3 / n_steps
    achieved = GS_BYTES_PER_CELL_STEP * cells / (ms / 1e3)
    res = _base("Gray-Scott cell-steps/s (4096^2, 2,000 steps, fp32)", cells / (ms / 1e3), "cell-steps/s",
                n_steps, 10, ms, {"workload": "Gray-Scott 4096x4096, 2000 steps as one HIP graph, config 4",
                                  "size": cfg.size, "math_mode": "fast"})
    res["roofline"] = {"bound": "hbm", "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                       "frac": achieved / HBM_PEAK, "traffic": None, "bytes_per_cell_step": GS_BYTES_PER_CELL_STEP,
                       "avg_launch_ms": ms}
    res["pattern_energy"] = float(np.sum(v, dtype=np.float64))
    if cpu:
        import oracle

        size = 1024
        su, sv = gray_scott_initial(size)
        t0 = time.perf_counter()
        oracle.gray_scott(su, sv, cfg, 20)
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": size * size * 20 / dt, "unit": "cell-steps/s", "cores": _cpu_cores(),
                               "kind": "port", "sample": f"{size}^2 grid x 20 steps, C oracle, {dt:.2f} s"}
    return res


def bench_bs3(steps: int, warmup: int, cpu: bool) -> dict:
    from palladium_amd import runtime as rt
    from palladium_amd.workloads import BS3_CFG, bs3_inputs, bs3_vdp_call

    cfg = BS3_CFG
    host = bs3_inputs(cfg.n)
    bound = bs3_vdp_call(cfg.n).bound(*host)
    ins = [rt.Buffer.from_numpy(a) for a in host]
    outs = [rt.Buffer.empty((cfg.n,), np.float32) for _ in range(3)] + [rt.Buffer.empty((cfg.n,), np.int32) for _ in range(2)]
    ms, avg = _timed_launches(bound, ins + outs, steps, warmup)
    acc = outs[3].to_numpy().astype(np.int64)
    rej = outs[4].to_numpy().astype(np.int64)
    attempts = acc + rej
    waves = attempts[: (cfg.n // 64) * 64].reshape(-1, 64)
    active = float(waves.sum() / (waves.max(axis=1).sum() * 64))
    total = int(attempts.sum())
    res = _base("BS3(2)+PI attempted steps/s (Van der Pol, N=262,144, fp32)", total / (ms / 1e3), "attempts/s",
                steps, warmup, ms, {"workload": "adaptive BS3(2) Van der Pol, config 2", "n": cfg.n, "math_mode": "fast"})
    res["roofline"] = {"bound": "valu", "achieved": None, "peak": None, "unit": None, "frac": None, "traffic": None,
                       "avg_launch_ms": avg, "active_lane_fraction": active, "total_attempts": total,
                       "accepted": int(acc.sum()), "rejected": int(rej.sum())}
    if cpu:
        import oracle

        n_cpu = 16384
        t0 = time.perf_counter()
        a2 = oracle.bs3_vdp(*(h[:n_cpu] for h in host), cfg)
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": float((a2[3].astype(np.int64) + a2[4]).sum() / dt), "unit": "attempts/s",
                               "cores": _cpu_cores(), "kind": "port", "sample": f"first {n_cpu} trajectories, C oracle, {dt:.2f} s"}
    return res


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
    fns = {"lv": bench_lv, "gbm": bench_gbm, "gs": bench_gs, "bs3": bench_bs3}
    if a.workload not in fns:
        raise SystemExit(f"unknown workload {a.workload} (choose from {', '.join(fns)})")
    res = fns[a.workload](a.steps, a.warmup, cpu=not a.no_cpu and rank == 0)
    if rank == 0:
        print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
