"""Headline benchmark: BF16-in / F32-accumulate C = A.B at 4096^3 on one MI355X.

BASELINE.json's metric is "matmul TFLOP/s (% MFMA peak) + SmolLM2-135M-shape
decoder tokens/sec, 1 GPU"; its matmul configuration (configs[1], the cube
sweep) at its target size, bf16 4096^3, is the workload of `value`.  A step is
one product of two resident [4096, 4096] BF16 matrices into a fresh F32 result
through the C ABI (`mi_matmul`), inputs already in HBM.

Printed: one JSON line with `value` (TFLOP/s over the timed steps, wall clock
with a stream sync on both sides), the kernel's roofline (achieved TFLOP/s
from HIP events recorded on the engine's own stream around the timed steps,
against MI355X's dense BF16 peak), and the CPU baseline (the oracle's F32
product timed on this host's cores on a bounded 1024^3 sample).

Flags: --gpus N (only 1: this build runs on one GPU), --steps K, --warmup W,
--n (cube size, default 4096), --dtype bf16|f32, --no-cpu.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "metalium-rs_amd"))

PEAK_TFLOPS = {"bf16": 2516.6, "f32": 157.3}  # MI355X dense MFMA (AMD published)
HBM_PEAK_GBS = 8000.0


def cpu_baseline(n: int = 1024) -> dict:
    """The oracle's F32 product (k ascending, F32 accumulation, OpenMP over
    rows) on this host's cores: the CPU restatement standing in for burn-flex,
    which cannot be built here."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as orc
    cores = len(os.sched_getaffinity(0))
    cores = min(cores, 16)  # the GPU box's CPU share
    rng = np.random.default_rng(1)
    a = rng.standard_normal((n, n)).astype(np.float32)
    b = rng.standard_normal((n, n)).astype(np.float32)
    orc.matmul_f32acc(a[:64], b, threads=cores)  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        orc.matmul_f32acc(a, b, threads=cores)
        reps += 1
        el = time.perf_counter() - t0
        if el > 3.0 or reps >= 20:
            break
    tflops = 2.0 * n ** 3 * reps / el / 1e12
    return {"value": round(tflops, 5), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"oracle F32 product {n}^3 (k-ascending F32 accumulation, OpenMP rows), {reps} reps in {el:.2f} s"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--n", type=int, default=4096)
    ap.add_argument("--dtype", choices=["bf16", "f32"], default="bf16")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(sharding is described in DESIGN.md, not run)", file=sys.stderr)
        return 2

    import miburn
    eng = miburn.Engine(0)
    n = args.n
    draw = miburn.DRAW_NORMAL
    a32 = eng.random_dram(n, n, draw, 0.0, 1.0, base=11)
    b32 = eng.random_dram(n, n, draw, 0.0, 1.0, base=12)
    if args.dtype == "bf16":
        a = eng.cast_float(a32, miburn.BF16)
        b = eng.cast_float(b32, miburn.BF16)
        eng.free(a32)
        eng.free(b32)
    else:
        a, b = a32, b32
    eng.sync()

    for _ in range(args.warmup):
        eng.free(eng.matmul_dram(a, False, b, False))
    eng.sync()

    eng.event_record(0)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        c = eng.matmul_dram(a, False, b, False)
        eng.free(c)
    eng.event_record(1)
    eng.sync()
    wall = time.perf_counter() - t0
    kernel_ms = eng.event_elapsed_ms(0, 1) / args.steps

    flop = 2.0 * n ** 3
    value = flop * args.steps / wall / 1e12
    achieved = flop / (kernel_ms * 1e-3) / 1e12
    peak = PEAK_TFLOPS[args.dtype]
    elt = 2 if args.dtype == "bf16" else 4
    traffic_min = (2 * n * n * elt + n * n * 4)
    line = {
        "metric": "matmul TFLOP/s (% MFMA peak) + SmolLM2-135M-shape decoder tokens/sec, 1 GPU",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (device N(0,1) draws)",
        "config": {"workload": f"matmul {args.dtype}-in/f32-acc C=A.B {n}^3, A and B row-major (NN)",
                   "m": n, "n": n, "k": n},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4), "traffic": None,
                     "kernel_ms": round(kernel_ms, 5), "min_hbm_bytes": traffic_min},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)
    eng.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
