"""Benchmark of the MLP training step on one MI355X.

Workload: 784 -> 4096 -> 4096 -> 10 MLP (ReLU, softmax cross-entropy on
one-hot targets), batch 1024, f32, one forward + backward + AdamW(1e-3, wd
0.01, betas 0.9/0.999, eps 1e-8) step per iteration on a fixed synthetic batch
already resident in HBM.  Prints ONE JSON line (see the keys below).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

`roofline` reports the dominant kernel (largest device time per step; GEMMs
are told apart by shape): achieved = algorithmic work per launch / mean launch
duration, measured with HIP events on the library's stream over a second pass
of the same K steps; traffic = that kernel's HBM bytes per launch from the
rocprofv3 counter summary under profiles/.
`cpu_baseline` times the CPU oracle (single-threaded sgemm-class GEMM, OpenMP
elementwise ops -- the reference CPU backend's cost structure) on one step of
the same workload on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

DIMS = (784, 4096, 4096, 10)
BATCH = 1024
OPT = dict(kind="adamw", lr=1e-3, weight_decay=0.01, betas=(0.9, 0.999), eps=1e-8)
SEED = 3
# MI355X published peaks.
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0


def step_flops(dims, batch) -> float:
    """2*M*N*K per GEMM: forward L, dW L, dX L-1 (the first layer has no dX)."""
    f = 0.0
    for l in range(len(dims) - 1):
        k, n = dims[l], dims[l + 1]
        f += 2.0 * batch * k * n * (3 if l > 0 else 2)
    return f


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(params, x, onehot) -> dict:
    """One reference-semantics CPU step of the same workload (oracle)."""
    threads = len(os.sched_getaffinity(0))
    os.environ.setdefault("OMP_NUM_THREADS", str(threads))
    from oracle import oracle as O

    opt = O.make_opt("adamw", OPT["lr"], OPT["weight_decay"], OPT["betas"], OPT["eps"])
    t0 = time.perf_counter()
    r = O.mlp_train(DIMS, params, x, onehot, opt, steps=1, want_grads=False)
    dt = time.perf_counter() - t0
    return {
        "value": 1.0 / dt,
        "unit": "steps/s",
        "cores": O.num_threads(),
        "kind": "port",
        "sample": f"1 full fwd+bwd+AdamW step of the same workload ({dt:.2f} s wall); C oracle restating "
                  f"orca-backend-cpu (single-threaded packed sgemm, OpenMP elementwise), CPU: {cpu_model()}",
        "loss": float(r["losses"][0]),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first run one device-to-device copy of this many MiB (a known-size kernel that "
                         "calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        return 2

    from orcaml_amd import synth
    from orcaml_amd.device import Context
    from orcaml_amd.mlp import MLPTrainer

    params, x, labels, onehot = synth.mlp_problem(SEED, DIMS, BATCH)
    ctx = Context(0)
    if args.copy_probe_mib > 0:
        nbytes = args.copy_probe_mib << 20
        src, dst = ctx.alloc(nbytes), ctx.alloc(nbytes)
        ctx.fill(src, 1.0, nbytes // 4)
        ctx.d2d(dst, src, nbytes)
        ctx.sync()
        src.free()
        dst.free()
    tr = MLPTrainer(ctx, DIMS, BATCH, kind=OPT["kind"], lr=OPT["lr"], weight_decay=OPT["weight_decay"],
                    betas=OPT["betas"], eps=OPT["eps"])
    tr.set_params(params)
    tr.set_batch(x, onehot=onehot)
    mallocs_before = None

    for _ in range(args.warmup):
        tr.step()
    ctx.sync()
    mallocs_before = ctx.mem_stats()["device_allocs"]

    # ---- timed region: K steps, synchronised on both sides ----
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        tr.step()
    ctx.sync()
    wall = time.perf_counter() - t0
    loss, correct = tr.metrics()
    mallocs_after = ctx.mem_stats()["device_allocs"]

    # ---- per-kernel device time over a second pass of K steps ----
    ctx.prof_reset()
    ctx.prof_enable(True)
    for _ in range(args.steps):
        tr.step()
    report = ctx.prof_report()
    ctx.prof_enable(False)
    kernels = report["kernels"]
    per_step = {k["name"]: k["total_ms"] / args.steps for k in kernels}
    dominant = max(kernels, key=lambda k: k["total_ms"])
    avg_ms = dominant["total_ms"] / dominant["launches"]
    if dominant["flops"] > 0:
        work = dominant["flops"] / dominant["launches"]
        achieved = work / (avg_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": achieved, "peak": PEAK_FP32_MFMA_TFLOPS, "unit": "TFLOP/s",
                "frac": achieved / PEAK_FP32_MFMA_TFLOPS, "traffic": None}
    else:
        work = dominant["bytes"] / dominant["launches"]
        achieved = work / (avg_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": achieved / PEAK_HBM_GBS, "traffic": None}
    roof["kernel"] = dominant["name"]
    roof["launches_per_step"] = dominant["launches"] / args.steps
    roof["mean_launch_ms"] = avg_ms
    # HBM bytes per launch of this kernel from the committed rocprofv3 FETCH_SIZE + WRITE_SIZE passes
    # (calibrated against a copy of known size); null when the kernel has no such record.
    traffic_file = os.path.join("profiles", "hbm_traffic_mlp784-4096-4096-10_b1024.json")
    if os.path.exists(os.path.join(HERE, traffic_file)):
        with open(os.path.join(HERE, traffic_file)) as fh:
            rec = json.load(fh)["kernels"].get(dominant["name"])
        if rec is not None:
            roof["traffic"] = rec["traffic_bytes"]
            roof["traffic_source"] = traffic_file
    gemm_ms = sum(k["total_ms"] for k in kernels if k["flops"] > 0) / args.steps
    gemm_flops = sum(k["flops"] for k in kernels if k["flops"] > 0) / args.steps

    ms_per_step = wall * 1e3 / args.steps
    steps_per_s = args.steps / wall
    flops = step_flops(DIMS, BATCH)
    out = {
        "metric": "MLP train steps/s (784-4096-4096-10 fp32, B=1024); % fp32 MFMA peak",
        "value": steps_per_s,
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "mlp_train_step", "dims": list(DIMS), "batch": BATCH, "optimizer": "adamw",
                   "lr": OPT["lr"], "weight_decay": OPT["weight_decay"], "seed": SEED},
        "samples_per_s": steps_per_s * BATCH,
        "step_tflops": flops * steps_per_s / 1e12,
        "step_frac_fp32_mfma_peak": flops * steps_per_s / 1e12 / PEAK_FP32_MFMA_TFLOPS,
        "gemm_tflops": gemm_flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms > 0 else None,
        "kernel_ms_per_step": per_step,
        "last_loss": loss,
        "last_correct": correct,
        "device_allocs_in_timed_region": mallocs_after - mallocs_before,
        "roofline": roof,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(params, x, onehot)
    print(json.dumps(out))
    tr.close()
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
