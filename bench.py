"""Benchmark of the MLP training step on one MI355X.

Workload: 784 -> 4096 -> 4096 -> 10 MLP (ReLU, softmax cross-entropy on
one-hot targets), batch 1024, f32, one forward + backward + AdamW(1e-3, wd
0.01, betas 0.9/0.999, eps 1e-8) step per iteration on a fixed synthetic batch
already resident in HBM.  Prints ONE JSON line (see the keys below).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-secondary]
                  [--batch B] [--workload NAME] [--path trainer|composed|composed-fused]
                  [--sustained-s S] [--update-shards G]

--batch measures one GPU's share of the 1024-row batch under data parallelism
(512, 256, 128 rows); the default is the benchmark workload itself.
--update-shards G (with --batch 1024 / G) measures that share with the optimizer
state sharded over the G ranks: the step's update passes cover one rank's 1/G
slice of each (the gradients' reduce-scatter and the parameters' all-gather,
which move the bytes of the all-reduce they replace, are not on one GPU).  --workload
and --path step another configuration or the drop-in path instead (for
profiling them); the defaults are the benchmark.

`roofline` reports the dominant kernel (largest device time per step; GEMMs
are told apart by shape): achieved = algorithmic work per launch / mean launch
duration, measured with HIP events on the library's stream over a second pass
of the same K steps; traffic = that kernel's HBM bytes per launch from the
rocprofv3 counter summary under profiles/.
`cpu_baseline` times the CPU oracle (single-threaded sgemm-class GEMM, OpenMP
elementwise ops -- the reference CPU backend's cost structure) on about 10 s of
whole steps of the same workload on this host.
`secondary` holds the path's other workloads measured on the same GPU (small
MLP step times, the [8192, 4096] backward epilogue and AdamW over 2^28
parameters in GB/s).
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

OPT = dict(kind="adamw", lr=1e-3, weight_decay=0.01, betas=(0.9, 0.999), eps=1e-8)
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


def cpu_baseline(dims, params, x, onehot, o=OPT, target_s: float = 8.0) -> dict:
    """Reference-semantics CPU steps of the same workload (the C oracle): one
    untimed warm-up step, then whole steps until about `target_s` seconds."""
    threads = len(os.sched_getaffinity(0))
    os.environ.setdefault("OMP_NUM_THREADS", str(threads))
    from oracle import oracle as O

    if o["kind"] == "adamw":
        opt = O.make_opt("adamw", o["lr"], o.get("weight_decay", 0.0), o.get("betas", (0.9, 0.999)), o.get("eps", 1e-8))
    else:
        opt = O.make_opt(o["kind"], o["lr"])
    r = O.mlp_train(dims, params, x, onehot, opt, steps=1, want_grads=False)  # warm-up (page-in, allocation)
    state = dict(m=r["m"], v=r["v"], t=r["t"])
    cur = r["params"]
    steps, t0 = 0, time.perf_counter()
    while True:
        r = O.mlp_train(dims, cur, x, onehot, opt, steps=1, m=state["m"], v=state["v"], t=state["t"], want_grads=False)
        cur, state = r["params"], dict(m=r["m"], v=r["v"], t=r["t"])
        steps += 1
        dt = time.perf_counter() - t0
        if (dt >= target_s and steps >= 2) or steps >= 25:
            break
    return {
        "value": steps / dt,
        "unit": "steps/s",
        "cores": O.num_threads(),
        "kind": "port",
        "sample": f"{steps} full fwd+bwd+{o['kind']} steps of the same workload after 1 warm-up step ({dt:.1f} s wall); "
                  f"C oracle restating orca-backend-cpu (single-threaded packed sgemm as matrixmultiply without "
                  f"threading, OpenMP elementwise ops as rayon), CPU: {cpu_model()}",
        "samples_per_s": x.shape[0] * steps / dt,
    }


def _call_ms(ctx, fn, reps: int) -> float:
    """Mean time per call of fn (ms) over `reps` back-to-back calls, one HIP event pair on the
    library's stream around all of them: every kernel of a call and the gaps between them."""
    fn()
    ctx.sync()
    ctx.timer_start()
    for _ in range(reps):
        fn()
    return ctx.timer_stop() / reps


def _kernel_times(ctx, fn, reps: int) -> dict:
    """Mean device time per launch (ms) of each profiled kernel over `reps` calls of fn."""
    fn()
    ctx.sync()
    ctx.prof_reset()
    ctx.prof_enable(True)
    for _ in range(reps):
        fn()
    rep = ctx.prof_report()
    ctx.prof_enable(False)
    return {k["name"]: k["total_ms"] / k["launches"] for k in rep["kernels"]}


def secondary(ctx) -> dict:
    """The other workloads of the path, on the same GPU: step time of the two
    small MLP configurations (784-128-128-10 B=64 SGD; 784-1024-1024-10 B=256
    AdamW), the 784-4096-4096-10 step through the drop-in path (reference
    frontend and tape over the trait ops), the fused backward epilogue on
    [8192, 4096] (softmax-CE gradient with int targets; ReLU-mask backward +
    bias column sum), and AdamW over one flat buffer of 2^28 parameters.
    Bandwidths are algorithmic bytes / mean kernel time."""
    import ctypes

    from orcaml_amd import _lib, synth
    from orcaml_amd.mlp import MLPTrainer

    out = {}
    for name in (synth.MLP_SMALL, synth.MLP_MEDIUM):
        w = synth.WORKLOADS[name]
        o = w["opt"]
        params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
        tr = MLPTrainer(ctx, w["dims"], w["batch"], kind=o["kind"], lr=o["lr"], weight_decay=o.get("weight_decay", 0.0),
                        betas=o.get("betas", (0.9, 0.999)), eps=o.get("eps", 1e-8))
        tr.set_params(params)
        tr.set_batch(x, onehot=onehot)
        for _ in range(5):
            tr.step()
        ctx.sync()
        n = 200
        t0 = time.perf_counter()
        for _ in range(n):
            tr.step()
        ctx.sync()
        dt = (time.perf_counter() - t0) / n
        out[w["name"]] = {"ms_per_step": dt * 1e3, "steps_per_s": 1.0 / dt, "samples_per_s": w["batch"] / dt}
        tr.close()

    # The drop-in path: the reference frontend (nn.Sequential of Linear/ReLU,
    # CrossEntropyLoss, AdamW) and the autodiff tape running on the backend's
    # trait ops, unchanged and with the opt-in fused loss and optimizer.
    from orcaml_amd import autodiff as A
    from orcaml_amd.backend import HipBackend

    w = synth.WORKLOADS[synth.MLP_LARGE]
    params, x, labels, onehot = synth.mlp_problem(w["seed"], w["dims"], w["batch"])
    composed = {}
    for tag, fused in (("unchanged", False), ("fused_loss_and_adamw", True)):
        ad = A.Autodiff(HipBackend(ctx))
        model = A.build_mlp(ad, params)
        opt = A.AdamW(model.parameters(), lr=OPT["lr"], weight_decay=OPT["weight_decay"], fused=fused)
        xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)

        def step():
            opt.zero_grad()
            A.CrossEntropyLoss(fused=fused)(model(xt), tt).backward()
            opt.step()

        for _ in range(10):  # the first steps compile the recurring program structures
            step()
        ctx.sync()
        # three windows of 20 steps, the median one reported (a host pause in one window,
        # a garbage collection say, does not decide the figure)
        n, windows = 20, []
        for _ in range(3):
            t0 = time.perf_counter()
            for _ in range(n):
                step()
            ctx.sync()
            windows.append((time.perf_counter() - t0) / n)
        dt = sorted(windows)[1]
        composed[tag] = {"ms_per_step": dt * 1e3, "steps_per_s": 1.0 / dt,
                         "windows_ms": [round(wd * 1e3, 4) for wd in windows]}
    out["composed_" + w["name"]] = composed

    # Fused backward epilogue, [8192, 4096].
    B, C = 8192, 4096
    logits = ctx.upload(synth.normal(4, 1, (B, C), 0.0, 2.0))
    labels = ctx.upload(synth.integers(4, 2, B, C))
    pre = ctx.upload(synth.normal(4, 3, (B, C)))
    loss, grad = ctx.alloc(4), ctx.alloc(4 * B * C)
    dpre, colsum = ctx.alloc(4 * B * C), ctx.alloc(4 * C)
    kt = _kernel_times(ctx, lambda: _lib.call("orca_hip_softmax_ce", ctx.handle, logits.ptr, B, C, None, labels.ptr,
                                              loss.ptr, grad.ptr, None, None), 20)
    ce_bytes = 8.0 * B * C + 4.0 * B
    def relu_bw():
        _lib.call("orca_hip_relu_bw_colsum", ctx.handle, grad.ptr, pre.ptr, B, C, dpre.ptr, colsum.ptr)

    kt2 = _kernel_times(ctx, relu_bw, 20)
    rb_ms = _call_ms(ctx, relu_bw, 20)  # the call: its two launches back to back
    rb_bytes = 12.0 * B * C + 4.0 * C
    out["epilogue_8192x4096"] = {
        "softmax_ce_grad": {"ms": kt["softmax_ce"], "bytes": ce_bytes,
                            "GB_per_s": ce_bytes / (kt["softmax_ce"] * 1e-3) / 1e9},
        "relu_bw_colsum": {"ms": rb_ms, "bytes": rb_bytes, "GB_per_s": rb_bytes / (rb_ms * 1e-3) / 1e9,
                           "timing": "per call over 20 back-to-back calls (one event pair)",
                           "kernel_ms": {"relu_bw_colsum": kt2["relu_bw_colsum"],
                                         "colsum_chunks": kt2.get("colsum_chunks", 0.0)}},
        "peak_GB_per_s": PEAK_HBM_GBS,
    }
    for b in (logits, labels, pre, loss, grad, dpre, colsum):
        b.free()

    # AdamW over 2^28 parameters, 10 steps (p, g tiled from 2^24 generated values).
    n, chunk = 1 << 28, 1 << 24
    bufs = [ctx.alloc(4 * n) for _ in range(4)]
    p_dev, g_dev, m_dev, v_dev = bufs
    pc = synth.normal_range(5, 1, 0, chunk, 0.0, 0.02)
    gc = synth.normal_range(5, 2, 0, chunk, 0.0, 1e-3)
    for buf, arr in ((p_dev, pc), (g_dev, gc)):
        for off in range(0, n, chunk):
            _lib.call("orca_hip_h2d", ctx.handle, buf.ptr + 4 * off, arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes)
    ctx.fill(m_dev, 0.0, n)
    ctx.fill(v_dev, 0.0, n)
    step = [0]

    def adamw():
        step[0] += 1
        _lib.call("orca_hip_adamw_step", ctx.handle, p_dev.ptr, g_dev.ptr, m_dev.ptr, v_dev.ptr, n, OPT["lr"],
                  OPT["betas"][0], OPT["betas"][1], OPT["eps"], OPT["weight_decay"], step[0])

    kt = _kernel_times(ctx, adamw, 9)  # one untimed + 9 timed = 10 steps
    ms = kt["adamw"]
    out["adamw_2pow28"] = {"ms_per_step": ms, "bytes_per_step": 28.0 * n, "GB_per_s": 28.0 * n / (ms * 1e-3) / 1e9,
                           "frac_hbm_peak": 28.0 * n / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                           "GB_per_s_at_20B_per_elem": 20.0 * n / (ms * 1e-3) / 1e9,
                           "data": "p ~ N(0, 0.02^2), g ~ N(0, 1e-3^2): 2^24 generated values tiled 16x; m = v = 0"}
    for b in bufs:
        b.free()
    return out


def _composed_step(ctx, dims, batch, o, params, x, onehot, fused: bool):
    """One step of the drop-in path: the reference frontend (nn.Sequential of Linear/ReLU,
    CrossEntropyLoss, SGD/AdamW) and the autodiff tape over HipBackend's trait ops."""
    from orcaml_amd import autodiff as A
    from orcaml_amd.backend import HipBackend

    ad = A.Autodiff(HipBackend(ctx))
    model = A.build_mlp(ad, params)
    if o["kind"] == "adamw":
        opt = A.AdamW(model.parameters(), lr=o["lr"], weight_decay=o.get("weight_decay", 0.0), fused=fused)
    else:
        opt = A.SGD(model.parameters(), lr=o["lr"], fused=fused)
    xt, tt = A.Tensor.from_numpy(ad, x), A.Tensor.from_numpy(ad, onehot)

    def step():
        opt.zero_grad()
        A.CrossEntropyLoss(fused=fused)(model(xt), tt).backward()
        opt.step()

    return step


def main() -> int:
    from orcaml_amd import synth

    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=30)  # 5 warm-up steps left the first timed ones ~1 % slower
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true", help="skip the other workloads' measurements")
    ap.add_argument("--workload", default=synth.MLP_LARGE, choices=sorted(synth.WORKLOADS),
                    help="the MLP configuration stepped (default: the benchmark workload)")
    ap.add_argument("--path", default="trainer", choices=("trainer", "composed", "composed-fused"),
                    help="trainer: the device-resident training step (the benchmark); composed: the reference "
                         "frontend and tape over the trait ops; composed-fused: the same with the opt-in fused "
                         "loss and optimizer")
    ap.add_argument("--batch", type=int, default=None,
                    help="rows per step (default: the workload's; for the benchmark workload 512 / 256 / 128 are "
                         "one GPU's share of its 1024-row batch under 2 / 4 / 8-way data parallelism)")
    ap.add_argument("--update-shards", type=int, default=1,
                    help="trainer path: update one rank's 1/G slice of each update pass (the optimizer state "
                         "sharded over G data-parallel ranks); 1, the default, updates every parameter")
    ap.add_argument("--sustained-s", type=float, default=3.0,
                    help="after the timed steps, keep stepping for about this many seconds and report that rate "
                         "too (a window long enough for an outside observer of the GPU); 0 skips it")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first run one device-to-device copy of this many MiB (a known-size kernel that "
                         "calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the library has no multi-GPU path",
              file=sys.stderr)
        return 2
    if args.update_shards < 1:
        print(f"--update-shards must be at least 1 (got {args.update_shards})", file=sys.stderr)
        return 2

    from orcaml_amd.device import Context
    from orcaml_amd.mlp import MLPTrainer

    w = synth.WORKLOADS[args.workload]
    dims, seed = tuple(w["dims"]), w["seed"]
    o = dict(OPT) if args.workload == synth.MLP_LARGE else dict(w["opt"])
    batch = args.batch if args.batch is not None else w["batch"]
    params, x, labels, onehot = synth.mlp_problem(seed, dims, batch)
    ctx = Context(0)
    if args.copy_probe_mib > 0:
        nbytes = args.copy_probe_mib << 20
        src, dst = ctx.alloc(nbytes), ctx.alloc(nbytes)
        ctx.fill(src, 1.0, nbytes // 4)
        ctx.d2d(dst, src, nbytes)
        ctx.sync()
        src.free()
        dst.free()
    tr = None
    if args.path == "trainer":
        tr = MLPTrainer(ctx, dims, batch, kind=o["kind"], lr=o["lr"], weight_decay=o.get("weight_decay", 0.0),
                        betas=o.get("betas", (0.9, 0.999)), eps=o.get("eps", 1e-8))
        tr.set_params(params)
        tr.set_batch(x, onehot=onehot)
        if args.update_shards > 1:
            tr.set_update_shard(0, args.update_shards)
        step = tr.step
    else:
        if args.update_shards != 1:
            print("--update-shards applies to the trainer path only", file=sys.stderr)
            return 2
        step = _composed_step(ctx, dims, batch, o, params, x, onehot, fused=args.path == "composed-fused")
    mallocs_before = None

    for _ in range(args.warmup):
        step()
    ctx.sync()
    mallocs_before = ctx.mem_stats()["device_allocs"]

    # ---- timed region: K steps, synchronised on both sides ----
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctx.sync()
    wall = time.perf_counter() - t0
    loss, correct = tr.metrics() if tr is not None else (None, None)
    mallocs_after = ctx.mem_stats()["device_allocs"]

    # ---- sustained: the same step for about --sustained-s seconds, in rounds of 100 ----
    sustained = None
    if args.sustained_s > 0:
        done, t0 = 0, time.perf_counter()
        while True:
            for _ in range(100):
                step()
            done += 100
            ctx.sync()
            elapsed = time.perf_counter() - t0
            if elapsed >= args.sustained_s:
                break
        sustained = {"steps": done, "seconds": elapsed, "steps_per_s": done / elapsed,
                     "ms_per_step": elapsed * 1e3 / done}

    # ---- per-kernel device time over a second pass of K steps ----
    ctx.prof_reset()
    ctx.prof_enable(True)
    for _ in range(args.steps):
        step()
    report = ctx.prof_report()
    ctx.prof_enable(False)
    kernels = report["kernels"]
    per_step = {k["name"]: k["total_ms"] / args.steps for k in kernels}
    # The dominant kernel of the step's critical path: launches on the second
    # stream ("*_overlapped", the optimizer update beside the GEMMs) last as
    # long as the work they run beside and are not counted.
    dominant = max((k for k in kernels if not k["name"].endswith("_overlapped")), key=lambda k: k["total_ms"])
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
    if args.path == "trainer" and os.path.exists(os.path.join(HERE, traffic_file)):
        with open(os.path.join(HERE, traffic_file)) as fh:
            rec = json.load(fh)["kernels"].get(dominant["name"])
        if rec is not None:
            roof["traffic"] = rec["traffic_bytes"]
            roof["traffic_source"] = traffic_file
    mfma = [k for k in kernels if k["name"].startswith("gemm_") and k["flops"] > 0]  # the MFMA GEMMs
    gemm_ms = sum(k["total_ms"] for k in mfma) / args.steps
    gemm_flops = sum(k["flops"] for k in mfma) / args.steps

    ms_per_step = wall * 1e3 / args.steps
    steps_per_s = args.steps / wall
    flops = step_flops(dims, batch)
    out = {
        "metric": f"MLP train steps/s ({'-'.join(str(d) for d in dims)} fp32, B={batch}); % fp32 MFMA peak",
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
        "config": {"workload": "mlp_train_step", "dims": list(dims), "batch": batch, "optimizer": o["kind"],
                   "lr": o["lr"], "weight_decay": o.get("weight_decay", 0.0), "seed": seed, "path": args.path,
                   "update_shard": f"1/{args.update_shards}" if args.update_shards > 1 else "all"},
        "samples_per_s": steps_per_s * batch,
        "step_tflops": flops * steps_per_s / 1e12,
        "step_frac_fp32_mfma_peak": flops * steps_per_s / 1e12 / PEAK_FP32_MFMA_TFLOPS,
        "gemm_tflops": gemm_flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms > 0 else None,
        "kernel_ms_per_step": per_step,
        "last_loss": loss,
        "last_correct": correct,
        "device_allocs_in_timed_region": mallocs_after - mallocs_before,
        "roofline": roof,
        "sustained": sustained,
    }
    if tr is not None:
        tr.close()
    step = None
    if not args.no_secondary:
        out["secondary"] = secondary(ctx)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(dims, params, x, onehot, o)
        out["gpu_over_cpu"] = steps_per_s / out["cpu_baseline"]["value"]
    print(json.dumps(out))
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
