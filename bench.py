"""Throughput of GoNeuron's fp32 training step (forward + backward + Adam) on
one MI355X, with the roofline fraction of the dominant kernel and the CPU
reference path timed beside it.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config wide]

Prints ONE JSON line.  `value` is samples/s with inputs resident in HBM; the
GEMM family's achieved TFLOP/s comes from HIP events recorded around every
GEMM launch on the library's stream during the timed steps.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBPS = 8000.0

# HBM bytes per training step moved by the GEMM family, from rocprofv3 --pmc
# FETCH_SIZE (x2.000) and WRITE_SIZE (x1.000) passes, each scaled by what the
# counter reads for a 1 GiB device-to-device copy (bench.py --copy-probe 1024).
# Keyed by workload; a changed GEMM kernel needs a new measurement.
GEMM_TRAFFIC_BYTES_PER_STEP = {"wide": 2861.0e6}


def gemm_flops(cfg, B):
    """Algorithmic GEMM FLOPs of one step: forward 2*B*in*out per Dense,
    dW the same, dX for every Dense but the first (its dX is discarded)."""
    f = 0
    dense = [d for d in cfg["layers"] if d["kind"] == "dense"]
    for i, d in enumerate(dense):
        mac = B * d["in"] * d["out"]
        f += 2 * mac + 2 * mac + (2 * mac if i > 0 else 0)
    return f


def cpu_baseline(cfg, x, y, budget_s=15.0, workers=1, threads=None):
    """The CPU oracle (C restatement of the reference's per-sample path) timed
    on the host, on a bounded sample, two ways:
      - parallel (the reported value): trainBatchParallel's structure
        (net.go:588-717) with T threads, each a private network (own layer
        state and gradient arena, as LightweightClone) running its own
        contiguous chunk; then the serial sum of the T gradient arenas and one
        Adam pass, per batch;
      - single thread: trainBatchSequential (net.go:721-784).
    samples/s = samples / (sample time + per-batch time * samples / B)."""
    import threading
    from oracle import refcpu
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from cfgutil import oracle_net
    refcpu.build()
    B = cfg["B"]
    T = threads or min(B, os.cpu_count() or 1, 16)
    nets = [oracle_net(refcpu, cfg) for _ in range(T)]
    net = nets[0]
    # calibrate with one sample, then fill the budget
    t0 = time.perf_counter()
    net.accumulate_batch(x[:1], y[:1], 1)
    t1 = time.perf_counter() - t0
    n1 = int(max(1, min(B, budget_s / 2 / max(t1, 1e-6))))
    t0 = time.perf_counter()
    net.accumulate_batch(x[:n1], y[:n1], n1)
    ts1 = time.perf_counter() - t0
    net.step()  # first touch of the Adam moments, untimed
    t0 = time.perf_counter()
    net.step()
    ta = time.perf_counter() - t0
    single = n1 / (ts1 + ta * n1 / B)
    # parallel: every thread takes npt samples of its own chunk of the batch
    chunk = (B + T - 1) // T
    npt = int(max(1, min(chunk, budget_s / 2 / max(t1, 1e-6))))

    def work(t, n):
        s0 = min(t * chunk, B - n)
        nets[t].accumulate_batch(x[s0:s0 + n], y[s0:s0 + n], n)

    def run_all(n):
        th = [threading.Thread(target=work, args=(t, n)) for t in range(T)]
        for h in th:
            h.start()
        for h in th:
            h.join()

    run_all(1)  # first touch of every worker's buffers, untimed
    acc = np.zeros_like(net.grads)
    acc += 1.0
    t0 = time.perf_counter()
    run_all(npt)
    tp = time.perf_counter() - t0
    t0 = time.perf_counter()  # serial sum of the worker arenas (net.go:694-700)
    acc[:] = 0.0
    for nt in nets:
        acc += nt.grads
    tsum = time.perf_counter() - t0
    done = T * npt
    par = done / (tp + (tsum + ta) * done / B)
    del nets
    return {"value": par, "unit": "samples/s", "cores": T, "kind": "port",
            "sample": f"oracle/refcpu (C restatement of the per-sample path, -O2 -ffp-contract=off): "
                      f"{T} threads x {npt} samples of their own chunks of the {B}-sample batch "
                      f"({tp:.2f} s), plus per batch the sum of {T} gradient arenas ({tsum:.3f} s) and one "
                      f"Adam pass over {net.n} params ({ta:.3f} s) scaled by samples/B",
            "single_thread": {"value": single, "cores": 1,
                              "sample": f"{n1} of {B} samples fwd+bwd ({ts1:.2f} s) + Adam scaled by n/B"}}


def predict_bench(args, cfg, model, dev, dx, B, workers):
    """Inference throughput (f3): K forward passes in inference mode over the
    config's batch, inputs and outputs in HBM."""
    import ctypes as C
    from goneuron_amd._lib import lib, check
    out = C.c_void_p()
    check(dev.h, lib().gn_malloc(dev.h, B * model.out_size * 4, C.byref(out)))
    run = lambda: check(dev.h, lib().gn_model_predict_device(model.h, dx, B, out))
    for _ in range(args.warmup):
        run()
    dev.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    dev.sync()
    el = time.perf_counter() - t0
    print(json.dumps({"metric": "predict samples/s (inference forward) on 1 MI355X", "value": args.steps * B / el,
                      "unit": "samples/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                      "ms_per_step": 1e3 * el / args.steps, "higher_is_better": True,
                      "dtype": "f32", "data": "synthetic",
                      "config": {"workload": cfg["name"], "batch": B, "mode": "inference"}}), flush=True)
    check(dev.h, lib().gn_free(dev.h, out))


def copy_probe(mib):
    """A copy kernel of known size: reads and writes mib MiB per launch."""
    import torch
    n = mib * (1 << 20) // 4
    a = torch.ones(n, device="cuda:0")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_per_launch": n * 4}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="wide", choices=["mlp", "cnn", "wide", "gpt", "lstm"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--cpu-threads", type=int, default=None,
                    help="threads of the parallel CPU baseline (default min(B, cores, 16))")
    ap.add_argument("--predict", action="store_true",
                    help="time the inference path instead (Sequential.PredictBatch: forward in "
                         "inference mode on HBM-resident inputs, gn_model_predict_device)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB, 3 times (the "
                         "calibration kernel for the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the data-parallel "
              "sharding across GPUs is a design (DESIGN.md), not built here.", file=sys.stderr)
        sys.exit(2)

    if args.copy_probe:
        copy_probe(args.copy_probe)
        return

    import ctypes as C
    import goneuron_amd as gn
    from goneuron_amd import configs
    from goneuron_amd._lib import lib, check

    cfg = configs.CONFIGS[args.config]()
    B = cfg["B"]
    dev = gn.GetDefaultDevice()
    x, y = configs.inputs(cfg)
    workers = configs.gpu_workers(B)
    model = configs.build(cfg, device=dev, workers=workers)

    def dbuf(a):
        p = C.c_void_p()
        check(dev.h, lib().gn_malloc(dev.h, a.nbytes, C.byref(p)))
        check(dev.h, lib().gn_memcpy_h2d(dev.h, p, a.ctypes.data, a.nbytes))
        return p

    dx, dy = dbuf(x), dbuf(y)
    if args.predict:
        predict_bench(args, cfg, model, dev, dx, B, workers)
        check(dev.h, lib().gn_free(dev.h, dx))
        check(dev.h, lib().gn_free(dev.h, dy))
        model.Close()
        return
    step = lambda: check(dev.h, lib().gn_model_train_step_device(model.h, dx, dy, B))
    for _ in range(args.warmup):
        step()
    dev.sync()
    # timed region: K steps, no instrumentation -> value
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    dev.sync()
    elapsed = time.perf_counter() - t0
    # the same K steps again with a HIP event pair around every kernel launch
    # on the library's stream -> per-class kernel time for the roofline
    check(dev.h, lib().gn_timing_enable(dev.h, 1))
    dev.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    dev.sync()
    elapsed_ev = time.perf_counter() - t0
    res = {}

    def report(classes):
        for cls, name in classes:
            n = C.c_int64()
            ms = C.c_double()
            check(dev.h, lib().gn_timing_report(dev.h, cls, C.byref(n), C.byref(ms)))
            res[name] = (n.value, ms.value)

    report(((0, "gemm"), (1, "adam_overlapped"), (2, "other")))
    check(dev.h, lib().gn_timing_enable(dev.h, 0))
    # Adam alone: in a train step each layer's update runs on a second stream
    # while the backward pass continues; Network.Step's full-arena update
    # (gn_model_step, one launch on the main stream) times the kernel by itself.
    check(dev.h, lib().gn_timing_enable(dev.h, 1))
    dev.sync()
    for _ in range(args.steps):
        check(dev.h, lib().gn_model_step(model.h))
    dev.sync()
    report(((1, "adam"),))
    check(dev.h, lib().gn_timing_enable(dev.h, 0))
    loss = C.c_float()
    check(dev.h, lib().gn_model_read_loss(model.h, C.byref(loss)))

    K = args.steps
    samples_per_s = B * K / elapsed
    ms_per_step = elapsed * 1e3 / K
    flops = gemm_flops(cfg, B)
    g_n, g_ms = res["gemm"]
    a_n, a_ms = res["adam"]
    gemm_tflops = flops * K / (g_ms * 1e-3) / 1e12 if g_ms > 0 else None
    per_launch_flops = flops * K / g_n if g_n else None
    adam_bytes = 28 * model.nparams  # per launch of the full-arena update
    adam_gbps = adam_bytes * a_n / (a_ms * 1e-3) / 1e9 if a_ms > 0 else None
    ao_n, ao_ms = res["adam_overlapped"]

    line = {
        "metric": "train samples/s (fwd+bwd+Adam) on 1 MI355X; % of fp32 MFMA / HBM roofline",
        "value": samples_per_s,
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (reference LCG, seeds 1000+cfg / 2000+cfg), reference LCG weight init",
        "config": {"workload": cfg["name"], "batch": B, "workers": workers,
                   "layers": [d["kind"] + (f"{d['in']}->{d['out']}" if d["kind"] == "dense" else "")
                              for d in cfg["layers"]],
                   "loss": cfg["loss"], "optimizer": "Adam lr=1e-3"},
        "roofline": {"bound": "mfma", "achieved": gemm_tflops, "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": (gemm_tflops / PEAK_FP32_MFMA_TFLOPS) if gemm_tflops else None,
                     "traffic": (GEMM_TRAFFIC_BYTES_PER_STEP[cfg["name"]] * K / g_n
                                 if cfg["name"] in GEMM_TRAFFIC_BYTES_PER_STEP and g_n else None),
                     "kernel": "gemm_f32_mfma (all instantiations)",
                     "flops_per_launch": per_launch_flops,
                     "avg_launch_ms": g_ms / g_n if g_n else None},
        "kernels": {
            "gemm": {"launches_per_step": g_n / K, "ms_per_step": g_ms / K},
            "adam": {"launches": a_n, "ms_per_launch": a_ms / a_n if a_n else None,
                     "bound": "hbm", "achieved_gbps": adam_gbps, "peak_gbps": PEAK_HBM_GBPS,
                     "frac": adam_gbps / PEAK_HBM_GBPS if adam_gbps else None,
                     "bytes_per_launch": adam_bytes,
                     "measured": "full-arena update (gn_model_step) launched alone"},
            "adam_in_step": {"launches_per_step": ao_n / K, "ms_per_step": ao_ms / K,
                             "note": "per-layer updates on a second stream, overlapped with the "
                                     "backward pass; durations include the sharing"},
            "other": {"launches_per_step": res["other"][0] / K, "ms_per_step": res["other"][1] / K},
            "instrumented_ms_per_step": elapsed_ev * 1e3 / K,
        },
        "loss": loss.value,
    }
    # explicit, ordered teardown: input buffers, the model, then (atexit) the device
    check(dev.h, lib().gn_free(dev.h, dx))
    check(dev.h, lib().gn_free(dev.h, dy))
    model.Close()
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(cfg, x, y, args.cpu_budget, workers, args.cpu_threads)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
