"""Throughput of GoNeuron's fp32 training step (forward + backward + Adam) on
one MI355X, with the roofline fraction of every kernel and the CPU reference
path timed beside it.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config wide]

Prints ONE JSON line last (under 4 KB).  `value` is samples/s of the headline
workload (C3, the wide Dense stack, unless --config says otherwise) with inputs
resident in HBM.  The `configs` key holds a short summary of the other four
BASELINE configurations, so one run times all five; every configuration's
full per-kernel table goes to gpurun_out/bench_detail.json.  Per-kernel rooflines come from
HIP events the library records around each of its launches (on the stream the
launch goes to), divided into the launch's algorithmic work (bytes for
memory-bound kernels, FLOPs for matrix-core kernels) that the library states
per launch site.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3   # MI355X dense fp32 matrix (and vector) peak
PEAK_FP64_MFMA_TFLOPS = 78.6
PEAK_HBM_GBPS = 8000.0
# the CPU share of one GPU on the GPU boxes (their nproc shows the whole host)
CPU_SHARE = 16
# Network.TrainBatch goes parallel from 64 samples up (net.go:428-435)
PARALLEL_THRESHOLD = 64
# the driver keeps the tail of stdout; the final line stays well inside it
MAX_LINE_BYTES = 4096
MAX_CPU_REPS = 2000  # whole-batch passes of a CPU baseline sample
DETAIL_PATH = os.path.join(ROOT, "gpurun_out", "bench_detail.json")

# HBM bytes per GEMM launch of the C3 step, from the FETCH_SIZE / WRITE_SIZE
# rocprofv3 passes of this bench scaled by a copy kernel of known size
# (bench.py --calibrate-copy); read from the committed summary.
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "wide_gemm_adam_hbm_traffic.md")


def gemm_traffic_per_launch():
    """The `gemm_bytes_per_launch: N` line of the committed counter summary."""
    try:
        with open(TRAFFIC_PROFILE) as fh:
            for line in fh:
                m = re.match(r"\s*gemm_bytes_per_launch:\s*([0-9.eE+]+)", line)
                if m:
                    return float(m.group(1))
    except OSError:
        pass
    return None


def kernel_bound(name):
    """(bound, peak, unit) a kernel is judged against."""
    if name.startswith("gemm_") or name in ("attn_fwd", "attn_bwd", "conv_wgrad", "conv_dgrad"):
        return "mfma", PEAK_FP32_MFMA_TFLOPS, "TFLOP/s"
    if name == "lstm_gram":
        return "mfma_fp64", PEAK_FP64_MFMA_TFLOPS, "TFLOP/s"
    if name in ("conv_fwd", "lstm_fwd", "lstm_bptt", "gru_fwd", "gru_bwd"):
        # fp32 VALU / latency-bound recurrences: FLOP rate against the fp32 peak
        return "valu", PEAK_FP32_MFMA_TFLOPS, "TFLOP/s"
    return "hbm", PEAK_HBM_GBPS, "GB/s"


def kernel_table(lib, dev, K):
    """Per-kernel stats of the timed steps: launches and ms per step, achieved
    rate, fraction of the bound's peak."""
    import ctypes as C
    from goneuron_amd._lib import KernelStat, check
    cap = 256
    arr = (KernelStat * cap)()
    n = C.c_int32()
    check(dev.h, lib.gn_timing_kernels(dev.h, arr, cap, C.byref(n)))
    out = {}
    for i in range(min(n.value, cap)):
        st = arr[i]
        name = st.name.decode()
        bound, peak, unit = kernel_bound(name)
        scale = 1e12 if unit == "TFLOP/s" else 1e9
        ach = st.units / (st.ms * 1e-3) / scale if st.ms > 0 and st.units > 0 else None
        out[name] = {"launches_per_step": st.launches / K, "ms_per_step": st.ms / K,
                     "us_per_launch": 1e3 * st.ms / st.launches if st.launches else None,
                     "bound": bound, "achieved": ach, "unit": unit, "peak": peak,
                     "frac": ach / peak if ach else None,
                     "units_per_launch": st.units / st.launches if st.launches else None}
    return out


def add_floors(kernels, launch_us):
    """Each kernel against the shortest time it could take: the longer of an
    empty launch (launch_us, timed like the kernels) and its algorithmic bytes
    or FLOPs at the bound's peak.  floor_frac near 1: the kernel is at its
    floor (for the small kernels of C1, C2 and C4 the launch sets it)."""
    if not launch_us:
        return
    for k in kernels.values():
        scale = 1e12 if k["unit"] == "TFLOP/s" else 1e9
        work = (k.get("units_per_launch") or 0.0) / (k["peak"] * scale) * 1e6
        k["floor_us"] = max(launch_us, work)
        k["floor_frac"] = k["floor_us"] / k["us_per_launch"] if k.get("us_per_launch") else None


def host_info():
    model = None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count()
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity": aff, "cpu_share": CPU_SHARE}


def cpu_baseline(cfg, x, y, budget_s, threads):
    """The CPU oracle (C restatement of the reference's per-sample path) timed
    on the host, on a bounded sample, two ways:
      - parallel (the reported value): trainBatchParallel's structure
        (net.go:588-717) with T threads, each a private network (own layer
        state and gradient arena, as LightweightClone) running its own
        contiguous chunk; then the serial sum of the T gradient arenas and one
        Adam pass, per batch;
      - single thread: trainBatchSequential (net.go:721-784), the reported
        value for batches below 64 samples, which the reference never runs
        in parallel (net.go:428-435).
    samples/s = samples / (sample time + per-batch time * samples / B)."""
    import threading
    from oracle import refcpu
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from cfgutil import oracle_net
    refcpu.build()
    B = cfg["B"]
    T = threads
    nets = [oracle_net(refcpu, cfg) for _ in range(T if B >= PARALLEL_THRESHOLD else 1)]
    net = nets[0]
    # calibrate with one sample, then fill the budget
    t0 = time.perf_counter()
    net.accumulate_batch(x[:1], y[:1], 1)
    t1 = time.perf_counter() - t0
    n1 = int(max(1, min(B, budget_s / 2 / max(t1, 1e-6))))
    # a whole batch far shorter than the budget is repeated (r1 passes), so
    # the figure comes from about budget/2 seconds of work
    r1 = int(max(1, min(MAX_CPU_REPS, budget_s / 2 / max(t1 * n1, 1e-6)))) if n1 == B else 1
    net.step()  # first touch of the Adam moments, untimed
    t0 = time.perf_counter()
    for _ in range(r1):
        net.accumulate_batch(x[:n1], y[:n1], n1)
        net.step()
    ts1 = time.perf_counter() - t0
    t0 = time.perf_counter()
    net.step()
    ta = time.perf_counter() - t0
    if r1 > 1:  # whole batches, each with its Adam pass
        single = r1 * n1 / ts1
        single_desc = f"{r1} passes over the {B}-sample batch, fwd+bwd+Adam ({ts1:.2f} s)"
    else:
        single = n1 / (ts1 + ta * n1 / B)
        single_desc = f"{n1} of {B} samples fwd+bwd ({ts1:.2f} s) + Adam scaled by n/B"
    # parallel: every thread takes npt samples of its own chunk of the batch
    chunk = (B + T - 1) // T
    npt = int(max(1, min(chunk, budget_s / 2 / max(t1, 1e-6))))
    rp = int(max(1, min(MAX_CPU_REPS, budget_s / 2 / max(t1 * npt, 1e-6)))) if npt == chunk else 1

    def work(t, n):
        s0 = min(t * chunk, B - n)
        nets[t].accumulate_batch(x[s0:s0 + n], y[s0:s0 + n], n)

    def run_all(n):
        th = [threading.Thread(target=work, args=(t, n)) for t in range(T)]
        for h in th:
            h.start()
        for h in th:
            h.join()

    if B < PARALLEL_THRESHOLD:
        # the reference trains batches below 64 samples sequentially on one
        # goroutine (Network.TrainBatch, net.go:428-435): the 1-thread figure
        # is the baseline
        del nets
        return {"value": single, "unit": "samples/s", "cores": 1, "kind": "port",
                "sample": f"oracle/refcpu (C restatement, -O2 -ffp-contract=off), trainBatchSequential "
                          f"(B = {B} < 64): {single_desc}"}
    run_all(1)  # first touch of every worker's buffers, untimed
    acc = np.zeros_like(net.grads)
    acc += 1.0
    t0 = time.perf_counter()
    for _ in range(rp):
        run_all(npt)
    tp = time.perf_counter() - t0
    t0 = time.perf_counter()  # serial sum of the worker arenas (net.go:694-700)
    acc[:] = 0.0
    for nt in nets:
        acc += nt.grads
    tsum = time.perf_counter() - t0
    done = rp * T * npt
    par = done / (tp + (tsum + ta) * done / B)
    del nets
    return {"value": par, "unit": "samples/s", "cores": T, "kind": "port",
            "sample": f"oracle/refcpu (C restatement, -O2 -ffp-contract=off), trainBatchParallel shape: "
                      f"{rp} x {T} threads x {npt} samples of their own chunks of the {B}-sample batch "
                      f"({tp:.2f} s) + per batch the sum of {T} gradient arenas ({tsum:.3f} s) and one "
                      f"Adam pass ({ta:.3f} s) scaled by samples/B",
            "single_thread": {"value": single, "cores": 1, "sample": single_desc}}


def dominant(kernels):
    """The roofline entry of the kernel with the most time per step."""
    if not kernels:
        return None
    name, k = max(kernels.items(), key=lambda kv: kv[1]["ms_per_step"])
    return {"kernel": name, "bound": k["bound"], "achieved": k["achieved"], "peak": k["peak"],
            "unit": k["unit"], "frac": k["frac"], "ms_per_step": k["ms_per_step"],
            "floor_frac": k.get("floor_frac")}


def run_config(name, args, dev, with_cpu, cpu_budget, threads):
    """One configuration: plain timed steps (value), the same steps with the
    library's per-launch events (kernel table), Adam alone, the host-pointer
    step (H2D included), and the CPU baseline."""
    import ctypes as C
    from goneuron_amd import configs
    from goneuron_amd._lib import lib, check
    L = lib()
    cfg = configs.get(name)
    B = cfg["B"]
    x, y = configs.inputs(cfg)
    workers = configs.gpu_workers(B)
    model = configs.build(cfg, device=dev, workers=workers)

    def dbuf(a):
        p = C.c_void_p()
        check(dev.h, L.gn_malloc(dev.h, a.nbytes, C.byref(p)))
        check(dev.h, L.gn_memcpy_h2d(dev.h, p, a.ctypes.data, a.nbytes))
        return p

    dx, dy = dbuf(x), dbuf(y)
    K = args.steps
    step = lambda: check(dev.h, L.gn_model_train_step_device(model.h, dx, dy, B))
    for _ in range(args.warmup):
        step()
    dev.sync()
    # timed region: K steps, no instrumentation -> value
    t0 = time.perf_counter()
    for _ in range(K):
        step()
    dev.sync()
    elapsed = time.perf_counter() - t0
    # the same K steps with a HIP event pair around every launch -> kernel table
    check(dev.h, L.gn_timing_enable(dev.h, 1))
    t0 = time.perf_counter()
    for _ in range(K):
        step()
    dev.sync()
    elapsed_ev = time.perf_counter() - t0
    kernels = kernel_table(L, dev, K)
    check(dev.h, L.gn_timing_enable(dev.h, 0))
    # Adam alone: Network.Step's full-arena update (gn_model_step), K launches
    check(dev.h, L.gn_timing_enable(dev.h, 1))
    for _ in range(K):
        check(dev.h, L.gn_model_step(model.h))
    dev.sync()
    adam = kernel_table(L, dev, K).get("adam")
    check(dev.h, L.gn_timing_enable(dev.h, 0))
    # the launch floor, timed the same way: K empty 256-block launches
    check(dev.h, L.gn_timing_enable(dev.h, 1))
    check(dev.h, L.gn_timing_floor(dev.h, 256, K))
    dev.sync()
    floor = kernel_table(L, dev, K).get("floor") or {}
    check(dev.h, L.gn_timing_enable(dev.h, 0))
    add_floors(kernels, floor.get("us_per_launch"))
    loss = C.c_float()
    check(dev.h, L.gn_model_read_loss(model.h, C.byref(loss)))
    # end to end from host buffers: the step copies x and y over PCIe first
    xh, yh = np.ascontiguousarray(x), np.ascontiguousarray(y)
    fp = lambda a: a.ctypes.data_as(C.POINTER(C.c_float))
    hstep = lambda: check(dev.h, L.gn_model_train_step(model.h, fp(xh), fp(yh), B, None))
    hstep()
    t0 = time.perf_counter()
    for _ in range(K):
        hstep()
    dev.sync()
    elapsed_h = time.perf_counter() - t0
    # explicit, ordered teardown: input buffers, then the model
    check(dev.h, L.gn_free(dev.h, dx))
    check(dev.h, L.gn_free(dev.h, dy))
    nparams = model.nparams
    model.Close()
    gemm = {k: v for k, v in kernels.items() if k.startswith("gemm_")}
    g_ms = sum(v["ms_per_step"] for v in gemm.values()) * K
    g_n = sum(v["launches_per_step"] for v in gemm.values()) * K
    g_units = sum(v["units_per_launch"] * v["launches_per_step"] for v in gemm.values()) * K
    res = {
        "workload": name, "batch": B, "workers": workers, "params": nparams,
        "value": B * K / elapsed, "unit": "samples/s", "ms_per_step": elapsed * 1e3 / K,
        "instrumented_ms_per_step": elapsed_ev * 1e3 / K,
        "kernels_per_step": sum(v["launches_per_step"] for v in kernels.values()),
        "gemm": {"launches_per_step": g_n / K, "ms_per_step": g_ms / K,
                 "flops_per_step": g_units / K,
                 "achieved_tflops": g_units / (g_ms * 1e-3) / 1e12 if g_ms > 0 else None,
                 "avg_launch_ms": g_ms / g_n if g_n else None},
        "dominant": dominant(kernels),
        "kernels": kernels,
        "adam_alone": adam,
        "launch_floor_us": floor.get("us_per_launch"),
        "h2d_step": {"value": B * K / elapsed_h, "unit": "samples/s", "ms_per_step": elapsed_h * 1e3 / K,
                     "note": "gn_model_train_step from host buffers: H2D copy of x and y inside "
                             "every step (never `value`)"},
        "loss": loss.value,
    }
    if with_cpu:
        res["cpu_baseline"] = cpu_baseline(cfg, x, y, cpu_budget, min(B, threads))
    return res


def predict_bench(args, dev):
    """Inference throughput (f3): K forward passes in inference mode over the
    config's batch, inputs and outputs in HBM."""
    import ctypes as C
    from goneuron_amd import configs
    from goneuron_amd._lib import lib, check
    L = lib()
    cfg = configs.get(args.config)
    B = cfg["B"]
    x, _ = configs.inputs(cfg)
    model = configs.build(cfg, device=dev)
    dx, out = C.c_void_p(), C.c_void_p()
    check(dev.h, L.gn_malloc(dev.h, x.nbytes, C.byref(dx)))
    check(dev.h, L.gn_memcpy_h2d(dev.h, dx, x.ctypes.data, x.nbytes))
    check(dev.h, L.gn_malloc(dev.h, B * model.out_size * 4, C.byref(out)))
    run = lambda: check(dev.h, L.gn_model_predict_device(model.h, dx, B, out))
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
    check(dev.h, L.gn_free(dev.h, dx))
    check(dev.h, L.gn_free(dev.h, out))
    model.Close()


def calibrate_copy(mib):
    """A copy kernel of known size (reads and writes mib MiB per launch, 3
    launches): the FETCH_SIZE / WRITE_SIZE counters of the traffic passes are
    scaled by what they read for it."""
    import torch
    n = mib * (1 << 20) // 4
    a = torch.ones(n, device="cuda:0")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": n * 4}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 200 steps: the small configurations' steps (tens of us) are then timed
    # in steady state; at 20 the host's launch rate, not the GPU, set them
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="wide",
                    choices=["mlp", "cnn", "wide", "gpt", "lstm", "gru", "cnn2", "gpt_long"],
                    help="headline workload (the `value` of the line); gru, cnn2 and gpt_long are not "
                         "BASELINE configs")
    ap.add_argument("--only", action="store_true", help="time the headline workload only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--cpu-budget", type=float, default=20.0,
                    help="seconds of CPU work per configuration's baseline (half single-thread, "
                         "half the threaded run)")
    ap.add_argument("--predict", action="store_true",
                    help="time the inference path instead (Sequential.PredictBatch: forward in "
                         "inference mode on HBM-resident inputs, gn_model_predict_device)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB, 3 times (the "
                         "calibration kernel for the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the data-parallel "
              "sharding across GPUs is a design (DESIGN.md), not built here.", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy(args.calibrate_copy)
        return

    import goneuron_amd as gn
    from goneuron_amd import configs
    dev = gn.GetDefaultDevice()
    if args.predict:
        predict_bench(args, dev)
        return
    host = host_info()
    threads = max(1, min(host["affinity"] or 1, CPU_SHARE))
    head = run_config(args.config, args, dev, not args.no_cpu, args.cpu_budget, threads)
    print(f"bench: {args.config} {head['value']:.0f} samples/s", file=sys.stderr, flush=True)
    others = {}
    if not args.only:
        for name in ("mlp", "cnn", "wide", "gpt", "lstm"):
            if name != args.config:
                others[name] = run_config(name, args, dev, not args.no_cpu, args.cpu_budget, threads)
                print(f"bench: {name} {others[name]['value']:.0f} samples/s", file=sys.stderr, flush=True)
    cfg = configs.get(args.config)
    traffic = gemm_traffic_per_launch() if args.config == "wide" else None
    write_detail({"host": dict(host, threads_used=min(head["batch"], threads)),
                  "headline": head, "configs": others})
    line = final_line(args, cfg, head, others, host, traffic)
    text = json.dumps(line, separators=(",", ":"))
    if len(text) > MAX_LINE_BYTES:  # never expected: drop the per-config map first
        line.pop("configs", None)
        text = json.dumps(line, separators=(",", ":"))
    print(text, flush=True)


def _r(v, nd=4):
    """A float rounded to nd significant digits (None passes through)."""
    if v is None:
        return None
    return float(f"{v:.{nd}g}")


def summarize(res):
    """What the final line keeps of one configuration: throughput, the
    dominant kernel's roofline fraction and the CPU baseline's value."""
    d = res.get("dominant") or {}
    cb = res.get("cpu_baseline") or {}
    return {"value": _r(res["value"]), "ms_per_step": _r(res["ms_per_step"]),
            "batch": res["batch"], "workers": res["workers"],
            "kernels_per_step": _r(res.get("kernels_per_step"), 3),
            "dominant": d.get("kernel"), "dominant_bound": d.get("bound"),
            "dominant_frac": _r(d.get("frac"), 3),
            "dominant_floor_frac": _r(d.get("floor_frac"), 3),
            "cpu_baseline": _r(cb.get("value")), "cpu_cores": cb.get("cores")}


def final_line(args, cfg, head, others, host, traffic):
    """The one JSON line the driver parses, kept under MAX_LINE_BYTES: the
    headline workload's value, roofline and CPU baseline, plus a short entry
    per other configuration.  Full per-kernel tables go to DETAIL_PATH."""
    g = head["gemm"]
    if g["launches_per_step"] and g["achieved_tflops"]:
        # GEMM family of the step: every launch of the fp32 MFMA GEMM kernels
        roof = {"bound": "mfma", "achieved": _r(g["achieved_tflops"]), "peak": PEAK_FP32_MFMA_TFLOPS,
                "unit": "TFLOP/s", "frac": _r(g["achieved_tflops"] / PEAK_FP32_MFMA_TFLOPS),
                "traffic": traffic,
                "kernel": "gemm_f32_mfma (gemm_fwd, gemm_dx, gemm_dw)",
                "flops_per_launch": _r(g["flops_per_step"] / g["launches_per_step"]),
                "avg_launch_ms": _r(g["avg_launch_ms"]),
                "launches_per_step": g["launches_per_step"]}
    else:
        d = head.get("dominant") or {}
        roof = {"bound": "hbm" if d.get("bound") == "hbm" else "mfma", "achieved": _r(d.get("achieved")),
                "peak": d.get("peak"), "unit": d.get("unit"), "frac": _r(d.get("frac")),
                "traffic": None, "kernel": d.get("kernel")}
    cb = head.get("cpu_baseline")
    if cb is not None:
        cb = {"value": _r(cb["value"]), "unit": cb["unit"], "cores": cb["cores"], "kind": cb["kind"],
              "sample": cb["sample"][:300],
              "single_thread": _r((cb.get("single_thread") or {}).get("value", cb["value"]))}
    adam = head.get("adam_alone") or {}
    return {
        "metric": "train samples/s (fwd+bwd+Adam) on 1 MI355X; % of fp32 MFMA / HBM roofline",
        "value": _r(head["value"], 6),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": _r(head["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (reference LCG inputs, seeds 1000+cfg / 2000+cfg; reference LCG weight init)",
        "config": {"workload": cfg["name"], "batch": head["batch"], "workers": head["workers"],
                   "params": head["params"], "loss": cfg["loss"], "optimizer": "Adam lr=1e-3"},
        "roofline": roof,
        "adam": {"achieved": _r(adam.get("achieved")), "unit": "GB/s", "peak": PEAK_HBM_GBPS,
                 "frac": _r(adam.get("frac"))},
        "h2d_ms_per_step": _r(head["h2d_step"]["ms_per_step"]),
        "cpu_baseline": cb,
        "host": {"cpu_model": (host.get("cpu_model") or "")[:60], "threads": min(head["batch"], CPU_SHARE,
                                                                                 host.get("affinity") or 1)},
        "configs": {k: summarize(v) for k, v in others.items()},
        "detail": os.path.relpath(DETAIL_PATH, ROOT),
    }


def write_detail(obj):
    """Full per-kernel tables of every configuration (not part of the line)."""
    try:
        os.makedirs(os.path.dirname(DETAIL_PATH), exist_ok=True)
        with open(DETAIL_PATH, "w") as fh:
            json.dump(obj, fh, indent=1)
    except OSError as e:
        print(f"bench: could not write {DETAIL_PATH}: {e}", file=sys.stderr, flush=True)


if __name__ == "__main__":
    main()
