"""bench.py's last stdout line is what the driver parses from a bounded tail of
stdout: it must stay under bench.MAX_LINE_BYTES with every per-kernel table of
five configurations in the results, and carry the contract's keys."""
import argparse
import json

import bench


def fake_result(name, nkernels=40, B=1024, with_cpu=True):
    kernels = {}
    for i in range(nkernels):
        kn = f"gemm_kernel_{i}" if i < 3 else f"some_long_kernel_name_{i}"
        kernels[kn] = {"launches_per_step": 5.0, "ms_per_step": 0.123456789 * (i + 1),
                       "us_per_launch": 24.69135780, "bound": "mfma" if i < 3 else "hbm",
                       "achieved": 123.456789, "unit": "TFLOP/s" if i < 3 else "GB/s",
                       "peak": 157.3 if i < 3 else 8000.0, "frac": 0.78485436,
                       "units_per_launch": 28791291904.0}
    bench.add_floors(kernels, 6.1234567)
    res = {"workload": name, "batch": B, "workers": 4, "params": 71222248,
           "value": 311220.123456789, "unit": "samples/s", "ms_per_step": 3.29023456789,
           "instrumented_ms_per_step": 3.4, "kernels_per_step": 37.0,
           "gemm": {"launches_per_step": 14.0, "ms_per_step": 3.19, "flops_per_step": 403.12e9,
                    "achieved_tflops": 123.9123456, "avg_launch_ms": 0.22812345},
           "dominant": bench.dominant(kernels), "kernels": kernels,
           "adam_alone": kernels["some_long_kernel_name_5"],
           "h2d_step": {"value": 260000.0, "unit": "samples/s", "ms_per_step": 3.9, "note": "x" * 120},
           "loss": 23.02585}
    if with_cpu:
        res["cpu_baseline"] = {"value": 214.3123, "unit": "samples/s", "cores": 16, "kind": "port",
                               "sample": "s" * 1000,
                               "single_thread": {"value": 16.7, "cores": 1, "sample": "t" * 200}}
    return res


def test_final_line_fits_and_has_contract_keys():
    args = argparse.Namespace(steps=20, warmup=5, config="wide")
    cfg = {"name": "wide", "loss": "crossentropy"}
    head = fake_result("wide")
    others = {n: fake_result(n) for n in ("mlp", "cnn", "gpt", "lstm")}
    host = {"cpu_model": "AMD EPYC " + "x" * 200, "nproc": 256, "affinity": 16, "cpu_share": 16}
    line = bench.final_line(args, cfg, head, others, host, 204.1e6)
    text = json.dumps(line, separators=(",", ":"))
    assert len(text) < bench.MAX_LINE_BYTES, len(text)
    back = json.loads(text)
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
              "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
              "roofline", "cpu_baseline"):
        assert k in back, k
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in back["roofline"], k
    for k in ("value", "unit", "cores", "kind", "sample"):
        assert k in back["cpu_baseline"], k
    assert back["config"]["workload"] == "wide"
    assert set(back["configs"]) == {"mlp", "cnn", "gpt", "lstm"}
    assert abs(back["roofline"]["frac"] - 123.9123456 / 157.3) < 1e-3


def test_final_line_without_gemms_uses_dominant_kernel():
    args = argparse.Namespace(steps=20, warmup=5, config="lstm")
    head = fake_result("lstm", with_cpu=False)
    head["gemm"] = {"launches_per_step": 0, "ms_per_step": 0, "flops_per_step": 0,
                    "achieved_tflops": None, "avg_launch_ms": None}
    line = bench.final_line(args, {"name": "lstm", "loss": "mse"}, head, {}, {}, None)
    assert line["roofline"]["kernel"] == head["dominant"]["kernel"]
    assert line["cpu_baseline"] is None
    assert len(json.dumps(line)) < bench.MAX_LINE_BYTES


def test_kernel_floor_is_the_longer_of_launch_and_work():
    """floor_us = max(empty-launch time, work at the bound's peak), floor_frac
    = floor_us / the kernel's time; no floors without a launch figure."""
    k = {"tiny": {"unit": "GB/s", "peak": 8000.0, "units_per_launch": 8e6, "us_per_launch": 10.0},
         "big": {"unit": "TFLOP/s", "peak": 157.3, "units_per_launch": 157.3e6 * 200, "us_per_launch": 250.0}}
    bench.add_floors(k, 6.0)
    assert k["tiny"]["floor_us"] == 6.0 and abs(k["tiny"]["floor_frac"] - 0.6) < 1e-12  # 1 us of bytes < launch
    assert abs(k["big"]["floor_us"] - 200.0) < 1e-9 and abs(k["big"]["floor_frac"] - 0.8) < 1e-12
    k2 = {"x": {"unit": "GB/s", "peak": 8000.0, "units_per_launch": 1.0, "us_per_launch": 5.0}}
    bench.add_floors(k2, None)
    assert "floor_us" not in k2["x"]
