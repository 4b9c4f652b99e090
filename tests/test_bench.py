"""bench.py's driver contract: the multi-GPU refusal and the byte accounting (CPU), the CPU
baseline's fields (CPU, a tiny time budget), and one short GPU run whose JSON line carries every
field the driver reads (GPU)."""

import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_algorithmic_bytes():
    # north star: M N (2 + 1/2 + 4/64) + 2 M r + 2 N r
    M, N, r = 16384, 4096, 16
    assert bench.algorithmic_bytes(M, N, r, 4, 64) == M * N * (2 + 0.5 + 4 / 64) + 2 * M * r + 2 * N * r
    assert abs(bench.algorithmic_bytes(M, N, r, 4, 64) / 1e6 - 172.62) < 0.01
    # fused consumer: codes + qparams + dY read, dX written, L, V
    assert bench.consumer_bytes(M, N, r, 4, 64) == M * N * (0.5 + 4 / 64 + 4) + 2 * M * r + 2 * N * r


@pytest.mark.parametrize("config", ["north_star", "c3", "lora", "legacy", "ref_enc", "ref_dec"])
def test_cpu_baseline_fields(config):
    """The CPU baseline is the torch-eager restatement on every core the process may use, with
    the host recorded (a tiny time budget here)."""
    import importlib
    import os

    import torch
    pkg = importlib.import_module("triton-kernel-test_amd")
    threads = torch.get_num_threads()
    try:
        cb = bench.cpu_baseline(pkg.inputs.CONFIGS[config], 0.05)
    finally:
        torch.set_num_threads(threads)
    assert cb["kind"] == "port" and cb["unit"] == "GB/s" and cb["value"] > 0
    assert cb["cores"] == len(os.sched_getaffinity(0))
    assert "rows" in cb["sample"] and "median of 3" in cb["sample"]
    assert cb["cpu"] and cb["torch"] == torch.__version__


@pytest.mark.gpu
def test_bench_line_on_gpu():
    r = subprocess.run([sys.executable, "-u", str(ROOT / "bench.py"), "--steps", "5", "--warmup", "1",
                        "--settle-seconds", "0", "--no-cpu-baseline"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    line = json.loads([x for x in r.stdout.splitlines() if x.startswith("{")][-1])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline"):
        assert k in line, k
    assert line["n_gpus"] == 1 and line["steps"] == 5 and line["warmup"] == 1 and line["value"] > 0
    rf = line["roofline"]
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and 0 < rf["frac"] < 1.2
    assert "workload" in line["config"]
