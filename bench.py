#!/usr/bin/env python3
"""Benchmark of the compressed-activation hot path on one MI355X.

Default workload (BASELINE.json metric): rank-16 int4/g64 encode + decode of a bf16
[16384, 4096] activation ("north_star").  One step = encode(X_i) then decode; inputs
rotate over several HBM-resident buffer sets (> 512 MB of X) so the 256 MB MALL cannot
serve them.  Prints ONE JSON line (driver contract).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config north_star|c1|c2|c3|c4|c5]
                  [--no-cpu-baseline]

value       = activation GB/s = 2*rows*hidden bytes / (encode + decode time per step)
roofline    = dominant kernel's algorithmic HBM bytes per launch / its mean duration
              (HIP events on the launch stream), against 8 TB/s
cpu_baseline= the CPU oracle (numpy, 1 thread) on a bounded row sample of the same workload
"""

from __future__ import annotations

import argparse
import ctypes
import importlib
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_DENSE_TFLOPS = 2500.0
METRIC = "encode+decode activation GB/s and % of HBM peak (bf16 4096-hidden, rank-16 int4)"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="north_star")
    ap.add_argument("--nbuf", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    return ap.parse_args()


def algorithmic_bytes(rows, hidden, rank, bits, group, n_side=0):
    """Encode bytes = M N (2 + b/8 + 4/G) + 2 M r + 2 N r (+ 2 M k side columns); decode is
    the same traffic with reads and writes swapped."""
    b = rows * hidden * (2 + bits / 8 + 4 / group) + 2 * rows * rank + 2 * hidden * rank
    return b + 2 * rows * n_side


def traffic_from_profiles(name: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if present."""
    p = ROOT / "profiles" / f"traffic_{name}.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text())
    except Exception:
        return None


def cpu_baseline(cfg, seconds: float):
    """Time the numpy oracle's encode+decode on a row sample sized to ~`seconds` of work."""
    import numpy as np
    try:
        from threadpoolctl import threadpool_limits
    except Exception:  # pragma: no cover
        threadpool_limits = None
    import oracle as O
    pkg = importlib.import_module("triton-kernel-test_amd")
    ctx = threadpool_limits(1) if threadpool_limits else None
    try:
        rows = 64
        V = pkg.inputs.basis(cfg.hidden, cfg.rank, cfg.seed) if cfg.rank else None
        vb = V.view(__import__("torch").int16).numpy().view(np.uint16) if V is not None else None

        def run(r):
            x = pkg.inputs.activation(r, cfg.hidden, cfg.n_outlier, cfg.outlier_scale, cfg.seed)
            xb = x.view(__import__("torch").int16).numpy().view(np.uint16)
            t0 = time.perf_counter()
            e = O.encode(xb, vb, cfg.bits, cfg.group)
            O.decode(e["L"], vb, e["codes"], e["scale"], e["zero"], cfg.bits, cfg.group)
            return time.perf_counter() - t0

        t = run(rows)
        while t < seconds / 8 and rows < cfg.rows:
            rows = min(cfg.rows, rows * 2)
            t = run(rows)
        if t < seconds and rows < cfg.rows:
            rows = min(cfg.rows, max(rows, int(rows * seconds / max(t, 1e-3))))
            t = run(rows)
        gbs = 2 * rows * cfg.hidden / t / 1e9
        return {"value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"numpy oracle encode+decode of {rows} of {cfg.rows} rows x {cfg.hidden} "
                          f"(same recipe), {t:.1f} s, 1 thread"}
    finally:
        if ctx is not None:
            ctx.__exit__(None, None, None)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU runs are not part of it",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    pkg = importlib.import_module("triton-kernel-test_amd")
    from importlib import import_module
    lib_mod = import_module("triton-kernel-test_amd._lib")
    lib = lib_mod.load()
    cfg = pkg.inputs.CONFIGS[args.config]
    if cfg.consumer != "decode" or cfg.hadamard or cfg.keep_channels:
        raise SystemExit(f"config {args.config} is not benchmarked by this script yet")
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    # ---- inputs: nbuf HBM-resident sets (device RNG: same recipe, fast)
    V = pkg.inputs.basis(cfg.hidden, cfg.rank, cfg.seed).to(dev)
    basis = pkg.LowRankBasis(V)
    _ = basis.Vt
    xs, comps, outs = [], [], []
    for i in range(args.nbuf):
        x = pkg.inputs.activation(cfg.rows, cfg.hidden, cfg.n_outlier, cfg.outlier_scale, cfg.seed + i, dev)
        xs.append(x)
        comps.append(pkg.encode(x, basis, bits=cfg.bits, group_size=cfg.group))
        outs.append(torch.empty_like(x))
    torch.cuda.synchronize()
    descs = [c.descriptor(for_encode=True) for c in comps]
    stream = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(stream.cuda_stream)
    enc, dec = lib.lrq_encode, lib.lrq_decode

    def step(i, ev=None):
        k = i % args.nbuf
        d = ctypes.byref(descs[k])
        if ev is not None:
            ev[0].record(stream)
        st = enc(d, ctypes.c_void_p(xs[k].data_ptr()), cfg.hidden, sp)
        if ev is not None:
            ev[1].record(stream)
        st |= dec(d, ctypes.c_void_p(outs[k].data_ptr()), cfg.hidden, sp)
        if ev is not None:
            ev[2].record(stream)
        if st:
            raise RuntimeError(f"launch failed: {lib_mod.status_string(st)}")

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # ---- timed region: K steps, per-kernel HIP events on the launch stream
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for i in range(args.steps):
        step(i, evs[i])
    t_end.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    ms_step = total_ms / args.steps
    enc_ms = [e[0].elapsed_time(e[1]) for e in evs]
    dec_ms = [e[1].elapsed_time(e[2]) for e in evs]
    enc_mean, dec_mean = statistics.mean(enc_ms), statistics.mean(dec_ms)
    enc_med, dec_med = statistics.median(enc_ms), statistics.median(dec_ms)

    act_bytes = 2 * cfg.rows * cfg.hidden
    alg = algorithmic_bytes(cfg.rows, cfg.hidden, cfg.rank, cfg.bits, cfg.group)
    value = act_bytes / (ms_step * 1e-3) / 1e9
    dominant = "encode" if enc_mean >= dec_mean else "decode"
    dom_ms = max(enc_mean, dec_mean)
    achieved = alg / (dom_ms * 1e-3) / 1e9
    traffic = traffic_from_profiles(f"{dominant}_{args.config}")
    # MFMA work: encode = projection (2 M N r) + residual (2 M N r); decode = 2 M N r
    enc_tf = 4 * cfg.rows * cfg.hidden * cfg.rank / (enc_mean * 1e-3) / 1e12
    dec_tf = 2 * cfg.rows * cfg.hidden * cfg.rank / (dec_mean * 1e-3) / 1e12

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) with scaled outlier channels; orthonormal QR basis)",
        "config": {"workload": f"{args.config}: encode+decode", "rows": cfg.rows, "hidden": cfg.hidden,
                   "rank": cfg.rank, "bits": cfg.bits, "group": cfg.group, "buffers": args.nbuf},
        "hbm_frac_step": round(2 * alg / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "kernels": {
            "encode": {"mean_us": round(enc_mean * 1e3, 2), "median_us": round(enc_med * 1e3, 2),
                       "alg_GBs": round(alg / (enc_mean * 1e-3) / 1e9, 1),
                       "mfma_tflops": round(enc_tf, 2), "mfma_util": round(enc_tf / BF16_DENSE_TFLOPS, 5)},
            "decode": {"mean_us": round(dec_mean * 1e3, 2), "median_us": round(dec_med * 1e3, 2),
                       "alg_GBs": round(alg / (dec_mean * 1e-3) / 1e9, 1),
                       "mfma_tflops": round(dec_tf, 2), "mfma_util": round(dec_tf / BF16_DENSE_TFLOPS, 5)},
        },
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": (traffic or {}).get("bytes_per_launch")},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
