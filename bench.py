#!/usr/bin/env python3
"""Benchmark of the compressed-activation hot path on one MI355X.

Default workload (BASELINE.json metric): rank-16 int4/g64 encode + decode of a bf16
[16384, 4096] activation ("north_star").  One step = encode(X_i) then decode; inputs
rotate over several HBM-resident buffer sets (> 512 MB of X) so the 256 MB MALL cannot
serve them.  Prints ONE JSON line (driver contract).

  python bench.py [--gpus 1] [--steps K] [--warmup W]
                  [--config north_star|c1|c2|c3|c4|c4l|c4s|c5|c5w|lora|legacy|ref_enc|ref_dec|ref_mm|offload|copy]
                  [--m M]
                  [--no-cpu-baseline]

value       = activation GB/s = 2*rows*hidden bytes / (encode + decode time per step);
              fused-consumer configs: / (consumer time); lora: / (x A + x^T g time);
              legacy: / (encode with its outlier compaction + decode time); ref_enc / ref_dec
              (the reference's own speed tests, x [4, M, M]): / (1-bit encode + compaction) and
              / (2-bit decode from COO); ref_mm (the reference's fused dequant-matmul bench,
              x [4, M, M] @ y [4, M, 32]): / (the fused legacy dequant-GEMM)
timing      = exactly --warmup untimed steps, then exactly --steps timed steps between two HIP
              events on the launch stream (synchronised before and after); `settled` repeats
              the timed steps after --settle-seconds of sustained work, as a separate field
cold_*      = the step's last kernel (decode / consumer) timed alone with its inputs HBM-cold:
              a 1 GiB fill before each launch evicts the L2s and the 256 MB MALL
roofline    = dominant kernel's algorithmic HBM bytes per launch / its mean duration
              (K back-to-back launches between HIP events on the launch stream, the queue
              pre-filled so host launch cost is not timed), against 8 TB/s; traffic =
              rocprofv3 FETCH_SIZE/WRITE_SIZE bytes per launch from profiles/
mfma        = MFMA utilisation of the projection / GEMM kernels from rocprofv3 counters
              (SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE) in profiles/, where measured
cpu_baseline= PyTorch-eager fp32 restatement (oracle/lrq_torch.py) on all host cores,
              1 warm-up + median of 3, on a bounded row sample of the same workload
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
MM_COLS = 32  # ref_mm: columns of y (the reference bench's R = 32, extraction_fuse_matmul.py:427)
METRIC = "encode+decode activation GB/s and % of HBM peak (bf16 4096-hidden, rank-16 int4)"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=20)
    # after the headline measurement: this much sustained work, then the K steps again,
    # reported as `settled` (the GPU's clocks settle over about a second of sustained work)
    ap.add_argument("--settle-seconds", type=float, default=2.0)
    ap.add_argument("--config", default="north_star")
    ap.add_argument("--m", type=int, default=0, help="ref_enc / ref_dec / ref_mm: M of x [4, M, M] (the reference's sweep)")
    ap.add_argument("--nbuf", type=int, default=4)
    ap.add_argument("--cold-steps", type=int, default=20, help="timed launches of the last kernel with HBM-cold inputs")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--lora-split", action="store_true",
                    help="lora: time x A and x^T g as the two separate kernels instead of the one-pass entry")
    ap.add_argument("--cpu-seconds", type=float, default=3.0, help="target seconds per CPU baseline run")
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


def mfma_from_profiles(config: str):
    """MFMA utilisation per kernel from the committed rocprofv3 counter summary, if present."""
    p = ROOT / "profiles" / f"mfma_{config}.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text())
    except Exception:
        return None


def cpu_baseline(cfg, seconds: float):
    """Time the PyTorch-eager fp32 restatement (oracle/lrq_torch.py) on the host's cores, on
    a row sample of the same workload sized to about `seconds` per run: encode + decode for
    the round-trip configs, decode + consumer for the fused ones (the encode is their
    producer and is not timed), decode + x A + x^T g for lora, the reference's torch
    encode + to_sparse + decode for legacy.  1 warm-up run, then the median of 3."""
    import platform

    import torch
    from oracle import lrq_torch as T
    pkg = importlib.import_module("triton-kernel-test_amd")
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cpu = platform.processor() or "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    V = pkg.inputs.basis(cfg.hidden, cfg.rank, cfg.seed) if cfg.rank else None

    def prepare(r):
        if cfg.consumer in ("ref_enc", "ref_dec", "ref_mm"):
            ops = pkg.inputs.ref_operands(cfg)
            g = torch.Generator().manual_seed(cfg.seed)
            d = dict(l=ops["l"][:r], r=ops["r"], s=ops["s"][:1])
            if cfg.consumer == "ref_mm":
                d["q"] = torch.randint(0, 256, (1, r, cfg.hidden * cfg.bits // 8), generator=g, dtype=torch.uint8)
                d["y"] = torch.randn((1, cfg.hidden, MM_COLS), generator=g).to(torch.bfloat16)
            elif cfg.consumer == "ref_enc":
                d["x"] = torch.randn((1, r, cfg.hidden), generator=g).to(torch.bfloat16)
            else:
                d["q"] = torch.randint(0, 256, (1, r, cfg.hidden * cfg.bits // 8), generator=g, dtype=torch.uint8)
                o = torch.randn((1, r, cfg.hidden), generator=g).to(torch.bfloat16)
                d["o"] = (o * (o > 1)).to_sparse()
            return d
        if cfg.consumer == "legacy":
            ops = pkg.inputs.legacy_operands(cfg)
            x = pkg.inputs.activation(r, cfg.hidden, cfg.n_outlier, cfg.outlier_scale, cfg.seed)[None]
            l = ops["l"][:r]
            tau = float(torch.kthvalue((x[0] - l @ ops["r"]).flatten().abs().float(), int(x[0].numel() * 0.99)).values)
            return dict(x=x, l=l, r=ops["r"], s=ops["s"], tau=tau)
        inp = pkg.inputs.make(cfg, rows=r)
        if cfg.keep_channels:
            inp["idx"] = torch.sort(torch.topk(inp["x"].float().abs().amax(0), cfg.keep_channels).indices).values
        if cfg.consumer != "decode":
            inp["enc"] = T.encode(inp["x"], V, cfg.bits, cfg.group, cfg.hadamard, inp.get("idx"))
        return inp

    def run(inp):
        t0 = time.perf_counter()
        if cfg.consumer == "ref_enc":
            o, q = T.legacy_encode(inp["l"], inp["r"], inp["x"], inp["s"], cfg.bits, cfg.tau)
            T.to_coo(o)
        elif cfg.consumer == "ref_dec":
            T.legacy_decode(inp["l"], inp["r"], inp["q"], inp["o"].to_dense(), inp["s"], cfg.bits)
        elif cfg.consumer == "ref_mm":
            xh = T.legacy_decode(inp["l"], inp["r"], inp["q"], None, inp["s"], cfg.bits)
            torch.matmul(xh.float(), inp["y"].float()).to(torch.bfloat16)
        elif cfg.consumer == "legacy":
            o, q = T.legacy_encode(inp["l"], inp["r"], inp["x"], inp["s"], cfg.bits, inp["tau"])
            o = T.to_coo(o)
            T.legacy_decode(inp["l"], inp["r"], q, o.to_dense(), inp["s"], cfg.bits)
        elif cfg.consumer == "decode":
            e = T.encode(inp["x"], V, cfg.bits, cfg.group, cfg.hadamard, inp.get("idx"))
            T.decode(e, V, cfg.bits, cfg.group, cfg.hadamard)
        else:
            xh = T.decode(inp["enc"], V, cfg.bits, cfg.group, cfg.hadamard)
            if cfg.consumer == "lora":
                xf = xh.float()
                (xf @ inp["a"].float()).bfloat16()
                xf.T @ inp["g"].float()
            else:
                {"silu": T.silu_bwd, "gelu": T.gelu_bwd, "softmax": T.softmax_bwd}[cfg.consumer](xh, inp["dy"])
        return time.perf_counter() - t0

    limit = cfg.hidden if cfg.consumer in ("ref_enc", "ref_dec", "ref_mm") else cfg.rows  # (one batch of x [B, M, M])
    rows = min(limit, 256)
    inp = prepare(rows)
    t = run(inp)
    while t < seconds / 4 and rows < limit:
        rows = min(limit, rows * 4)
        inp = prepare(rows)
        t = run(inp)
    if t < 0.7 * seconds and rows < limit:
        rows = min(limit, max(rows, int(rows * seconds / max(t, 1e-3))))
        inp = prepare(rows)
        run(inp)  # warm-up at the final size
    times = [run(inp) for _ in range(3)]
    t = statistics.median(times)
    gbs = 2 * rows * cfg.hidden / t / 1e9
    what = {"decode": "encode+decode", "lora": "decode + x A + x^T g (LoRA factor gradients)",
            "legacy": "reference torch encode + to_sparse + decode",
            "ref_enc": "reference torch encode + to_sparse (one batch's rows of x [B, M, M])",
            "ref_dec": "reference to_dense + torch decode (one batch's rows of x [B, M, M])",
            "ref_mm": "reference torch decode + matmul with y [M, 32] (one batch's rows of x [B, M, M])"}.get(
                cfg.consumer, f"decode+{cfg.consumer} backward")
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"PyTorch-eager fp32 {what} (oracle/lrq_torch.py) of {rows} of {cfg.rows} rows x {cfg.hidden} "
                      f"(same recipe), median of 3 runs {', '.join(f'{x:.2f}' for x in times)} s after 1 warm-up, "
                      f"{cores} threads",
            "cpu": cpu, "torch": torch.__version__}


def consumer_bytes(rows, hidden, rank, bits, group, n_side=0):
    """Fused consumer bytes = M N (b/8 + 4/G + 2 + 2) + 2 M r + 2 N r (+ 2 M k side columns)."""
    b = rows * hidden * (bits / 8 + 4 / group + 4) + 2 * rows * rank + 2 * hidden * rank
    return b + 2 * rows * n_side


def dense_pieces(ptr) -> int:
    """64-column pieces with more entries than the legacy encode's staged record holds (2), from
    the compacted piece pointers: the pieces whose dense values the encode writes."""
    return int(((ptr[1:] - ptr[:-1]) > 2).sum().item())


def staged_bytes(E, bits, npieces, nnz, ndense, small):
    """Algorithmic bytes of lrq_legacy_encode_coo on its staged path: encode = x read, codes
    written, each piece's 8-byte record written (and the 128 dense bytes of the pieces a record
    cannot hold); compaction = those read once, the COO entries (3 int64 indices + bf16 value)
    and the piece pointers written."""
    handoff = npieces * 8 + ndense * 128
    return E * (2 + bits / 8) + small + handoff, handoff + nnz * 26 + npieces * 8


def build_plan_legacy(cfg, pkg, lib, dev, nbuf):
    """The reference's own format: encode (codes + each piece's staged outliers), the GPU
    compaction of the outliers to COO, and the decode reading the COO pieces; l / r rows sized
    for x[1, M, N]."""
    import torch
    c_void_p = ctypes.c_void_p
    sp = c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    M, N, K, bits = cfg.rows, cfg.hidden, cfg.rank, cfg.bits
    ops = pkg.inputs.legacy_operands(cfg, dev)
    l, r, s = ops["l"], ops["r"], ops["s"]
    rt = r.t().contiguous()
    npc = (N + 63) // 64
    cap = M * N // 32
    wsb = lib.lrq_coo_workspace(1, M, N)
    sets = []
    for i in range(nbuf):
        x = pkg.inputs.activation(M, N, cfg.n_outlier, cfg.outlier_scale, cfg.seed + i, dev).view(1, M, N)
        sets.append(dict(x=x, o=torch.empty_like(x), q=torch.empty((1, M, N * bits // 8), dtype=torch.uint8, device=dev),
                         idx=torch.empty((3, cap), dtype=torch.int64, device=dev),
                         vals=torch.empty((cap,), dtype=torch.bfloat16, device=dev),
                         nnz=torch.empty((1,), dtype=torch.int64, device=dev),
                         ptr=torch.empty((M * npc + 1,), dtype=torch.int64, device=dev),
                         ws=torch.empty(((wsb + 7) // 8,), dtype=torch.int64, device=dev),
                         out=torch.empty_like(x)))
    tau = float(pkg.outlier_threshold(l, r, sets[0]["x"]).item())  # 1 % outliers, as the reference calibrates
    P = lambda t: c_void_p(t.data_ptr())  # noqa: E731
    # the encode and the outlier compaction in one call (the encode stages each piece's count and
    # first entries, so the compaction reads those instead of dense outliers)
    enc = lambda k: lib.lrq_legacy_encode_coo(P(l), P(rt), K, P(sets[k]["x"]), 1, M, N, M * N, N, P(s), 1,  # noqa: E731
                                              bits, tau, P(sets[k]["o"]), P(sets[k]["q"]), P(sets[k]["idx"]), cap,
                                              P(sets[k]["vals"]), cap, P(sets[k]["nnz"]), P(sets[k]["ptr"]),
                                              P(sets[k]["ws"]), wsb, sp)
    dec = lambda k: lib.lrq_legacy_decode_coo(P(l), P(rt), K, P(sets[k]["q"]), P(sets[k]["ptr"]),  # noqa: E731
                                              c_void_p(sets[k]["idx"].data_ptr() + 2 * cap * 8), P(sets[k]["vals"]),
                                              cap, P(s), 1, 1, M, N, bits, P(sets[k]["out"]), sp)
    for k in range(nbuf):
        if enc(k):
            raise RuntimeError("legacy encode / compaction failed")
    torch.cuda.synchronize()
    nnz = max(int(st["nnz"].item()) for st in sets)
    if nnz > cap:
        raise RuntimeError(f"{nnz} outliers exceed the bench capacity {cap}")
    small = 2 * (M * K + N * K) + 2 * N
    enc_b, cmp_b = staged_bytes(M * N, bits, M * npc, nnz, max(dense_pieces(st["ptr"]) for st in sets), small)
    entries = [
        ("encode_coo", enc, enc_b + cmp_b, 2 * M * N * K),
        ("decode", dec, M * N * (bits / 8 + 2) + nnz * 10 + M * npc * 8 + small, 2 * M * N * K),
    ]
    sets[0]["alg_split"] = {"encode": enc_b, "compact": cmp_b}
    # the reference's sparse conversion of the same outliers, dense (lrq_legacy_encode), for
    # comparison (it synchronises the host to size its output): mean over 20 calls
    o0, q0 = torch.empty_like(sets[0]["x"]), torch.empty_like(sets[0]["q"])
    if lib.lrq_legacy_encode(P(l), P(rt), K, P(sets[0]["x"]), 1, M, N, M * N, N, P(s), 1, bits, tau, P(o0), P(q0), sp):
        raise RuntimeError("legacy encode failed")
    o0.to_sparse()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        o0.to_sparse()
    torch.cuda.synchronize()
    sets[0]["torch_to_sparse_us"] = (time.perf_counter() - t0) / 20 * 1e6
    sets[0]["nnz_count"] = nnz
    sets[0]["tau"] = tau
    return entries, 2 * M * N, ["encode_coo", "decode"], sets


def build_plan_ref(cfg, pkg, lib, dev, nbuf):
    """The reference's own speed tests of its format, x [B, M, M] (see inputs.CONFIGS): ref_enc =
    the 1-bit encode (codes + staged outliers) and the GPU compaction of the outliers to COO (the
    reference's o.to_sparse(), without its host synchronisation); ref_dec = the 2-bit decode
    reading COO outliers o = N(0,1) * (o > 1) (built once by the same compaction, not timed)."""
    import torch
    c_void_p = ctypes.c_void_p
    sp = c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    B, M, N, K, bits = cfg.batch, cfg.hidden, cfg.hidden, cfg.rank, cfg.bits
    ops = pkg.inputs.ref_operands(cfg, dev)
    l, r, s = ops["l"], ops["r"], ops["s"]
    rt = r.t().contiguous()
    npc = (N + 63) // 64
    P = lambda t: c_void_p(t.data_ptr())  # noqa: E731
    wsb = lib.lrq_coo_workspace(B, M, N)
    cap = B * M * N // 64 if cfg.consumer == "ref_enc" else int(0.2 * B * M * N) + 1024
    sets = []
    for i in range(nbuf):
        g = torch.Generator(device=dev)
        g.manual_seed(cfg.seed + 101 * i)
        if cfg.consumer == "ref_mm":  # no outliers: no COO buffers
            st = dict(nnz=torch.zeros((1,), dtype=torch.int64, device=dev))
        else:
            st = dict(idx=torch.empty((3, cap), dtype=torch.int64, device=dev),
                      vals=torch.empty((cap,), dtype=torch.bfloat16, device=dev),
                      nnz=torch.empty((1,), dtype=torch.int64, device=dev),
                      ptr=torch.empty((B * M * npc + 1,), dtype=torch.int64, device=dev),
                      ws=torch.empty(((wsb + 7) // 8,), dtype=torch.int64, device=dev))
        if cfg.consumer == "ref_mm":
            st["q"] = torch.randint(0, 256, (B, M, N * bits // 8), generator=g, device=dev, dtype=torch.uint8)
            st["y"] = torch.randn((B, N, MM_COLS), generator=g, device=dev).to(torch.bfloat16)
            st["out"] = torch.empty((B, M, MM_COLS), dtype=torch.bfloat16, device=dev)
        elif cfg.consumer == "ref_enc":
            st["x"] = torch.randn((B, M, N), generator=g, device=dev).to(torch.bfloat16)
            st["o"] = torch.empty_like(st["x"])
            st["q"] = torch.empty((B, M, N * bits // 8), dtype=torch.uint8, device=dev)
        else:
            st["q"] = torch.randint(0, 256, (B, M, N * bits // 8), generator=g, device=dev, dtype=torch.uint8)
            st["out"] = torch.empty((B, M, N), dtype=torch.bfloat16, device=dev)
            o = torch.randn((B, M, N), generator=g, device=dev).to(torch.bfloat16)
            o = o * (o > 1)
            if lib.lrq_coo_compact(P(o), B, M, N, P(st["idx"]), cap, P(st["vals"]), cap, P(st["nnz"]), P(st["ptr"]),
                                   P(st["ws"]), wsb, sp):
                raise RuntimeError("compaction failed")
            torch.cuda.synchronize()
            del o
        sets.append(st)
    enc = lambda k: lib.lrq_legacy_encode_coo(P(l), P(rt), K, P(sets[k]["x"]), B, M, N, M * N, N, P(s), B,  # noqa: E731
                                              bits, cfg.tau, P(sets[k]["o"]), P(sets[k]["q"]), P(sets[k]["idx"]),
                                              cap, P(sets[k]["vals"]), cap, P(sets[k]["nnz"]), P(sets[k]["ptr"]),
                                              P(sets[k]["ws"]), wsb, sp)
    dec = lambda k: lib.lrq_legacy_decode_coo(P(l), P(rt), K, P(sets[k]["q"]), P(sets[k]["ptr"]),  # noqa: E731
                                              c_void_p(sets[k]["idx"].data_ptr() + 2 * cap * 8), P(sets[k]["vals"]),
                                              cap, P(s), B, B, M, N, bits, P(sets[k]["out"]), sp)
    if cfg.consumer == "ref_enc":
        for k in range(nbuf):
            if enc(k):
                raise RuntimeError("encode / compaction failed")
    torch.cuda.synchronize()
    nnz = max(int(st["nnz"].item()) for st in sets)
    if nnz > cap:
        raise RuntimeError(f"{nnz} outliers exceed the bench capacity {cap}")
    small = 2 * (M * K + N * K) + 2 * B * N
    E = B * M * N
    if cfg.consumer == "ref_mm":
        # algorithmic: the codes, l, r, s and y read once, out written once (x_hat never stored)
        mm = lambda k: lib.lrq_legacy_dequant_gemm(P(l), P(rt), K, P(sets[k]["q"]), P(s), B, B, M, N, bits,  # noqa: E731
                                                   P(sets[k]["y"]), MM_COLS, MM_COLS, P(sets[k]["out"]), MM_COLS, sp)
        mm_b = E * bits / 8 + small + 2 * B * N * MM_COLS + 2 * B * M * MM_COLS
        entries = [("legacy_gemm", mm, mm_b, 2 * E * K + 2 * E * MM_COLS)]
        timed = ["legacy_gemm"]
    elif cfg.consumer == "ref_enc":
        enc_b, cmp_b = staged_bytes(E, bits, B * M * npc, nnz, max(dense_pieces(st["ptr"]) for st in sets), small)
        entries = [("encode_coo", enc, enc_b + cmp_b, 2 * E * K)]
        timed = ["encode_coo"]
        sets[0]["alg_split"] = {"encode": enc_b, "compact": cmp_b}
    else:
        entries = [("decode", dec, E * (bits / 8 + 2) + nnz * 10 + B * M * npc * 8 + small, 2 * E * K)]
        timed = ["decode"]
    sets[0]["nnz_count"] = nnz
    sets[0]["tau"] = cfg.tau
    return entries, 2 * E, timed, sets


def build_plan(cfg, pkg, lib, dev, nbuf, lora_split=False):
    """Per-config step: a list of (name, launch(k) -> status, algorithmic bytes, mfma flops) run
    in order on buffer set k, plus the step's activation bytes and how `value` is formed."""
    import torch
    if cfg.consumer == "legacy":
        return build_plan_legacy(cfg, pkg, lib, dev, nbuf)
    if cfg.consumer in ("ref_enc", "ref_dec", "ref_mm"):
        return build_plan_ref(cfg, pkg, lib, dev, nbuf)
    c_void_p = ctypes.c_void_p
    sp = c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    M, N, r = cfg.rows, cfg.hidden, cfg.rank
    V = pkg.inputs.basis(N, r, cfg.seed).to(dev) if r else None
    basis = pkg.LowRankBasis(V) if r else None
    if basis is not None:
        _ = basis.Vt
    sets = []
    for i in range(nbuf):
        if cfg.consumer == "softmax":
            x = pkg.inputs.softmax_probs((M, N), seed=cfg.seed + i, device=dev)
        else:
            x = pkg.inputs.activation(M, N, cfg.n_outlier, cfg.outlier_scale, cfg.seed + i, dev)
        idx = None
        if cfg.keep_channels:
            idx = pkg.topk_channels(pkg.column_absmax(x), cfg.keep_channels)
        c = pkg.encode(x, basis, bits=cfg.bits, group_size=cfg.group, hadamard=cfg.hadamard, outlier_idx=idx)
        st = dict(x=x, c=c, out=torch.empty_like(x), enc=c.descriptor(for_encode=True), dec=c.descriptor())
        if cfg.hadamard:
            st["y"] = torch.empty_like(x)
        if cfg.keep_channels:
            st["cm"] = torch.empty((N,), dtype=torch.float32, device=dev)
        if cfg.consumer == "lora":
            n = cfg.lora_rank
            st["a"] = pkg.inputs.lora_factor(N, n, cfg.seed + i, dev)
            st["g"] = pkg.inputs.gradient((M, n), 0.05, cfg.seed + i, dev)
            st["xa"] = torch.empty((M, n), dtype=torch.bfloat16, device=dev)
            st["da"] = torch.empty((N, n), dtype=torch.float32, device=dev)
            wsb = lib.lrq_dequant_gemm_t_workspace(ctypes.byref(st["dec"]), n)
            st["ws"] = torch.empty((max(wsb, 16) + 15) // 16 * 4, dtype=torch.float32, device=dev)
        elif cfg.consumer != "decode":
            st["dy"] = pkg.inputs.gradient((M, N), cfg.grad_std, cfg.seed + i, dev)
        sets.append(st)
    torch.cuda.synchronize()
    P = lambda t: c_void_p(t.data_ptr())  # noqa: E731
    B = lambda d: ctypes.byref(d)  # noqa: E731
    side = cfg.keep_channels
    enc_b = algorithmic_bytes(M, N, r, cfg.bits, cfg.group, side)
    entries = []
    if cfg.keep_channels:
        entries.append(("colmax", lambda k: lib.lrq_colmax(P(sets[k]["x"]), N, M, N, P(sets[k]["cm"]), sp),
                        2 * M * N, 0))
        entries.append(("topk", lambda k: lib.lrq_topk(P(sets[k]["cm"]), N, side, c_void_p(sets[k]["c"].idx.data_ptr()),
                                                       sp), 4 * N, 0))
    enc_flops = 4 * M * N * r
    src = "x"
    if cfg.hadamard:
        # rotated format: the library's encode rotates x as it reads it where it can (flagged
        # descriptor); otherwise a separate rotation pass into y, then the plain encode of y
        flag = importlib.import_module("triton-kernel-test_amd._lib").LRQ_FLAG_HADAMARD
        for st_ in sets:
            st_["enc"].flags = flag
        if lib.lrq_encode(B(sets[0]["enc"]), P(sets[0]["x"]), N, sp) == 0:
            enc_flops += 2 * M * N * 128
        else:
            for st_ in sets:
                st_["enc"].flags = 0
            entries.append(("wht128", lambda k: lib.lrq_wht128(P(sets[k]["x"]), N, M, N, P(sets[k]["y"]), N, sp),
                            4 * M * N, 2 * M * N * 128))
            src = "y"
        torch.cuda.synchronize()
    entries.append(("encode", lambda k: lib.lrq_encode(B(sets[k]["enc"]), P(sets[k][src]), N, sp), enc_b,
                    enc_flops))
    if cfg.consumer == "decode":
        dec_flops = 2 * M * N * r + (2 * M * N * 128 if cfg.hadamard else 0)
        # the rotation is part of the decode's algorithm, not of its minimal traffic: a decode
        # that rotates in a separate pass moves more than these bytes and shows a lower fraction
        entries.append(("decode", lambda k: lib.lrq_decode(B(sets[k]["dec"]), P(sets[k]["out"]), N, sp),
                        enc_b, dec_flops))
        timed = None  # value over the whole step (round trip)
    elif cfg.consumer == "lora":
        # the LoRA layer's backward on the codes: x A (dequant-GEMM, bf16 out) and
        # dA = x^T g (transposed dequant-GEMM, fp32 out); bytes = codes + qparams + L + V read
        # once per kernel, plus each kernel's small operands and output
        n = cfg.lora_rank
        base = M * N * (cfg.bits / 8 + 4 / cfg.group) + 2 * M * r + 2 * N * r
        lws = lib.lrq_lora_grads_workspace(B(sets[0]["dec"]), n)
        if lws > 0 and not lora_split:
            # both products from one pass over the codes (lrq_lora_grads): codes + qparams + L + V
            # once, A and g, x A out (bf16) and dA out (fp32)
            lw = torch.empty((lws + 15) // 16 * 4, dtype=torch.float32, device=dev)
            entries.append(("lora_grads", lambda k: lib.lrq_lora_grads(B(sets[k]["dec"]), P(sets[k]["a"]), n, P(sets[k]["g"]),
                                                                  n, n, P(sets[k]["xa"]), n, 0, P(sets[k]["da"]), n, 1,
                                                                  P(lw), lw.numel() * 4, sp),
                            base + 2 * N * n + 4 * M * n + 4 * N * n, 2 * M * N * r + 4 * M * N * n))
            return entries, 2 * M * N, ["lora_grads"], sets
        rot = 2 * M * N * 128 if cfg.hadamard else 0  # the rotation's MFMA flops, once per kernel
        entries.append(("xa", lambda k: lib.lrq_dequant_gemm(B(sets[k]["dec"]), P(sets[k]["a"]), n,
                                                             P(sets[k]["xa"]), n, 0, sp),
                        base + 2 * N * n + 2 * M * n, 2 * M * N * r + 2 * M * N * n + rot))
        entries.append(("da", lambda k: lib.lrq_dequant_gemm_t(B(sets[k]["dec"]), P(sets[k]["g"]), n, n,
                                                               P(sets[k]["da"]), n, 1, P(sets[k]["ws"]),
                                                               sets[k]["ws"].numel() * 4, sp),
                        base + 2 * M * n + 4 * N * n, 2 * M * N * r + 2 * M * N * n + rot))
        timed = ["xa", "da"]  # value over both gradient kernels (the encode is the producer)
    else:
        fn = {"silu": lib.lrq_silu_bwd, "gelu": lib.lrq_gelu_bwd, "softmax": lib.lrq_softmax_bwd}[cfg.consumer]
        name = f"{cfg.consumer}_bwd"
        # (the rotated softmax rotates each block twice, once per sweep)
        rot = (2 if cfg.consumer == "softmax" else 1) * 2 * M * N * 128 if cfg.hadamard else 0
        entries.append((name, lambda k: fn(B(sets[k]["dec"]), P(sets[k]["dy"]), N, P(sets[k]["out"]), N, sp),
                        consumer_bytes(M, N, r, cfg.bits, cfg.group, side), 2 * M * N * r + rot))
        timed = [name]  # value over the fused consumer (the encode is the producer)
    return entries, 2 * M * N, timed, sets


def offload_bench(args, pkg, lib, dev):
    """--config offload: the north-star compressed activation (codes, qparams, L: 37.2 MB)
    offloaded to pinned host memory and prefetched back (offload.py, on its copy stream) while
    the compute stream runs north-star encode + decode steps.  Times on the GPU (HIP events):
    each copy alone, the compute alone, and both started together; the hidden fraction of a copy
    is (copy + compute - both) / copy, 1.0 when the copy costs the compute nothing."""
    import torch
    OF = importlib.import_module("triton-kernel-test_amd.offload")
    cfg = pkg.inputs.CONFIGS["north_star"]
    entries, _, _, _ = build_plan(cfg, pkg, lib, dev, args.nbuf)
    stream = torch.cuda.current_stream(dev)
    x = pkg.inputs.activation(cfg.rows, cfg.hidden, cfg.n_outlier, cfg.outlier_scale, cfg.seed + 99, dev)
    c = pkg.encode(x, pkg.LowRankBasis(pkg.inputs.basis(cfg.hidden, cfg.rank, cfg.seed).to(dev)), bits=cfg.bits,
                   group_size=cfg.group)
    del x
    pool = OF.PinnedPool()

    def steps(n):
        for i in range(n):
            for _, fn, _, _ in entries:
                if fn(i % args.nbuf):
                    raise RuntimeError("launch failed")

    def run(copy, n):
        """Returns (copy ms, compute ms) from a common start; copy None / n 0 leave one out."""
        torch.cuda.synchronize()
        torch.cuda._sleep(1 << 22)  # the host enqueues everything before the start
        t0, tc = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        ev = copy() if copy is not None else None
        steps(n)
        tc.record(stream)
        torch.cuda.synchronize()
        return (t0.elapsed_time(ev) if ev is not None else 0.0), (t0.elapsed_time(tc) if n else 0.0)

    held = []
    # both copies run on `cs` and start after the common start (the offload makes its stream wait
    # on the compute stream's queue; the prefetch's is made to); the prefetch's consumer is a side
    # stream, so the compute stream does not wait for it
    cs, side = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)

    def done_event():
        e = torch.cuda.Event(enable_timing=True)
        e.record(cs)
        return e

    def d2h():
        # the previous host copies are complete (each run synchronises): back to the pool
        for h in held:
            h.release()
        held.clear()
        held.append(OF.offload(c, stream=cs, pool=pool))
        return done_event()

    def h2d():
        cs.wait_stream(stream)
        with torch.cuda.stream(side):
            OF.prefetch(held[-1], dev, stream=cs)
        return done_event()

    for _ in range(3):  # warm: the pool holds the buffers after the first offload
        run(d2h, 2)
        run(h2d, 2)
        for h in held:
            h.release()
        held.clear()
    allocs0 = pool.allocations
    res = {}
    for name, fn in (("d2h", d2h), ("h2d", h2d)):
        if name == "h2d":
            run(d2h, 0)  # a host copy to read
        alone = statistics.median(run(fn, 0)[0] for _ in range(5))
        n = max(4, int(2.0 * alone / 0.062))  # about twice the copy's time of compute
        comp = statistics.median(run(None, n)[1] for _ in range(5))
        pairs = [run(fn, n) for _ in range(5)]
        both = statistics.median(max(a, b) for a, b in pairs)
        copy_in = statistics.median(a for a, _ in pairs)
        res[name] = {"copy_alone_us": round(alone * 1e3, 1), "GBs_alone": round(c.nbytes() / (alone * 1e-3) / 1e9, 2),
                     "copy_overlapped_us": round(copy_in * 1e3, 1), "compute_steps": n,
                     "compute_alone_us": round(comp * 1e3, 1), "both_us": round(both * 1e3, 1),
                     "hidden_frac": round((alone + comp - both) / alone, 4),
                     "compute_slowdown": round(both / comp, 4)}
        for h in held:
            h.release()
        held.clear()
    line = {"metric": "offload: compressed-activation copy GB/s (device -> pinned host) and the fraction hidden "
                      "behind encode + decode steps",
            "value": res["d2h"]["GBs_alone"], "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
            "dtype": "u8", "data": "synthetic", "config": {"workload": "offload: north-star compressed activation, "
                                                                       "copy stream against the step's kernels",
                                                           "bytes": c.nbytes()},
            "offload": res, "pool": {"allocations_after_warmup": pool.allocations - allocs0,
                                     "cached_bytes": pool.cached_bytes}}
    print(json.dumps(line), flush=True)


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
    if args.config == "offload":
        dev = torch.device("cuda", 0)
        torch.cuda.set_device(dev)
        return offload_bench(args, pkg, lib, dev)
    if args.config == "copy":
        # counter calibration: 5 device copies of 128 MiB (the traffic summaries scale
        # rocprofv3's FETCH_SIZE / WRITE_SIZE by what these report for a known byte count)
        n = 128 * 1024 * 1024
        a = torch.ones(n, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"metric": "copy: calibration copies", "bytes_each": n, "copies": 5}), flush=True)
        return
    cfg = pkg.inputs.CONFIGS[args.config]
    if args.m and cfg.consumer in ("ref_enc", "ref_dec", "ref_mm"):
        import dataclasses
        cfg = dataclasses.replace(cfg, rows=cfg.batch * args.m, hidden=args.m)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)

    entries, act_bytes, timed, _sets = build_plan(cfg, pkg, lib, dev, args.nbuf, lora_split=args.lora_split)

    def step(i, ev=None):
        k = i % args.nbuf
        st = 0
        for e, (name, fn, _, _) in enumerate(entries):
            if ev is not None:
                ev[e].record(stream)
            st |= fn(k)
        if ev is not None:
            ev[len(entries)].record(stream)
        if st:
            raise RuntimeError(f"launch failed: {lib_mod.status_string(st)}")

    # ---- exactly W untimed warm-up steps
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    def timed_steps():
        """Exactly K steps between two events on the launch stream, synchronised before and
        after; returns (ms per step, host ms spent enqueueing them)."""
        t_start = torch.cuda.Event(enable_timing=True)
        t_end = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        h0 = time.perf_counter()
        t_start.record(stream)
        for i in range(args.steps):
            step(i)
        t_end.record(stream)
        h1 = time.perf_counter()
        torch.cuda.synchronize()
        return t_start.elapsed_time(t_end) / args.steps, (h1 - h0) * 1e3

    # ---- timed region (the headline): exactly K steps, nothing else on the stream
    ms_step, host_ms = timed_steps()

    # ---- the same K steps again after a stretch of sustained work (clock-settled figure)
    settled = None
    if args.settle_seconds > 0:
        n_settle, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.settle_seconds:
            for _ in range(50):
                step(n_settle)
                n_settle += 1
            torch.cuda.synchronize()
        ms_settled, _ = timed_steps()
        settled = {"ms_per_step": round(ms_settled, 5), "after_steps": n_settle,
                   "after_seconds": args.settle_seconds}

    # The per-kernel measurements below pre-fill the stream with a spin kernel so that the host
    # can enqueue every launch before the first one starts: what is timed is the GPU, not the
    # host's launch cost (ctypes + several launches per entry can take longer than a kernel).
    probe_a, probe_b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    probe_a.record(stream)
    torch.cuda._sleep(1 << 20)
    probe_b.record(stream)
    torch.cuda.synchronize()
    cycles_per_us = (1 << 20) / max(probe_a.elapsed_time(probe_b) * 1e3, 1.0)

    def prefill(host_us):
        torch.cuda._sleep(int(max(host_us * 1.5 + 200.0, 200.0) * cycles_per_us))

    # ---- in-step breakdown (a separate pass): HIP events between the kernels of each step
    ne = len(entries)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(ne + 1)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    prefill(host_ms * 1e3 * 1.5)
    for i in range(args.steps):
        step(i, evs[i])
    torch.cuda.synchronize()

    # ---- per-kernel duration: K back-to-back launches of that kernel alone between two
    # events on its stream (dispatch latency overlaps, as in a rocprofv3 kernel trace)
    solo = []
    for e, (name, fn, _, _) in enumerate(entries):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        h0 = time.perf_counter()
        for i in range(2):
            fn(i % args.nbuf)
        torch.cuda.synchronize()
        per_call_us = (time.perf_counter() - h0) * 1e6 / 2
        prefill(per_call_us * args.steps)
        a.record(stream)
        for i in range(args.steps):
            fn(i % args.nbuf)
        b.record(stream)
        torch.cuda.synchronize()
        solo.append(a.elapsed_time(b) / args.steps)

    # ---- the step's last kernel (decode / fused consumer) with its inputs HBM-cold: before each
    # timed launch a 1 GiB fill evicts the L2s and the 256 MB MALL, so the codes the encode
    # wrote are read from HBM (in the step they may still sit in the MALL)
    cold = None
    if args.cold_steps > 0:
        last_name, last_fn = entries[-1][0], entries[-1][1]
        scrub = torch.empty((1 << 29,), dtype=torch.bfloat16, device=dev)
        cms = []
        for i in range(args.cold_steps):
            scrub.fill_(float(i % 7))
            ca, cb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ca.record(stream)
            last_fn(i % args.nbuf)
            cb.record(stream)
            torch.cuda.synchronize()
            cms.append(ca.elapsed_time(cb))
        del scrub
        cold = (last_name, statistics.median(cms))

    kernels = {}
    for e, (name, _, alg, flops) in enumerate(entries):
        ms = [ev[e].elapsed_time(ev[e + 1]) for ev in evs]
        in_step, med = statistics.mean(ms), statistics.median(ms)
        mean = solo[e]
        kernels[name] = {"mean_us": round(mean * 1e3, 2), "in_step_mean_us": round(in_step * 1e3, 2),
                         "in_step_median_us": round(med * 1e3, 2),
                         "alg_GBs": round(alg / (mean * 1e-3) / 1e9, 1),
                         "hbm_frac": round(alg / (mean * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if cold is not None and cold[0] == name:
            kernels[name].update(cold_median_us=round(cold[1] * 1e3, 2),
                                 cold_hbm_frac=round(alg / (cold[1] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4))
        if flops:
            tf = flops / (mean * 1e-3) / 1e12
            kernels[name].update(mfma_tflops=round(tf, 2), mfma_util_derived=round(tf / BF16_DENSE_TFLOPS, 5))
    if timed is None:
        value = act_bytes / (ms_step * 1e-3) / 1e9  # whole step, kernels interleaved as in use
        workload = "encode+decode" + (" with WHT-128 rotation" if cfg.hadamard else "")
    else:
        value = act_bytes / (sum(kernels[t]["mean_us"] for t in timed) * 1e-6) / 1e9
        workload = f"fused {' + '.join(timed)} on the compressed activation (encode timed alongside)"
        if cfg.consumer == "legacy":
            workload = "reference format: encode + outliers to COO on the GPU + decode from the COO pieces"
        elif cfg.consumer == "ref_enc":
            workload = (f"reference speed test, x [{cfg.batch}, {cfg.hidden}, {cfg.hidden}]: {cfg.bits}-bit encode, "
                        f"threshold {cfg.tau:g}, outliers compacted to COO on the GPU")
        elif cfg.consumer == "ref_dec":
            workload = (f"reference speed test, x [{cfg.batch}, {cfg.hidden}, {cfg.hidden}]: {cfg.bits}-bit decode "
                        f"from COO outliers N(0,1) * (o > 1)")
        elif cfg.consumer == "ref_mm":
            workload = (f"reference dequant-matmul bench, x [{cfg.batch}, {cfg.hidden}, {cfg.hidden}] {cfg.bits}-bit "
                        f"rank {cfg.rank} @ y [{cfg.batch}, {cfg.hidden}, {MM_COLS}], one fused kernel")
    dom_name, dom_alg, dom_us = None, 0, -1.0
    for name, _, alg, _ in entries:
        if kernels[name]["mean_us"] > dom_us:
            dom_name, dom_alg, dom_us = name, alg, kernels[name]["mean_us"]
    achieved = dom_alg / (dom_us * 1e-6) / 1e9
    traffic = traffic_from_profiles(f"{dom_name}_{args.config}")
    step_alg = sum(e[2] for e in entries)

    line = {
        "metric": METRIC if args.config == "north_star" else f"{args.config}: activation GB/s and % of HBM peak",
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
        "config": {"workload": f"{args.config}: {workload}", "rows": cfg.rows, "hidden": cfg.hidden,
                   "rank": cfg.rank, "bits": cfg.bits, "group": cfg.group, "buffers": args.nbuf},
        "hbm_frac_step": round(step_alg / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "host_enqueue_ms": round(host_ms, 3),
        "kernels": kernels,
        "roofline": {"bound": "hbm", "kernel": dom_name, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": (traffic or {}).get("bytes_per_launch")},
    }
    if settled is not None:
        ms_s = settled["ms_per_step"]
        settled["value"] = round(act_bytes / (ms_s * 1e-3) / 1e9, 2) if timed is None else None
        settled["hbm_frac_step"] = round(step_alg / (ms_s * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
        line["settled"] = settled
    mf = mfma_from_profiles(args.config)
    if mf is not None:
        line["mfma"] = {k: {"util": v.get("mfma_util"), "busy_cycles_per_launch": v.get("busy_cycles_per_launch")}
                        for k, v in mf.get("kernels", {}).items()}
        line["mfma"]["source"] = f"profiles/mfma_{args.config}.json (rocprofv3 counters)"
    if cfg.consumer == "legacy":
        line["legacy"] = {"outliers": _sets[0]["nnz_count"], "threshold": _sets[0]["tau"],
                          "torch_to_sparse_us": round(_sets[0]["torch_to_sparse_us"], 1)}
    if cfg.consumer in ("ref_enc", "ref_dec", "ref_mm"):
        line["legacy"] = {"outliers": _sets[0]["nnz_count"], "threshold": _sets[0]["tau"], "batch": cfg.batch,
                          "M": cfg.hidden}
    if "alg_split" in _sets[0]:
        line["legacy"]["alg_bytes"] = _sets[0]["alg_split"]
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
