"""Seeded synthetic inputs for the five BASELINE.json configurations.

Parity inputs are drawn on the CPU with ``torch.Generator().manual_seed(seed)`` in fp32 and
cast to bf16, so the HIP path and the CPU oracle see identical bits.  Full-size benchmark
inputs may instead be drawn on the device (``device="cuda"``): same recipe, different
random stream, much faster.

Recipes (BASELINE.json "configs"):
  c1 / north_star  X[rows, 4096] ~ N(0,1), 8 seeded channels x20; V = QR(randn(4096, 16)).Q;
                   rank 16, int4, group 64 (c1: 2048 rows, north star: 16384 rows)
  c2               X[8192, 11008] ~ N(0,1); V[11008, 32]; int4/g64; dY = 0.02 N(0,1)  (SiLU bwd)
  c3               X[16384, 4096] ~ N(0,1), 41 channels x50; top-41 channels to fp16 side columns;
                   rest int8/g128, rank 0; dY = 0.02 N(0,1)                              (GELU bwd)
  c4               X[16384, 5120] ~ N(0,1), 16 channels x30; WHT-128 rotation; V[5120, 16]; int4/g64
  c5               P = softmax(N(0,1)/sqrt(128)) over [2, 32, 2048, 2048] (rows of 2048);
                   V[2048, 16]; int4/g64 per row; dP = 0.02 N(0,1)                       (softmax bwd)
Further workloads of the same recipes (lora, c4l, c4s, c5w, legacy, ref_*) are described at
their CONFIGS entries.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

__all__ = ["Config", "CONFIGS", "REF_M", "activation", "basis", "gradient", "softmax_probs", "lora_factor",
           "legacy_operands", "ref_operands", "make"]


@dataclass(frozen=True)
class Config:
    name: str
    rows: int
    hidden: int
    rank: int
    bits: int
    group: int
    n_outlier: int = 0          # channels scaled to act as outliers
    outlier_scale: float = 1.0
    keep_channels: int = 0      # channels kept dense as fp16 side columns (top-k by abs-max)
    hadamard: bool = False
    consumer: str = "decode"    # decode | silu | gelu | softmax | lora | legacy | ref_enc | ref_dec | ref_mm
    lora_rank: int = 16         # consumer "lora": n of the LoRA factor A [hidden, n] and of g [rows, n]
    grad_std: float = 0.02
    seed: int = 0
    softmax_shape: tuple = field(default=())
    batch: int = 1              # ref_enc / ref_dec: x is [batch, rows / batch, hidden]
    tau: float = 0.0            # ref_enc: the outlier threshold


CONFIGS = {
    "north_star": Config("north_star", 16384, 4096, 16, 4, 64, n_outlier=8, outlier_scale=20.0, seed=0),
    "c1": Config("c1", 2048, 4096, 16, 4, 64, n_outlier=8, outlier_scale=20.0, seed=1),
    "c2": Config("c2", 8192, 11008, 32, 4, 64, consumer="silu", seed=2),
    "c3": Config("c3", 16384, 4096, 0, 8, 128, n_outlier=41, outlier_scale=50.0, keep_channels=41,
                 consumer="gelu", seed=3),
    "c4": Config("c4", 16384, 5120, 16, 4, 64, n_outlier=16, outlier_scale=30.0, hadamard=True, seed=4),
    "c5": Config("c5", 2 * 32 * 2048, 2048, 16, 4, 64, consumer="softmax", seed=5,
                 softmax_shape=(2, 32, 2048, 2048)),
    # config 5's recipe at the reference softmax bench's widest rows (softmax_backward.py:80, N = 4096):
    # 4 of the 64 (batch, head) pairs of [2, 32, 4096, 4096], i.e. 16384 rows of 4096 (two-sweep kernel)
    "c5w": Config("c5w", 4 * 4096, 4096, 16, 4, 64, consumer="softmax", seed=8, softmax_shape=(2, 32, 4096, 4096)),
    # the LoRA layer's backward from the north-star format: x A and dA = x^T (dy B^T)
    "lora": Config("lora", 16384, 4096, 16, 4, 64, n_outlier=8, outlier_scale=20.0, consumer="lora", seed=6),
    # the rotated format's consumers that reduce over the hidden dimension: the two LoRA products
    # (x A and dA = x^T g, the rotation inside each) and the softmax backward, at 4096 columns
    "c4l": Config("c4l", 16384, 4096, 16, 4, 64, n_outlier=8, outlier_scale=20.0, hadamard=True, consumer="lora",
                  seed=12),
    "c4s": Config("c4s", 16384, 4096, 16, 4, 64, hadamard=True, consumer="softmax", seed=13,
                  softmax_shape=(1, 4, 4096, 4096)),
    # the reference's own format (legacy): rank-16 factors, 2-bit symmetric codes (the system
    # profile's quantize_bit=2), outliers above the 99th percentile kept as COO
    "legacy": Config("legacy", 16384, 4096, 16, 2, 0, n_outlier=8, outlier_scale=20.0, consumer="legacy", seed=7),
    # the reference's own speed tests of its format (low_rank_kernel_encode_speed_test.py:28-48,
    # low_rank_kernel_decode_speed_test.py:28-53): x [4, M, M] ~ N(0,1), l [M, 16] and r [16, M]
    # ~ N(0,1), s = N(0,1) + 2 per batch row; 1-bit encode with threshold 12 (outliers compacted to
    # COO on the GPU), 2-bit decode from COO outliers o = N(0,1) * (o > 1).  M is 256 * {2, 12, ..,
    # 72} there; bench.py --m picks it (default 8192).
    "ref_enc": Config("ref_enc", 4 * 8192, 8192, 16, 1, 0, consumer="ref_enc", seed=9, batch=4, tau=12.0),
    "ref_dec": Config("ref_dec", 4 * 8192, 8192, 16, 2, 0, consumer="ref_dec", seed=10, batch=4),
    # the reference's fused dequant-matmul benchmark (extraction_fuse_matmul.py:425-436): codes
    # q [4, M, M/4] (2-bit), l [M, 32], r [32, M], s [4, M] = N(0,1) + 2, y [4, M, 32]; out
    # [4, M, 32].  bench.py --m picks M (default 4096).
    "ref_mm": Config("ref_mm", 4 * 4096, 4096, 32, 2, 0, consumer="ref_mm", seed=11, batch=4),
}

REF_M = [256 * i for i in range(2, 80, 10)]  # the reference speed tests' sweep: 512 .. 18432


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def activation(rows: int, hidden: int, n_outlier: int = 0, outlier_scale: float = 1.0, seed: int = 0,
               device="cpu") -> torch.Tensor:
    """X ~ N(0,1) [rows, hidden] with ``n_outlier`` seeded channels scaled; bf16."""
    g = _gen(seed, device)
    x = torch.randn((rows, hidden), generator=g, device=device, dtype=torch.float32)
    if n_outlier:
        ch = torch.randperm(hidden, generator=g, device=device)[:n_outlier]
        x[:, ch] *= outlier_scale
    return x.to(torch.bfloat16)


def basis(hidden: int, rank: int, seed: int = 0) -> torch.Tensor:
    """Orthonormal V[hidden, rank] = QR(randn).Q, drawn on the CPU, cast to bf16."""
    g = _gen(seed + 1_000_003, "cpu")
    q, _ = torch.linalg.qr(torch.randn((hidden, rank), generator=g, dtype=torch.float32))
    return q.to(torch.bfloat16)


def gradient(shape, std: float = 0.02, seed: int = 0, device="cpu") -> torch.Tensor:
    g = _gen(seed + 2_000_003, device)
    return (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std).to(torch.bfloat16)


def softmax_probs(shape, seed: int = 0, device="cpu") -> torch.Tensor:
    """P = softmax(N(0,1)/sqrt(128)) along the last axis, computed in fp32, cast to bf16."""
    g = _gen(seed, device)
    logits = torch.randn(shape, generator=g, device=device, dtype=torch.float32) / math.sqrt(128.0)
    return torch.softmax(logits, dim=-1).to(torch.bfloat16)


def make(cfg: Config, rows: int | None = None, device="cpu") -> dict:
    """Inputs for ``cfg`` with the row count optionally reduced (parity sizes)."""
    rows = cfg.rows if rows is None else rows
    out = {}
    if cfg.consumer == "softmax":
        out["x"] = softmax_probs((rows, cfg.hidden), seed=cfg.seed, device=device)
    else:
        out["x"] = activation(rows, cfg.hidden, cfg.n_outlier, cfg.outlier_scale, cfg.seed, device)
    out["V"] = basis(cfg.hidden, cfg.rank, cfg.seed) if cfg.rank else None
    if cfg.consumer == "lora":
        out["a"] = lora_factor(cfg.hidden, cfg.lora_rank, cfg.seed, device)
        out["g"] = gradient((rows, cfg.lora_rank), 0.05, cfg.seed, device)
    elif cfg.consumer != "decode":
        out["dy"] = gradient((rows, cfg.hidden), cfg.grad_std, cfg.seed, device)
    return out


def legacy_operands(cfg: Config, device="cpu") -> dict:
    """Factors l [rows, K], r [K, hidden] (N(0, 0.25)) and per-column scale s [1, hidden]
    (U(0.05, 0.35)) of the legacy format, bf16, drawn on the CPU."""
    g = _gen(cfg.seed + 4_000_037, "cpu")
    l = (torch.randn((cfg.rows, cfg.rank), generator=g) * 0.5).to(torch.bfloat16)
    r = (torch.randn((cfg.rank, cfg.hidden), generator=g) * 0.5).to(torch.bfloat16)
    s = (0.05 + 0.3 * torch.rand((1, cfg.hidden), generator=g)).to(torch.bfloat16)
    return {"l": l.to(device), "r": r.to(device), "s": s.to(device)}


def ref_operands(cfg: Config, device="cpu") -> dict:
    """The reference speed tests' operands for x [B, M, M]: l [M, 16], r [16, M] ~ N(0,1),
    s [B, M] = N(0,1) + 2 (bf16)."""
    B, M = cfg.batch, cfg.hidden
    g = _gen(cfg.seed + 5_000_011, device)
    l = torch.randn((M, cfg.rank), generator=g, device=device).to(torch.bfloat16)
    r = torch.randn((cfg.rank, M), generator=g, device=device).to(torch.bfloat16)
    s = (torch.randn((B, M), generator=g, device=device) + 2).to(torch.bfloat16)
    return {"l": l, "r": r, "s": s}


def lora_factor(hidden: int, n: int, seed: int = 0, device="cpu") -> torch.Tensor:
    """A LoRA factor A[hidden, n] ~ N(0, 1/hidden); bf16."""
    g = _gen(seed + 3_000_017, device)
    return (torch.randn((hidden, n), generator=g, device=device, dtype=torch.float32) / math.sqrt(hidden)
            ).to(torch.bfloat16)
