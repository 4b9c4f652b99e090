"""Writes tests/golden/known_answers.json: hand-built known-answer cases whose expected
outputs follow from the construction alone (integer arithmetic and bit formulas), never from
the CPU oracle, so tests/test_oracle.py can pin the oracle against them.

The reference holds no golden vectors for this path; these cases follow its own smoke tests
and formulas instead:
  * legacy encode (low_rank_extraction_fuse_compression_quantization.py:153-171) with
    l @ r = 0, power-of-two scales so x / s is exact, values on the quantiser grid, exact
    .5 ties (round half to even), outliers above the threshold, and saturation at s = 1e-5
    (after low_rank_kernel_accuracy_test.py:25-26);
  * legacy decode (low_rank_extraction_fuse_decompression_dequantization.py:155-165) of
    chosen codes with a power-of-two scale and an outlier tensor;
  * row-planar packing (byte j holds column j + p*N/NP in bits p*b ..);
  * the group quantiser on a ramp whose scale is exact in fp16, and on a constant group;
  * the normalised WHT-128 of unit vectors (a column of H128 / sqrt(128), H by popcount).

Run: python tests/golden/make_known_answers.py
"""

from __future__ import annotations

import json
import math
import struct
from pathlib import Path

OUT = Path(__file__).resolve().parent / "known_answers.json"


def bf16_bits(v: float) -> int:
    """bf16 bits of a value that is exactly representable in bf16 (asserted)."""
    u = struct.unpack("<I", struct.pack("<f", v))[0]
    assert u & 0xFFFF == 0, f"{v} is not exact in bf16"
    return u >> 16


def bf16_rne_bits(v: float) -> int:
    """Round-to-nearest-even fp32 -> bf16 (integer formula)."""
    u = struct.unpack("<I", struct.pack("<f", v))[0]
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF


def rne(x2: int) -> int:
    """round(x2 / 2) half to even, for an integer x2 (the value times two)."""
    q, r = divmod(x2, 2)
    if r == 0:
        return q
    return q if q % 2 == 0 else q + 1  # exact half: to the even neighbour


def pack_rowplanar(codes: list[list[int]], bits: int) -> list[list[int]]:
    npl = 8 // bits
    out = []
    for row in codes:
        nb = len(row) // npl
        out.append([sum(row[p * nb + j] << (bits * p) for p in range(npl)) for j in range(nb)])
    return out


def legacy_encode_case(name, bits, s_exp2, tau, ks, M, N):
    """x = k * s / 2 for integers k (exact in bf16; x / s is a multiple of 1/2, so .5 ties
    occur), l @ r = 0, scale s = 2^s_exp2 everywhere."""
    s = 2.0 ** s_exp2
    half = 1 << (bits - 1)
    values = [k * s / 2 for k in ks]
    x = [[values[(m * N + n) % len(values)] for n in range(N)] for m in range(M)]
    codes, outl = [], []
    for row in x:
        crow, orow = [], []
        for v in row:
            if abs(v) > tau:
                orow.append(bf16_bits(v))
                q = 0
            else:
                orow.append(0)
                x2 = round(2 * v / s)  # v / s is a multiple of 1/2 by construction
                assert abs(x2 * s / 2 - v) < 1e-12
                q = rne(x2)
            crow.append(min(max(q, -half), half - 1) + half)
        codes.append(crow)
        outl.append(orow)
    return dict(name=name, bits=bits, M=M, N=N, K=16, tau=tau,
                x=[[bf16_bits(v) for v in row] for row in x], s=[bf16_bits(s)] * N,
                q=pack_rowplanar(codes, bits), o=outl, codes=codes)


def legacy_saturation_case():
    """s = 1e-5 (bf16-rounded): every non-outlier, non-zero value saturates."""
    bits, M, N, tau = 4, 2, 8, 5.0
    vals = [0.5, -0.5, 1.0, -2.0, 0.0, 3.0, -4.0, 6.0]
    s_bits = bf16_rne_bits(1e-5)
    half = 1 << (bits - 1)
    codes, outl = [], []
    for _ in range(M):
        crow, orow = [], []
        for v in vals:
            if abs(v) > tau:
                orow.append(bf16_bits(v)); crow.append(half)
            else:
                orow.append(0)
                crow.append(half if v == 0 else (half - 1 + half if v > 0 else 0))
        codes.append(crow); outl.append(orow)
    return dict(name="legacy_saturation", bits=bits, M=M, N=N, K=16, tau=tau,
                x=[[bf16_bits(v) for v in vals] for _ in range(M)], s=[s_bits] * N,
                q=pack_rowplanar(codes, bits), o=outl, codes=codes)


def legacy_decode_case():
    """codes c, s = 0.25, outliers o, l @ r = 0: x_hat = (c - 8) * 0.25 + o exactly."""
    bits, M, N = 4, 2, 16
    codes = [[(3 * n + 5 * m) % 16 for n in range(N)] for m in range(M)]
    o = [[(2.5 if (n + m) % 7 == 0 else 0.0) for n in range(N)] for m in range(M)]
    xh = [[(codes[m][n] - 8) * 0.25 + o[m][n] for n in range(N)] for m in range(M)]
    return dict(name="legacy_decode", bits=bits, M=M, N=N, K=16, s=[bf16_bits(0.25)] * N,
                q=pack_rowplanar(codes, bits), o=[[bf16_bits(v) for v in r] for r in o],
                x_hat=[[bf16_bits(v) for v in r] for r in xh])


def rowplanar_cases():
    cases = []
    for bits in (1, 2, 4, 8):
        N = 16
        codes = [[(7 * n + 3) % (1 << bits) for n in range(N)], [(n * n) % (1 << bits) for n in range(N)]]
        cases.append(dict(bits=bits, codes=codes, packed=pack_rowplanar(codes, bits)))
    return cases


def group_ramp_case():
    """r = (k mod 16) / 8 over a 64-group: mn = 0, mx = 15/8, scale = 1/8 (fp16-exact),
    zero = 0, codes = k mod 16; plus a constant group (scale guarded to 1, codes 0)."""
    G = 64
    ramp = [(k % 16) / 8.0 for k in range(G)]
    const = [3.0] * G
    return dict(bits=4, group=G, r=[ramp + const], codes=[[k % 16 for k in range(G)] + [0] * G],
                scale=[[0.125, 1.0]], zero=[[0.0, 3.0]])


def wht_unit_cases():
    """WHT128(e_k) = H128[:, k] / sqrt(128): entries +-fp32(1/sqrt(128)), rounded to bf16."""
    cases = []
    mag = bf16_rne_bits(struct.unpack("<f", struct.pack("<f", 1.0 / math.sqrt(128.0)))[0])
    for k in (0, 1, 37, 127):
        row = []
        for o in range(128):
            neg = bin(o & k).count("1") & 1
            row.append(mag | (0x8000 if neg else 0))
        cases.append(dict(k=k, y=row))
    return cases


def main():
    # multiples of s/2: odd k are exact .5 ties; large |k| saturate or exceed the threshold
    ks = [0, 1, -1, 2, -3, 3, 5, -5, 7, -7, 9, 14, -15, 16, -17, 30, 41, -44, 100, -120]
    data = dict(
        legacy_encode=[
            legacy_encode_case("legacy_grid_b4", 4, -1, 5.0, ks, 3, 32),
            legacy_encode_case("legacy_grid_b8", 8, -3, 5.0, ks, 2, 16),
            legacy_encode_case("legacy_grid_b2", 2, 0, 1.6, ks, 2, 16),
            legacy_saturation_case(),
        ],
        legacy_decode=[legacy_decode_case()],
        rowplanar=rowplanar_cases(),
        group_ramp=group_ramp_case(),
        wht_unit=wht_unit_cases(),
    )
    OUT.write_text(json.dumps(data, indent=1) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
