"""The legacy encode's division by the scale and its code step (csrc/lrq_legacy.hip, the MFMA
encode) against the reference's (low_rank_extraction_fuse_compression_quantization.py:165-166,
torch form: `(x - o) / s`, bf16, then round and clamp), exhaustively on the host
(tests/legacy_code_check.c):

* the code forms: at 1 bit one compare of the fp32 quotient with -(0.5 + 2^-9); at 2, 4 and 8
  bits the clamped bits of bf16(q) + 1.5 * 2^23; both equal clamp(rint(bf16(q))) + 2^(b-1) for
  every fp32 quotient but NaN;
* the quotient: for every finite bf16 numerator and every bf16 scale with
  2^-100 <= |s| <= 2^100, the estimate a * RN32(1/s) gives the IEEE quotient's code at 1, 2, 4
  and 8 bits.

The check fails for a threshold of -0.5, a bias of 2^23, or an estimate off by 10^-4."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_code_step_forms_give_the_reference_codes(tmp_path):
    exe = tmp_path / "legacy_code_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-o", str(exe), str(HERE / "legacy_code_check.c"),
                    "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=600).stdout.split()
    checked, bad1, bad2, bad4, bad8, pairs, e1, e2, e4, e8 = map(int, out)
    assert checked == 2 ** 32 - 2 * (2 ** 23 - 1)  # every bit pattern but the NaNs
    assert (bad1, bad2, bad4, bad8) == (0, 0, 0, 0)
    # scales: the 200 binades 2^-100 .. 2^99 (128 each) and 2^100, both signs; numerators: the
    # 65280 finite bf16 values
    assert pairs == 2 * (200 * 128 + 1) * 65280
    assert (e1, e2, e4, e8) == (0, 0, 0, 0)
