"""The legacy encode's division by the scale (csrc/lrq_legacy.hip, legacy_code_rc) against the
reference's IEEE division (low_rank_extraction_fuse_compression_quantization.py:165,
`(x - o) / s` in the torch form), exhaustively on the host: every bf16 scale the fast form
serves (2^-100 <= |s| <= 2^100) and every finite bf16 numerator, at 1, 2, 4 and 8 bits
(tests/legacy_div_check.c).  The identity rests on Markstein's correction of a quotient by a
correctly rounded reciprocal; the check also covers the clamp of very large quotients."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_reciprocal_division_gives_the_ieee_codes(tmp_path):
    exe = tmp_path / "legacy_div_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-o", str(exe), str(HERE / "legacy_div_check.c"), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=600).stdout.split()
    checked, bad1, bad2, bad4, bad8 = map(int, out)
    # scales: the 200 binades 2^-100 .. 2^99 (128 each) and 2^100, both signs; numerators: the
    # 65280 finite bf16 values
    assert checked == 2 * (200 * 128 + 1) * 65280
    assert (bad1, bad2, bad4, bad8) == (0, 0, 0, 0)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_code_step_forms_give_the_reference_codes(tmp_path):
    """The MFMA encode's code step (csrc/lrq_legacy.hip): at 1 bit one compare of the fp32
    quotient with -(0.5 + 2^-9); at 2, 4 and 8 bits the biased integer of bf16(q) + 1.5 * 2^23
    clamped, and at 2 bits three compares of the quotient; all equal clamp(rint(bf16(q))) + 2^(b-1)
    for every fp32 quotient but NaN.  At 1 and 2 bits the quotient may be the estimate
    a * RN32(1/sc): its compares equal the IEEE quotient's for every finite bf16 a and every scale
    the reciprocal path serves (tests/legacy_code_check.c).
    The check fails for a threshold of -0.5 or a bias of 2^23."""
    exe = tmp_path / "legacy_code_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-o", str(exe), str(HERE / "legacy_code_check.c"),
                    "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=600).stdout.split()
    checked, bad1, bad2, bad4, bad8, pairs, bad_est, bad_est2 = map(int, out)
    assert checked == 2 ** 32 - 2 * (2 ** 23 - 1)  # every bit pattern but the NaNs
    assert (bad1, bad2, bad4, bad8) == (0, 0, 0, 0)
    # scales: the 200 binades 2^-100 .. 2^99 (128 each) and 2^100, both signs; numerators: the
    # 65280 finite bf16 values
    assert pairs == 2 * (200 * 128 + 1) * 65280
    assert (bad_est, bad_est2) == (0, 0)
