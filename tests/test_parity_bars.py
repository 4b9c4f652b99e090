"""The parity bars themselves (tests/parity.py), on the CPU: each admits the differences it is
written for and rejects a plausible kernel mistake."""

import numpy as np
import pytest

import oracle as O
from parity import assert_decode_close, assert_rotated_close


def _bf16(x):
    return O.bf16_round(np.asarray(x, dtype=np.float32))


def test_rotated_bar_admits_one_ulp_inputs_and_rejects_a_sign():
    rng = np.random.default_rng(0)
    y = _bf16(rng.standard_normal((64, 1024)) * 4)
    ref = O.wht128_bf16(y)
    # a few reconstructed values one ulp off before the rotation (the rank-32 MFMA case)
    y2 = y.copy()
    for r, c in [(0, 5), (3, 700), (17, 128), (40, 1023)]:
        y2[r, c] += 1
    dev = O.wht128_bf16(y2)
    rep = assert_rotated_close(dev, ref, "one-ulp inputs")
    assert rep["frac_ulp"] > 0  # the perturbation is visible, and admitted
    # a sign error in one row of one block
    bad = dev.copy()
    bad[9, 256:384] ^= np.uint16(0x8000)
    with pytest.raises(AssertionError):
        assert_rotated_close(bad, ref, "sign")
    # a block rotated from the wrong columns (neighbouring block's input)
    y3 = y.copy()
    y3[:, 0:128] = y[:, 128:256]
    with pytest.raises(AssertionError):
        assert_rotated_close(O.wht128_bf16(y3), ref, "columns")


def test_decode_bar_rejects_two_ulps():
    rng = np.random.default_rng(1)
    ref = _bf16(rng.standard_normal((16, 256)) + 3)
    dev = ref.copy()
    dev[2, 7] += 1
    assert_decode_close(dev, ref, "one ulp")
    dev[5, 9] += 2
    with pytest.raises(AssertionError):
        assert_decode_close(dev, ref, "two ulps")
