"""The parity bars themselves, on CPU. util.assert_gemv must reject a result one bf16 step too far on
an ordinary output and accept fp32 accumulation noise on an output that cancels to nothing.
util.assert_moe_sum must accept one step of one expert's output in a sum that cancels, and reject a
sum that lost a term or took a wrong route weight."""

import numpy as np
import pytest

import oracle
from util import assert_gemv, assert_moe_sum


def _bf16(v):
    return oracle.bf16_round(np.asarray(v, np.float32))


def test_bar_rejects_two_steps_on_an_ordinary_output():
    want = np.array([30.3, -12.7, 5.1, 0.8], np.float64)
    got16 = _bf16(want).copy()
    got16[1] = np.float32(got16[1]) - np.float32(2 * 0.0625)  # bf16 step at 8..16 is 1/16
    with pytest.raises(AssertionError, match="steps away"):
        assert_gemv(want.astype(np.float32), got16, want)


def test_bar_accepts_noise_on_a_cancelled_output():
    # 5.856e-5 next to outputs of ~30: 3.9e-7 off is two bf16 steps there, and fp32 noise
    want = np.array([30.3, -12.7, 5.1, 5.856342613697052e-05], np.float64)
    got = want.astype(np.float32)
    got[3] = np.float32(5.8174133e-05)  # flips nothing else, so the flip rate counts resolved outputs only
    assert_gemv(got, _bf16(got), want)


def _moe_case():
    rng = np.random.default_rng(4)
    terms = _bf16(rng.standard_normal((9, 512)) * 0.05)  # nine bf16 expert outputs per element
    terms[:, 7] = _bf16([0.5, -0.5, 0.25, -0.25, 0.125, -0.125, 0.03125, -0.03125, 0.0009765625])  # cancels
    want = _bf16(terms.astype(np.float32).sum(0, dtype=np.float32))
    return terms, want


def test_moe_bar_accepts_one_step_of_a_term_in_a_cancelling_sum():
    terms, want = _moe_case()
    moved = terms.copy()
    moved[0, 7] = 0.5 + 2.0 ** -8  # one bf16 step of the first term (0.5 .. 1: step 2^-8)
    got = _bf16(moved.astype(np.float32).sum(0, dtype=np.float32))
    assert abs(got[7] - want[7]) > 2 * 2.0 ** -17  # several steps of the small result
    assert_moe_sum(got, want.astype(np.float64), np.abs(terms).sum(0))


def test_moe_bar_rejects_a_lost_term_or_a_wrong_weight():
    terms, want = _moe_case()
    lost = _bf16(terms[1:].astype(np.float32).sum(0, dtype=np.float32))
    with pytest.raises(AssertionError):
        assert_moe_sum(lost, want.astype(np.float64), np.abs(terms).sum(0))
    scaled = terms.copy()
    scaled[2] *= 1.25  # one route weight 25% off
    wrong = _bf16(scaled.astype(np.float32).sum(0, dtype=np.float32))
    with pytest.raises(AssertionError):
        assert_moe_sum(wrong, want.astype(np.float64), np.abs(terms).sum(0))
