"""The GEMV parity bar itself (util.assert_gemv), on CPU: it must reject a result one bf16 step too
far on an ordinary output and accept fp32 accumulation noise on an output that cancels to nothing."""

import numpy as np
import pytest

import oracle
from util import assert_gemv


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
