"""GPU parity of the decoders, quantizers and epilogues against the oracle: bit-exact.

Dequantization must match ref/kernel.py bit for bit (ref/kernel.py:89-90, :98-101), so every
e4m3 and e2m1 code is decoded under a spread of scales, including the E8M0 edge codes 0 and 255.
"""

import numpy as np
import pytest
import torch

import oracle
from stblarge_amd import data, ops
from util import bits_equal, np_

pytestmark = pytest.mark.gpu


def test_dequant_fp4_every_code_every_scale(gpu):
    # 256 rows: row r uses scale byte r for all its groups; each row holds every code byte twice
    k = 1024
    codes = np.tile(np.arange(256, dtype=np.uint8), (256, 2))
    scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], k // 32, axis=1)
    got = ops.dequant_fp4(torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu))
    want = oracle.dequant_fp4(codes, scales)
    assert bits_equal(np_(got), want)


def test_dequant_fp8_every_code(gpu):
    rng = np.random.default_rng(0)
    codes = np.tile(np.arange(256, dtype=np.uint8), (256, 2))  # includes the NaN codes 0x7f, 0xff
    scales = (rng.random((2, 4)) * 0.01).astype(np.float32)
    scales[0, 0] = 1.0
    got = ops.dequant_fp8(torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu))
    assert bits_equal(np_(got), oracle.dequant_fp8_b128(codes, scales))
    e8 = rng.integers(0, 256, (8, 16), dtype=np.uint8)
    got = ops.dequant_fp8(torch.from_numpy(codes).to(gpu), torch.from_numpy(e8).to(gpu), e8m0=True)
    assert bits_equal(np_(got), oracle.dequant_fp8_e8m0_b32(codes, e8))


def test_dequant_gguf17(gpu):
    rng = np.random.default_rng(1)
    rows, k = 37, 512
    codes = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
    scales = rng.integers(0, 256, (rows, k // 32), dtype=np.uint8)
    blocks = oracle.ocp_to_gguf17(codes, scales)
    got = ops.dequant_gguf17(torch.from_numpy(blocks).to(gpu), rows, k)
    assert bits_equal(np_(got), oracle.dequant_fp4(codes, scales))


@pytest.mark.parametrize("rows,k", [(8, 64), (33, 96), (2048, 7168), (7168, 2048)])
def test_quant_fp4_matches_oracle(gpu, rows, k):
    w = data.weight(rows, k, seed=rows + k)
    if rows == 33:  # edge groups: all zero, tiny, signed zeros, huge
        w[0, :32] = 0.0
        w[1, :32] = -1e-30
        w[2, 5] = -0.0
        w[3, :32] = 3.0e38
        w[4, 40] = 1e-39
    codes, scales = ops.quant_fp4(w.to(gpu))
    oc, os_ = oracle.quant_fp4(w.numpy())
    assert np.array_equal(np_(codes), oc)
    assert np.array_equal(np_(scales), os_)


@pytest.mark.parametrize("rows,k", [(130, 260), (2048, 7168), (7168, 2048)])
def test_quant_fp8_b128_matches_oracle(gpu, rows, k):
    w = data.weight(rows, k, seed=3 * rows + k)
    if rows == 130:
        w[129, 259] = 0.5
        w[0:128, 128:256] = 0.0  # an all-zero block: amax clamps to 1e-4
    codes, scales = ops.quant_fp8_b128(w.to(gpu))
    oc, os_ = oracle.quant_fp8_b128(w.numpy())
    assert np.array_equal(np_(scales), os_)
    assert np.array_equal(np_(codes), oc)

@pytest.mark.parametrize("rows,k", [(70, 96), (33, 32), (2304, 5120), (5120, 2304)])
def test_quant_fp8_e8m0_matches_oracle(gpu, rows, k):
    w = data.weight(rows, k, seed=rows + k)
    w[0, :32] = 0  # a block row with a zero part
    codes, scales = ops.quant_fp8_e8m0(w.to(gpu))
    oc, os_ = oracle.quant_fp8_e8m0_b32(w.numpy())
    assert np.array_equal(np_(codes), oc) and np.array_equal(np_(scales), os_)
    deq = ops.dequant_fp8(codes, scales, e8m0=True)
    assert bits_equal(np_(deq), oracle.dequant_fp8_e8m0_b32(oc, os_))



@pytest.mark.parametrize("block,pow2", [(32, True), (128, True), (128, False)])
def test_act_quant_matches_oracle(gpu, block, pow2):
    x = (data.normal((5, 1024), 1.0, seed=block) * torch.logspace(-3, 3, 1024)).to(torch.bfloat16)
    x[0, :block] = 0
    # non-finite values (the engine's rules, stbl/kernels.cu:56-63): a block holding an infinity has
    # scale +Inf, codes x / Inf and a NaN in-place form; a NaN is skipped by its block's maximum
    x[1, 3], x[2, block + 5], x[3, 2 * block] = float("inf"), float("-inf"), float("nan")
    codes, scales, deq = ops.act_quant(x.to(gpu), block, pow2, want_deq=True)
    oc, os_, od = oracle.act_quant(x.float().numpy(), block, pow2)
    assert np.array_equal(np_(scales), os_)
    assert np.array_equal(np_(codes), oc)
    assert bits_equal(np_(deq), od)


def test_stbl_act_quant_fp8_inplace(gpu):
    # the reference engine's form (stbl/kernels.cu:54-63): fp32 buffer of bf16 values, block 32
    x = (data.normal((4, 256), 3.0, seed=7)).to(torch.bfloat16).float()
    x[1, 40], x[2, 70], x[3, 100] = float("inf"), float("-inf"), float("nan")  # NaN blocks, NaN skipped
    got = ops.stbl_act_quant_fp8(x.clone().to(gpu))
    want = oracle.act_quant(x.numpy(), 32, True)[2]
    assert bits_equal(np_(got), want)


@pytest.mark.parametrize("n", [13824, 13824 + 96, 32])
def test_stbl_act_quant_fp8_inplace_fp32_scales(gpu, n):
    # any fp32 values (not only bf16 ones), blocks spread over 2^-30 .. 2^40, an all-zero block and a
    # block below the 1e-4 floor, at the engine's SwiGLU-output size and with a partial workgroup
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * np.repeat(2.0 ** rng.integers(-30, 41, n // 32), 32)).astype(np.float32)
    if n >= 96:
        x[32:64] = 0
        x[64:96] *= 1e-12
    got = ops.stbl_act_quant_fp8(torch.from_numpy(x.copy()).to(gpu))
    want = oracle.act_quant(x[None], 32, True)[2][0]
    assert bits_equal(np_(got), want)


def test_round_bf16_axpy(gpu):
    x = data.normal((5000,), 10.0, seed=8)
    got = ops.stbl_round_bf16(x.clone().to(gpu))
    assert bits_equal(np_(got), oracle.bf16_round(x.numpy()))
    y = data.normal((5000,), 1.0, seed=9)
    got = ops.stbl_axpy(y.clone().to(gpu), x.to(gpu), 1.0, 5000)
    assert bits_equal(np_(got), (y.numpy() + x.numpy()).astype(np.float32))
    got = ops.stbl_axpy(y.clone().to(gpu), x.to(gpu), 0.3, 5000)
    want = (y.double() + 0.3 * x.double()).float().numpy()  # one rounding: a fused multiply-add
    assert np.max(np.abs(np_(got) - want)) <= 1e-6 * np.max(np.abs(want))


def test_swiglu_batch(gpu):
    n, count = 2304, 3
    g = (data.normal((count * n,), 4.0, seed=10)).to(torch.bfloat16).float()
    u = (data.normal((count * n,), 4.0, seed=11)).to(torch.bfloat16).float()
    ws = [0.37, 1.0, 0.05]
    for limit in (0.0, 10.0):
        out = torch.empty(count * n, device=gpu)
        ops.stbl_swiglu_batch(out, g.to(gpu), u.to(gpu), ws, limit, n)
        want = np.concatenate([oracle.swiglu(g[j * n:(j + 1) * n].numpy(), u[j * n:(j + 1) * n].numpy(), ws[j], limit)
                               for j in range(count)])
        got = np_(out)
        # exp differs from libm's by at most an ulp, so a rare bf16 rounding may flip
        assert np.mean(got != want) < 0.01
        assert np.max(np.abs(got - want)) <= 2.0 ** -7 * np.max(np.abs(want))
