"""GPU parity of the multi-token GEMM (scaled f8f6f4 MFMA) against the oracle.

Oracle: act_quant(X, block, ue8m0) (ref/kernel.py:35-45) then Aq . Wdeq^T in double (ref/kernel.py:
85-102). Bar: fp32 output within 1e-3 (max error over max output, the reference's check() metric); the bf16 output is
exactly our fp32 output rounded, and within 1e-3 + one bf16 half-step by the same metric. The MFMA's internal
accumulation is not IEEE fp32 round-per-add (about 1e-4 relative on a 128-term step, measured), so
outputs near zero can be many bf16 steps from the oracle while the max-over-max error stays ~1e-4; an
elementwise ulp bar does not apply here.
"""

import numpy as np
import pytest
import torch

import oracle
from stblarge_amd import data, ops
from util import bits_equal, np_, rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("block", [32, 128])
def test_act_quant_e4m3_bit_exact(gpu, block):
    x = (data.normal((64, 7168), 1.0, seed=block) * torch.logspace(-2, 2, 7168)).to(torch.bfloat16)
    x[3, :block] = 0
    # non-finite values: a block holding an infinity takes the scale +Inf (its codes are x / Inf: 0,
    # and NaN clamped to -448 for the infinity itself); a NaN is skipped by the block's maximum and
    # clamps to -448 (fmaxf, as the engine's stbl/kernels.cu:56-63 and the oracle do)
    x[5, 10], x[6, block + 3], x[7, 2 * block + 1] = float("inf"), float("-inf"), float("nan")
    codes, sc = ops.act_quant_e4m3(x.to(gpu), block)
    oc, os_, _ = oracle.act_quant(x.float().numpy(), block, True)
    assert np.array_equal(np_(codes), oc)
    assert bits_equal((np_(sc).astype(np.uint32) << 23).view(np.float32), os_)


def _check(y32, y16, want):
    e = rel_err(y32, want)
    print(f"gemm relative error {e:.2e}")
    assert e <= 1e-3, e
    assert np.array_equal(y16, oracle.bf16_round(y32))
    assert rel_err(y16, want) <= 1e-3 + 2.0 ** -8  # bf16 half-step is up to 2^-8 relative


def _oracle_gemm(x, w_deq, block):
    oc, os_, _ = oracle.act_quant(x.float().numpy(), block, True)
    k = oc.shape[1]
    a = (oracle.e4m3_decode(oc).reshape(oc.shape[0], k // block, block) * os_[..., None]).reshape(-1, k)
    return oracle.gemm(a, w_deq)


@pytest.mark.parametrize("m,n,k", [(64, 2048, 7168), (64, 7168, 2048), (64, 2048, 6656), (16, 256, 512), (37, 200, 384)])
@pytest.mark.parametrize("block", [32, 128])
def test_gemm_fp4(gpu, m, n, k, block):
    # 64 x 2048 x 6656: 52 K steps over waves of 8, the last wave with 4
    w = data.weight(n, k, seed=n + k)
    codes, scales = oracle.quant_fp4(w.numpy())
    x = data.activation(m, k, seed=m)
    want = _oracle_gemm(x, oracle.dequant_fp4(codes, scales), block)
    dc, ds = torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu)
    y32 = np_(ops.gemm(dc, ds, x.to(gpu), ops.FP4, block, out_f32=True))
    y16 = np_(ops.gemm(dc, ds, x.to(gpu), ops.FP4, block))
    _check(y32, y16, want)


@pytest.mark.parametrize("m,n,k", [(64, 2048, 7168), (64, 7168, 2048), (16, 256, 512), (37, 200, 384)])
def test_gemm_fp8(gpu, m, n, k):
    w = data.weight(n, k, seed=3 * n + k)
    codes, scales = oracle.quant_fp8_b128(w.numpy())
    x = data.activation(m, k, seed=m + 1)
    want = _oracle_gemm(x, oracle.dequant_fp8_b128(codes, scales), 128)
    dc, ds = torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu)
    y32 = np_(ops.gemm(dc, ds, x.to(gpu), ops.FP8, 128, out_f32=True))
    y16 = np_(ops.gemm(dc, ds, x.to(gpu), ops.FP8, 128))
    _check(y32, y16, want)


@pytest.mark.parametrize("fmt", [0, 1])
def test_gemm_more_than_64_rows(gpu, fmt):
    # M = 150 runs as launches of 64, 64 and 22 rows (ref/kernel.py's GEMMs take any M): against the
    # oracle, and each 64-row block equal to a call on those rows alone, gemm and gemm_q alike
    m, n, k = 150, 1024, 2048
    w = data.weight(n, k, seed=91 + fmt)
    q, deq = (oracle.quant_fp4, oracle.dequant_fp4) if fmt == 0 else (oracle.quant_fp8_b128, oracle.dequant_fp8_b128)
    codes, scales = q(w.numpy())
    x = data.activation(m, k, seed=92)
    want = _oracle_gemm(x, deq(codes, scales), 128)
    dc, ds, xg = torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu), x.to(gpu)
    y32 = np_(ops.gemm(dc, ds, xg, fmt, 128, out_f32=True))
    _check(y32, np_(ops.gemm(dc, ds, xg, fmt, 128)), want)
    assert np.array_equal(y32[64:128], np_(ops.gemm(dc, ds, xg[64:128].contiguous(), fmt, 128, out_f32=True)))
    assert np.array_equal(y32[128:], np_(ops.gemm(dc, ds, xg[128:].contiguous(), fmt, 128, out_f32=True)))
    aq, a_s = ops.act_quant_e4m3(xg, 128)
    assert np.array_equal(np_(ops.gemm_q(dc, ds, aq, a_s, fmt, 128, out_f32=True)), y32)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("block", [32, 128])
def test_gemm_q_matches_gemm_and_oracle(gpu, fmt, block):
    # fp8_gemm(a, a_s, b, b_s) form: the activation quantized by a separate call (ref/kernel.py:85-102)
    if fmt == 1 and block == 32:
        pytest.skip("FP8 weights pair with act_block 128 in the reference configuration")
    m, n, k = 64, 2048, 7168
    w = data.weight(n, k, seed=77 + fmt)
    q = oracle.quant_fp4 if fmt == 0 else oracle.quant_fp8_b128
    codes, scales = q(w.numpy())
    deq = oracle.dequant_fp4(codes, scales) if fmt == 0 else oracle.dequant_fp8_b128(codes, scales)
    x = data.activation(m, k, seed=78)
    want = _oracle_gemm(x, deq, block)
    dc, ds = torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu)
    aq, a_s = ops.act_quant_e4m3(x.to(gpu), block)
    y32 = np_(ops.gemm_q(dc, ds, aq, a_s, fmt, block, out_f32=True))
    y16 = np_(ops.gemm_q(dc, ds, aq, a_s, fmt, block))
    _check(y32, y16, want)
    assert bits_equal(y32, np_(ops.gemm(dc, ds, x.to(gpu), fmt, block, out_f32=True)))


@pytest.mark.parametrize("which", ["act", "weight"])
def test_gemm_q_unaligned_scales(gpu, which):
    # the one-launch tile plans load scale words 16 bytes at a time; scale arrays that are not 16-byte
    # aligned take the split-K plan, which reads them byte by byte: both must match the oracle
    m, n, k = 64, 2048, 7168
    w = data.weight(n, k, seed=91)
    codes, scales = oracle.quant_fp4(w.numpy())
    x = data.activation(m, k, seed=92)
    want = _oracle_gemm(x, oracle.dequant_fp4(codes, scales), 128)
    dc, ds = torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu)
    aq, a_s = ops.act_quant_e4m3(x.to(gpu), 128)

    def shifted(t):
        buf = torch.zeros(t.numel() + 16, dtype=t.dtype, device=gpu)
        v = buf[1:1 + t.numel()].view(t.shape)
        v.copy_(t)
        return v

    a_s2, ds2 = (shifted(a_s), ds) if which == "act" else (a_s, shifted(ds))
    y32 = np_(ops.gemm_q(dc, ds2, aq, a_s2, ops.FP4, 128, out_f32=True))
    y16 = np_(ops.gemm_q(dc, ds2, aq, a_s2, ops.FP4, 128))
    _check(y32, y16, want)


def test_gemm_deterministic_and_work_reuse(gpu):
    # split-K partials are added in slice order, so repeated calls agree bit for bit; one work buffer
    # (sized for the largest shape) serves every shape
    shapes = [(64, 2048, 7168), (64, 7168, 2048), (16, 256, 512), (64, 2048, 7168)]
    work = ops.gemm_work(64, 7168, 7168, gpu)
    first = {}
    for i, (m, n, k) in enumerate(shapes * 2):
        w = data.weight(n, k, seed=n + 2 * k)
        codes, scales = oracle.quant_fp4(w.numpy())
        x = data.activation(m, k, seed=k)
        dc, ds = torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu)
        y = np_(ops.gemm(dc, ds, x.to(gpu), ops.FP4, 128, out_f32=True, work=work))
        if (m, n, k) in first:
            assert bits_equal(y, first[(m, n, k)]), (m, n, k)
        else:
            first[(m, n, k)] = y
            assert rel_err(y, _oracle_gemm(x, oracle.dequant_fp4(codes, scales), 128)) <= 1e-3


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("block", [32, 128])
@pytest.mark.parametrize("m,n,k,shift", [(16, 7168, 2048, False), (22, 7168, 2048, False), (40, 7168, 2048, False),
                                         (40, 2048, 7168, False), (64, 7168, 2048, True)])
def test_gemm_tile_plans(gpu, fmt, block, m, n, k, shift):
    # each tile plan of the GEMM against the oracle: 64 x 32 tiles in one slice (m <= 32 at N >= 6144,
    # also the 22-row tail of a 150-row call), one-launch 32 x 64 tiles with a partial second row
    # group (40 rows at 7168x2048), one-launch 16 x 32 tiles with a partial third group (40 rows at
    # 2048x7168), and two 32-row groups of 64-column tiles when the activation scales are not
    # 16-byte aligned (the one-launch plans load them 16 bytes at a time)
    w = data.weight(n, k, seed=n + k + m)
    q, deq = (oracle.quant_fp4, oracle.dequant_fp4) if fmt == 0 else (oracle.quant_fp8_b128, oracle.dequant_fp8_b128)
    codes, scales = q(w.numpy())
    x = data.activation(m, k, seed=m + 7)
    want = _oracle_gemm(x, deq(codes, scales), block)
    dc, ds = torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu)
    aq, a_s = ops.act_quant_e4m3(x.to(gpu), block)
    if shift:
        buf = torch.zeros(a_s.numel() + 16, dtype=a_s.dtype, device=gpu)
        a_s2 = buf[1:1 + a_s.numel()].view(a_s.shape)
        a_s2.copy_(a_s)
        a_s = a_s2
    y32 = np_(ops.gemm_q(dc, ds, aq, a_s, fmt, block, out_f32=True))
    y16 = np_(ops.gemm_q(dc, ds, aq, a_s, fmt, block))
    _check(y32, y16, want)


@pytest.mark.parametrize("fmt", [0, 1])
def test_gemm_non_finite_activations(gpu, fmt):
    # an infinity in a row's activations makes its block scale +Inf (E8M0 byte 255, NaN to the scaled
    # MFMA; the oracle's codes x / Inf and the infinity's own clamped code times +Inf give NaN), so
    # that row is NaN in every output, as the oracle's; a NaN is skipped by the block maximum and
    # clamps to -448 (the engine's fmaxf), so its row stays finite and meets the GEMM bar with the rest
    m, n, k = 16, 256, 512
    q, deq = (oracle.quant_fp4, oracle.dequant_fp4) if fmt == 0 else (oracle.quant_fp8_b128, oracle.dequant_fp8_b128)
    codes, scales = q(data.weight(n, k, seed=5 + fmt).numpy())
    x = data.activation(m, k, seed=6)
    x[3, 10], x[5, 20], x[7, 300] = float("inf"), float("nan"), float("-inf")
    with np.errstate(invalid="ignore"):
        want = _oracle_gemm(x, deq(codes, scales), 128)
    nan_rows = [3, 7]
    assert np.isnan(want[nan_rows]).all() and np.isfinite(np.delete(want, nan_rows, axis=0)).all()
    dc, ds, xg = torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu), x.to(gpu)
    aq, a_s = ops.act_quant_e4m3(xg, 128)
    for y32, y16 in ((np_(ops.gemm(dc, ds, xg, fmt, 128, out_f32=True)), np_(ops.gemm(dc, ds, xg, fmt, 128))),
                     (np_(ops.gemm_q(dc, ds, aq, a_s, fmt, 128, out_f32=True)), np_(ops.gemm_q(dc, ds, aq, a_s, fmt, 128)))):
        assert np.isnan(y32[nan_rows]).all() and np.isnan(y16.astype(np.float32)[nan_rows]).all()
        keep = np.delete(np.arange(m), nan_rows)
        _check(y32[keep], y16[keep], want[keep])


def _pack_reference(codes, fmt):
    # the operand-order layout, restated: per 16-column group G and 128-K step s, lane 16 g + r holds
    # bytes [16g, 16g + 16) of column 16 G + r's step (FP4: 64-byte steps; FP8: 128-byte steps in two
    # kilobyte pieces, bytes [64h + 16g, 64h + 16g + 16) in piece h)
    n, kb = codes.shape
    if fmt == 0:
        return codes.reshape(n // 16, 16, kb // 64, 4, 16).transpose(0, 2, 3, 1, 4).reshape(-1)
    return codes.reshape(n // 16, 16, kb // 128, 2, 4, 16).transpose(0, 2, 3, 4, 1, 5).reshape(-1)


@pytest.mark.parametrize("fmt,n,k", [(0, 48, 384), (1, 32, 256), (0, 2048, 7168), (1, 7168, 2048)])
def test_gemm_pack_layout(gpu, fmt, n, k):
    rng = np.random.default_rng(n + k)
    codes = rng.integers(0, 256, (n, k // 2 if fmt == 0 else k), dtype=np.uint8)
    got = np_(ops.gemm_pack(torch.from_numpy(codes).to(gpu), fmt)).reshape(-1)
    assert np.array_equal(got, _pack_reference(codes, fmt))


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("block", [32, 128])
@pytest.mark.parametrize("m,n,k,shift", [(64, 2048, 7168, False), (64, 7168, 2048, False), (40, 2048, 6656, False),
                                         (16, 7168, 2048, False), (37, 208, 384, False), (64, 7168, 2048, True),
                                         (150, 1024, 2048, False)])
def test_gemm_packed_matches_row_major(gpu, fmt, block, m, n, k, shift):
    # every tile plan (one-launch 16 x 32 and 32 x 64 tiles, 64 x 32 tiles in one slice, split K,
    # two 32-row groups for unaligned activation scales, 64-row launches) reads packed weights to the
    # same outputs bit for bit, and so against the oracle as the row-major call is checked
    if fmt == 1 and block == 32:
        pytest.skip("FP8 weights pair with act_block 128 in the reference configuration")
    w = data.weight(n, k, seed=n + k + m)
    q = oracle.quant_fp4 if fmt == 0 else oracle.quant_fp8_b128
    codes, scales = q(w.numpy())
    x = data.activation(m, k, seed=m + 3)
    dc, ds, xg = torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu), x.to(gpu)
    pk = ops.gemm_pack(dc, fmt)
    aq, a_s = ops.act_quant_e4m3(xg, block)
    if shift:
        buf = torch.zeros(a_s.numel() + 16, dtype=a_s.dtype, device=gpu)
        a_s2 = buf[1:1 + a_s.numel()].view(a_s.shape)
        a_s2.copy_(a_s)
        a_s = a_s2
    want_q = np_(ops.gemm_q(dc, ds, aq, a_s, fmt, block, out_f32=True))
    assert bits_equal(np_(ops.gemm_q_packed(pk, ds, aq, a_s, fmt, block, out_f32=True)), want_q)
    assert np.array_equal(np_(ops.gemm_q_packed(pk, ds, aq, a_s, fmt, block)), np_(ops.gemm_q(dc, ds, aq, a_s, fmt, block)))
    assert bits_equal(np_(ops.gemm_packed(pk, ds, xg, fmt, block, out_f32=True)), np_(ops.gemm(dc, ds, xg, fmt, block, out_f32=True)))
    if m == 64 and not shift:
        deq = oracle.dequant_fp4(codes, scales) if fmt == 0 else oracle.dequant_fp8_b128(codes, scales)
        assert rel_err(want_q, _oracle_gemm(x, deq, block)) <= 1e-3


def test_gemm_pack_refuses_bad_shapes(gpu):
    codes = torch.zeros((40, 64), dtype=torch.uint8, device=gpu)  # n % 16 != 0
    with pytest.raises(RuntimeError):
        ops.gemm_pack(codes, 0)
    w = torch.zeros((40, 128), dtype=torch.uint8, device=gpu)
    s = torch.zeros((40, 8), dtype=torch.uint8, device=gpu)
    aq = torch.zeros((64, 256), dtype=torch.uint8, device=gpu)
    a_s = torch.zeros((64, 2), dtype=torch.uint8, device=gpu)
    with pytest.raises(RuntimeError):
        ops.gemm_q_packed(w, s, aq, a_s, 0)
