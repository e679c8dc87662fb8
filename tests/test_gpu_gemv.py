"""GPU parity of the quantized GEMVs against the oracle (ref/kernel.py:85-102, stbl/kernels.cu:92-191).

The bar: fp32 outputs within 1e-3 (max error over max output, the reference's check() metric) of the
oracle's exact-product double sum (the GPU sums in a different order, so a few ulp of fp32); bf16
outputs at most one bf16 step from bf16(oracle), with flips rare. The weights are seeded N(0, 0.02) quantized by the GPU quantizers,
which test_gpu_quant.py pins bit-exactly to the oracle's.
"""

import numpy as np
import pytest
import torch

import oracle
from stblarge_amd import data, ops
from util import assert_gemv, np_

pytestmark = pytest.mark.gpu

SHAPES = [(8, 32), (13, 96), (64, 2048), (100, 2080), (4100, 1024), (2048, 7168), (7168, 2048)]


def _fp4(gpu, rows, k, seed):
    w = data.weight(rows, k, seed)
    codes, scales = oracle.quant_fp4(w.numpy())
    return codes, scales, torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu)


def _fp8(gpu, rows, k, seed):
    w = data.weight(rows, k, seed)
    codes, scales = oracle.quant_fp8_b128(w.numpy())
    return codes, scales, torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu)


@pytest.mark.parametrize("rows,k", SHAPES)
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_gemv_fp4(gpu, rows, k, m):
    if m > 1 and rows * k > 2048 * 7168 // 4:
        m = 4 if m == 4 else 1  # full shapes: M = 1 and 4 only (oracle time)
    codes, scales, dc, ds = _fp4(gpu, rows, k, seed=rows * 31 + k)
    x = data.activation(m, k, seed=m + k)
    want = oracle.gemv_fp4(codes, scales, x.float().numpy())
    y32 = ops.gemv_fp4(dc, ds, x.to(gpu), out_f32=True)
    y16 = ops.gemv_fp4(dc, ds, x.to(gpu))
    assert tuple(y16.shape) == (m, rows) and y16.dtype == torch.bfloat16
    assert_gemv(np_(y32), np_(y16), want)


@pytest.mark.parametrize("rows,k", SHAPES)
@pytest.mark.parametrize("m", [1, 2, 4])
def test_gemv_fp8(gpu, rows, k, m):
    if m > 1 and rows * k > 2048 * 7168 // 4:
        m = 4 if m == 4 else 1
    codes, scales, dc, ds = _fp8(gpu, rows, k, seed=rows * 17 + k)
    x = data.activation(m, k, seed=2 * m + k)
    want = oracle.gemv_fp8_b128(codes, scales, x.float().numpy())
    y32 = ops.gemv_fp8(dc, ds, x.to(gpu), out_f32=True)
    y16 = ops.gemv_fp8(dc, ds, x.to(gpu))
    assert_gemv(np_(y32), np_(y16), want)


@pytest.mark.parametrize("fmt,rows,k,m", [(0, 8195, 1024, 2), (0, 8195, 1024, 3), (0, 8195, 1024, 4), (0, 4100, 2048, 4),
                                          (0, 1030, 7168, 3), (0, 514, 4096, 4), (1, 7170, 1024, 3), (1, 4100, 4096, 4),
                                          (1, 2050, 4096, 3), (1, 2050, 7168, 2), (1, 6150, 2048, 2),
                                          (0, 4102, 2048, 1), (0, 16390, 2048, 1), (0, 2046, 4096, 1), (0, 8190, 3072, 1)])
def test_gemv_multi_token_tile_heights(gpu, fmt, rows, k, m):
    # 2-4 tokens take tiles of 8, 4 or 2 rows by format, waves per row and tiles per CU; these shapes
    # reach each height with a partial last tile (8195 rows of FP4 K = 1024: 8-row tiles, 3 rows in
    # the last; 514 x 4096: 2-row tiles; 7170 x 1024 FP8: 4-row tiles; 4100 x 4096 FP8: 8-row tiles).
    # One token of FP4 rows of one wave: 4-row tiles at 4102 x 2048, 8-row ones at 16390 x 2048; of
    # two or three waves: 8-row tiles at 2046 x 4096 (one round over the CUs) and 8190 x 3072 (four)
    q = oracle.quant_fp4 if fmt == 0 else oracle.quant_fp8_b128
    ref = oracle.gemv_fp4 if fmt == 0 else oracle.gemv_fp8_b128
    run = ops.gemv_fp4 if fmt == 0 else ops.gemv_fp8
    c, sc = q(data.weight(rows, k, seed=rows + k + m).numpy())
    x = data.activation(m, k, seed=rows + m)
    want = ref(c, sc, x.float().numpy())
    dc, ds = torch.from_numpy(c).to(gpu), torch.from_numpy(sc).to(gpu)
    assert_gemv(np_(run(dc, ds, x.to(gpu), out_f32=True)), np_(run(dc, ds, x.to(gpu))), want)


@pytest.mark.parametrize("fmt,k", [(0, 16384), (1, 8192)])
@pytest.mark.parametrize("m", [1, 4])
def test_gemv_maximum_k_and_ragged_rows(gpu, fmt, k, m):
    # the largest K a launch takes (512 chunks of 32 FP4 / 16 FP8 elements: 8 waves) with row counts
    # that fill no tile: one row, and 33 (one past a 32-row scale block for FP8)
    q = oracle.quant_fp4 if fmt == 0 else oracle.quant_fp8_b128
    ref = oracle.gemv_fp4 if fmt == 0 else oracle.gemv_fp8_b128
    run = ops.gemv_fp4 if fmt == 0 else ops.gemv_fp8
    for rows in (1, 33):
        c, sc = q(data.weight(rows, k, seed=rows + k).numpy())
        x = data.activation(m, k, seed=rows + m)
        want = ref(c, sc, x.float().numpy())
        dc, ds = torch.from_numpy(c).to(gpu), torch.from_numpy(sc).to(gpu)
        assert_gemv(np_(run(dc, ds, x.to(gpu), out_f32=True)), np_(run(dc, ds, x.to(gpu))), want)


def test_gemv_official_mode(gpu):
    # the reference engine quantizes the activation first (stbl/model.cu:236-242): act_quant per 32
    # then the GEMV on the dequantized activation
    rows, k = 2048, 7168
    codes, scales, dc, ds = _fp4(gpu, rows, k, seed=5)
    x = data.activation(1, k, seed=6)
    _, _, xq = ops.act_quant(x.to(gpu), 32, True, want_deq=True)
    xo = oracle.act_quant(x.float().numpy(), 32, True)[2]
    assert np.array_equal(np_(xq), xo)
    want = oracle.gemv_fp4(codes, scales, xo)
    assert_gemv(np_(ops.gemv_fp4(dc, ds, xq, out_f32=True)), np_(ops.gemv_fp4(dc, ds, xq)), want)


def test_gemv_fp4_zero_and_extreme_inputs(gpu):
    rows, k = 64, 256
    codes, scales, dc, ds = _fp4(gpu, rows, k, seed=9)
    x = torch.zeros(1, k, dtype=torch.bfloat16)
    assert float(ops.gemv_fp4(dc, ds, x.to(gpu), out_f32=True).abs().max()) == 0.0
    x = data.activation(1, k, seed=10) * 1e30
    want = oracle.gemv_fp4(codes, scales, x.float().numpy())
    assert_gemv(np_(ops.gemv_fp4(dc, ds, x.to(gpu), out_f32=True)), None, want)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("m", [1, 4])
def test_gemv_non_finite_activations(gpu, fmt, m):
    # x with an infinity (token 0), a NaN (token 1) and both infinities (token 2): every output is
    # NaN or the same infinity exactly where the oracle's IEEE double sum puts them (an infinity
    # times a zero weight is NaN, +Inf plus -Inf is NaN), in fp32 and bf16; token 3, all finite,
    # meets the GEMV bar, so a non-finite token leaves the others alone
    rows, k = 300, 2048
    q = oracle.quant_fp4 if fmt == 0 else oracle.quant_fp8_b128
    ref = oracle.gemv_fp4 if fmt == 0 else oracle.gemv_fp8_b128
    run = ops.gemv_fp4 if fmt == 0 else ops.gemv_fp8
    codes, scales = q(data.weight(rows, k, seed=41 + fmt).numpy())
    x = data.activation(m, k, seed=42)
    x[0, 100] = float("inf")
    if m > 1:
        x[1, 5] = float("nan")
        x[2, 700], x[2, 1500] = float("-inf"), float("inf")
    with np.errstate(invalid="ignore"):
        want = ref(codes, scales, x.float().numpy())
    assert np.isinf(want[0]).any() and (np.isnan(want[0]).any() or fmt == 1)
    dc, ds = torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu)
    y32 = np_(run(dc, ds, x.to(gpu), out_f32=True)).astype(np.float64)
    y16 = np_(run(dc, ds, x.to(gpu)).float()).astype(np.float64)
    bad = slice(0, min(m, 3))
    for got in (y32, y16):
        assert np.array_equal(np.isnan(got[bad]), np.isnan(want[bad]))
        inf = np.isinf(want[bad])
        assert np.array_equal(got[bad][inf], want[bad][inf])
        assert not np.isfinite(got[bad]).any()
    if m == 4:
        assert_gemv(y32[3:], y16[3:], want[3:])


# ---- the reference engine's ABI ------------------------------------------------------------------

@pytest.mark.parametrize("rows,k,round_out", [(1000, 1280, 1), (2048, 7168, 0), (64, 96, 1),
                                               # the attention-side shapes of stbl/bench_gemv.py:103-107
                                               (32768, 1280, 1), (5120, 8192, 1), (1280, 5120, 0), (512, 5120, 1),
                                               (16388, 1280, 1), (999, 1280, 1), (2304, 5120, 1), (2560, 1280, 0),
                                               (2300, 2048, 1)])
def test_stbl_gemv_fp8_e8m0(gpu, rows, k, round_out):
    # stbl/test_kernels.py:82-98 input idiom: e4m3 weights, E8M0 scales 2^U[-14,-7] per 32x32;
    # 16388 x 1280 takes 8-row tiles, the last one half full; 999 x 1280 2-row tiles, the last one
    # half full; 64 x 96 1-row tiles; 2304 x 5120, 2560 x 1280 and 2300 x 2048 (ragged) 4-row tiles
    rng = np.random.default_rng(rows)
    w = np.clip(rng.standard_normal((rows, k)) * 100, -448, 448).astype(np.float32)
    codes = oracle.e4m3_encode(w)
    sc = rng.integers(127 - 14, 127 - 6, ((rows + 31) // 32, k // 32), dtype=np.uint8)
    x = data.activation(1, k, seed=rows).float().numpy()[0]
    xq = oracle.act_quant(x[None], 32, True)[2][0]
    want = oracle.gemm(xq[None], oracle.dequant_fp8_e8m0_b32(codes, sc))[0]
    y = torch.empty(rows, device=gpu)
    ops.stbl_gemv_fp8(y, torch.from_numpy(codes).to(gpu), torch.from_numpy(sc).to(gpu), torch.from_numpy(xq).to(gpu),
                      rows, k, round_out)
    got = np_(y)
    if round_out:
        # max |err| / max |want| of bf16-rounded outputs reaches 2^-8 from the rounding alone (half a
        # step of the largest output's binade); the reference's own bar is 1e-2 (stbl/test_kernels.py:98),
        # and the one-bf16-step check holds every element
        assert_gemv(got, got, want, tol=2.0 ** -8)
    else:
        assert_gemv(got, None, want)


@pytest.mark.parametrize("rows,k", [(512, 2560), (2048, 7168), (7168, 2048), (64, 256), (999, 2560)])
def test_stbl_gemv_mxfp4_gguf(gpu, rows, k):
    # stbl/test_kernels.py:101-117: random codes, scale bytes 118..125, repacked to GGUF blocks;
    # small matrices whose 4-row tiles would leave CUs idle take 1-row (64 x 256) or 2-row tiles
    # (999 x 2560, the last tile half full)
    rng = np.random.default_rng(k)
    codes = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
    sc = rng.integers(118, 126, (rows, k // 32), dtype=np.uint8)
    blocks = oracle.ocp_to_gguf17(codes, sc)
    x = data.activation(1, k, seed=rows).float().numpy()[0]
    want = oracle.gemv_fp4(codes, sc, x[None])[0]
    y = torch.empty(rows, device=gpu)
    ops.stbl_gemv_mxfp4(y, torch.from_numpy(blocks).to(gpu), torch.from_numpy(x).to(gpu), rows, k)
    got = np_(y)
    assert_gemv(got, got, want, tol=2.0 ** -8)


@pytest.mark.parametrize("per_cu,n,trim", [(9, 1, 4), (10, 1, 7), (9, 2, 1), (10, 1, 0)])
def test_stbl_gemv_mxfp4_one_round_tiles(gpu, per_cu, n, trim):
    # launches with 9-10 rows per CU take tiles of that many rows (one workgroup per CU; on 256 CUs
    # 9 x 256 - 4 = 2300 rows, the reference's 2304 x 5120 shape less a ragged last tile), also over
    # two matrices whose tiles must not cross from one matrix into the next
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    rows, k = (per_cu * cus + n - 1) // n - trim, 2560
    rng = np.random.default_rng(per_cu * 10 + n)
    ys, ws, xs, wants = [], [], [], []
    for j in range(n):
        codes = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
        sc = rng.integers(118, 126, (rows, k // 32), dtype=np.uint8)
        x = data.activation(1, k, seed=200 + j).float().numpy()[0]
        wants.append(oracle.gemv_fp4(codes, sc, x[None])[0])
        ws.append(torch.from_numpy(oracle.ocp_to_gguf17(codes, sc)).to(gpu))
        xs.append(torch.from_numpy(x).to(gpu))
        ys.append(torch.empty(rows, device=gpu))
    if n == 1:
        ops.stbl_gemv_mxfp4(ys[0], ws[0], xs[0], rows, k)
    else:
        ops.stbl_gemv_mxfp4_batch(ys, ws, xs, rows, k)
    for y, want in zip(ys, wants):
        assert_gemv(np_(y), np_(y), want, tol=2.0 ** -8)


@pytest.mark.parametrize("rows,k,n", [(256, 1024, 16), (2304, 5120, 12), (5120, 2304, 6), (2300, 5120, 16),
                                      (1100, 2560, 16), (40, 512, 3)])
def test_stbl_gemv_mxfp4_batch(gpu, rows, k, n):
    # small; the reference engine's V4.1 expert batches (12 gate/up, 6 down matrices), which take 16-
    # and 8-row tiles; 16-row tiles with the last one 12 rows full; 8-row tiles at K = 2560 (80 blocks
    # a row, the second wave mostly idle) with the last one 4 rows full; three 40 x 512 matrices in
    # 1-row tiles
    rng = np.random.default_rng(3)
    ys, ws, xs, wants = [], [], [], []
    for j in range(n):
        codes = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
        sc = rng.integers(118, 126, (rows, k // 32), dtype=np.uint8)
        x = data.activation(1, k, seed=100 + j).float().numpy()[0]
        wants.append(oracle.gemv_fp4(codes, sc, x[None])[0])
        ws.append(torch.from_numpy(oracle.ocp_to_gguf17(codes, sc)).to(gpu))
        xs.append(torch.from_numpy(x).to(gpu))
        ys.append(torch.empty(rows, device=gpu))
    ops.stbl_gemv_mxfp4_batch(ys, ws, xs, rows, k)
    for y, want in zip(ys, wants):
        assert_gemv(np_(y), np_(y), want, tol=2.0 ** -8)


def _quantized_x(k, seed, gain=None):
    # x as the reference engine hands it to the GGUF GEMVs: act_quant(x, 32) (stbl/model.cu:516-540),
    # e4m3 codes times a power of two per 32 elements; `gain` spreads the blocks over 2^-30..2^40
    x = data.activation(1, k, seed=seed).float().numpy()[0]
    if gain is not None:
        x = x * np.repeat(gain, 32).astype(np.float32)
    return oracle.act_quant(x[None], 32, True)[2][0]


@pytest.mark.parametrize("rows,k,n", [(2304, 5120, 1), (5120, 2304, 1), (2304, 5120, 12), (5120, 2304, 6),
                                      (2300, 5120, 16), (1100, 2560, 16), (999, 2560, 1), (40, 512, 3), (64, 256, 1)])
def test_stbl_gemv_mxfp4_quantized_x(gpu, rows, k, n):
    # x quantized as the reference engine's is (bf16-exact): the batched launches' 8- and 16-row
    # tiles take the packed-bf16 products; the reference engine's shapes and batches, 16- and 8-row
    # tiles with a partial last tile, 9-10 row one-round tiles, 2-row and 1-row tiles
    rng = np.random.default_rng(rows + k + n)
    ys, ws, xs, wants = [], [], [], []
    for j in range(n):
        codes = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
        sc = rng.integers(118, 126, (rows, k // 32), dtype=np.uint8)
        x = _quantized_x(k, 300 + j)
        wants.append(oracle.gemv_fp4(codes, sc, x[None])[0])
        ws.append(torch.from_numpy(oracle.ocp_to_gguf17(codes, sc)).to(gpu))
        xs.append(torch.from_numpy(x).to(gpu))
        ys.append(torch.empty(rows, device=gpu))
    if n == 1:
        ops.stbl_gemv_mxfp4(ys[0], ws[0], xs[0], rows, k)
    else:
        ops.stbl_gemv_mxfp4_batch(ys, ws, xs, rows, k)
    for y, want in zip(ys, wants):
        assert_gemv(np_(y), np_(y), want, tol=2.0 ** -8)


def test_stbl_gemv_mxfp4_mixed_x(gpu):
    # one launch over x that the packed-bf16 products take and x they must not: (0) quantized x whose
    # blocks span 2^-30..2^40, with zero blocks; (1) quantized x with one element moved off the bf16
    # grid, so the wave holding its block takes the fp32 products and the other waves bf16; (2) x with
    # an infinite element (every output inf or nan, as fp32 products give); (3) random fp32 x
    rows, k = 640, 5120
    rng = np.random.default_rng(17)
    gain = 2.0 ** rng.integers(-30, 41, k // 32)
    gain[[3, 90]] = 0.0
    x0 = _quantized_x(k, 400, gain)
    x1 = _quantized_x(k, 401)
    x1[70 * 32 + 5] = np.nextafter(x1[70 * 32 + 5], np.float32(np.inf))
    x2 = _quantized_x(k, 402)
    x2[2000] = np.inf
    x3 = data.activation(1, k, seed=403).float().numpy()[0]
    ys, ws, xs, want = [], [], [], []
    for j, x in enumerate((x0, x1, x2, x3)):
        codes = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
        sc = rng.integers(118, 126, (rows, k // 32), dtype=np.uint8)
        want.append(oracle.gemv_fp4(codes, sc, x[None])[0] if j != 2 else None)
        ws.append(torch.from_numpy(oracle.ocp_to_gguf17(codes, sc)).to(gpu))
        xs.append(torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(gpu))
        ys.append(torch.empty(rows, device=gpu))
    ops.stbl_gemv_mxfp4_batch(ys, ws, xs, rows, k)
    for j in (0, 1, 3):
        assert_gemv(np_(ys[j]), np_(ys[j]), want[j], tol=2.0 ** -8)
    assert not np.isfinite(np_(ys[2])).any()


def _assert_special_rows(got, want):
    # the special classes exactly (NaN where the oracle gives NaN, the same infinities), the finite
    # rows to the bf16-output bar
    assert np.array_equal(np.isnan(got), np.isnan(want)), np.nonzero(np.isnan(got) != np.isnan(want))[0][:8]
    inf = np.isinf(want)
    assert np.array_equal(got[inf], want[inf])
    fin = np.isfinite(want)
    if np.any(want[fin] != 0):
        assert_gemv(got[fin], got[fin], want[fin], tol=2.0 ** -8)
    else:  # every finite row scaled to exactly 0
        assert np.all(got[fin] == 0)


def _edge_scales(rng, shape):
    # ordinary E8M0 bytes with the engine's two special ones planted: some blocks 0 or 255, the
    # first block 255 and the last scale row all 0
    sc = rng.integers(118, 126, shape, dtype=np.uint8)
    sc[rng.random(shape) < 0.02] = 0
    sc[rng.random(shape) < 0.01] = 255
    sc[0, 0] = 255
    sc[-1] = 0
    return sc


@pytest.mark.parametrize("rows,k,n,quant", [(2304, 5120, 1, False), (5120, 2304, 1, False), (999, 2560, 1, False),
                                            (64, 256, 1, False), (2304, 5120, 12, True), (2304, 5120, 12, False),
                                            (5120, 2304, 6, True), (1100, 2560, 16, True), (300, 20480, 1, True),
                                            (64, 16640, 3, False)])
def test_stbl_gemv_mxfp4_edge_scale_bytes(gpu, rows, k, n, quant):
    # GGUF blocks with E8M0 bytes 0 and 255, in every GGUF tile (one-round 9-10 rows, 4, 2 and 1 rows,
    # the batches' 16- and 8-row tiles with the packed-bf16 and the fp32 products, and the any-K
    # kernel past 16384): the reference engine decodes byte 0 as 0.0 and 255 as +Inf times the
    # block's sum (stbl/kernels.cu:32,185; oracle.gemv_gguf_engine), so a row with a 255 block is
    # +-Inf (NaN when it also holds -+Inf, or the block's sum is 0), and a 0 block adds nothing.
    rng = np.random.default_rng(rows * 7 + n)
    ys, ws, xs, engine = [], [], [], []
    for j in range(n):
        codes = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
        sc = _edge_scales(rng, (rows, k // 32))
        codes[5, :16], sc[5, 0] = 0, 255  # row 5's first block: a zero sum times +Inf, NaN
        sc[6, :] = 0  # row 6: every block scaled to 0.0
        x = _quantized_x(k, 700 + j) if quant else data.activation(1, k, seed=700 + j).float().numpy()[0]
        blocks = oracle.ocp_to_gguf17(codes, sc)
        engine.append(oracle.gemv_gguf_engine(blocks, x, rows, k))
        ws.append(torch.from_numpy(blocks).to(gpu))
        xs.append(torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(gpu))
        ys.append(torch.empty(rows, device=gpu))
    if n == 1:
        ops.stbl_gemv_mxfp4(ys[0], ws[0], xs[0], rows, k)
    else:
        ops.stbl_gemv_mxfp4_batch(ys, ws, xs, rows, k)
    for j in range(n):
        want = engine[j]
        assert np.isnan(want[5]) and want[6] == 0 and np.isinf(want).any() and np.isfinite(want).any()
        got = np_(ys[j]).astype(np.float64)
        assert got[6] == 0
        _assert_special_rows(got, want)


@pytest.mark.parametrize("rows,k,n", [(130, 20480, 1), (37, 16640, 2), (64, 32768, 1)])
def test_stbl_gemv_mxfp4_any_k(gpu, rows, k, n):
    # rows longer than the one-pass tiles hold (16384 elements: 512 GGUF blocks) take the any-K
    # kernel, as the reference's kernel loops over K (stbl/kernels.cu:159-189); the engine's x
    # (act_quant) and random fp32 x
    rng = np.random.default_rng(k + n)
    ys, ws, xs, wants = [], [], [], []
    for j in range(n):
        codes = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
        sc = rng.integers(118, 126, (rows, k // 32), dtype=np.uint8)
        x = _quantized_x(k, 900 + j) if j % 2 == 0 else data.activation(1, k, seed=900 + j).float().numpy()[0]
        blocks = oracle.ocp_to_gguf17(codes, sc)
        wants.append(oracle.gemv_gguf_engine(blocks, x, rows, k))
        ws.append(torch.from_numpy(blocks).to(gpu))
        xs.append(torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(gpu))
        ys.append(torch.empty(rows, device=gpu))
    if n == 1:
        ops.stbl_gemv_mxfp4(ys[0], ws[0], xs[0], rows, k)
    else:
        ops.stbl_gemv_mxfp4_batch(ys, ws, xs, rows, k)
    for y, want in zip(ys, wants):
        assert_gemv(np_(y), np_(y), want, tol=2.0 ** -8)


@pytest.mark.parametrize("rows,k,round_out", [(100, 12288, 1), (70, 8224, 0), (33, 24576, 1)])
def test_stbl_gemv_fp8_any_k(gpu, rows, k, round_out):
    # FP8 E8M0 rows past 8192 elements (the one-pass tiles' 512 chunks of 16) take the any-K kernel,
    # as the reference's loops over 32-block slices (stbl/kernels.cu:104-131); engine scale bytes 0
    # and 255 planted as in the one-pass test
    rng = np.random.default_rng(rows + k)
    w = np.clip(rng.standard_normal((rows, k)) * 100, -448, 448).astype(np.float32)
    codes = oracle.e4m3_encode(w)
    sc = rng.integers(127 - 14, 127 - 6, ((rows + 31) // 32, k // 32), dtype=np.uint8)
    sc[0, 3], sc[1, 0] = 255, 0  # rows 0-31 +-Inf (one block times +Inf); rows 32-63 lose a block
    x = oracle.act_quant(data.activation(1, k, seed=k).float().numpy(), 32, True)[2][0]
    want = oracle.gemv_fp8_e8m0_engine(codes, sc, x)
    assert np.isinf(want[:32]).all() and np.isfinite(want[32:]).all()
    y = torch.empty(rows, device=gpu)
    ops.stbl_gemv_fp8(y, torch.from_numpy(codes).to(gpu), torch.from_numpy(sc).to(gpu), torch.from_numpy(x).to(gpu),
                      rows, k, round_out)
    got = np_(y).astype(np.float64)
    if round_out:
        _assert_special_rows(got, want)
    else:
        assert np.array_equal(got[:32], want[:32])
        assert_gemv(got[32:], None, want[32:])


@pytest.mark.parametrize("rows,k", [(2304, 5120), (5120, 8192), (512, 5120), (64, 96), (999, 1280)])
def test_stbl_gemv_fp8_engine_scale_bytes(gpu, rows, k):
    # the same for the FP8 E8M0 GEMV (stbl/kernels.cu:127), whose 32-wide block spans two lanes:
    # 4-, 8-, 2- and 1-row tiles
    rng = np.random.default_rng(rows + k)
    w = np.clip(rng.standard_normal((rows, k)) * 100, -448, 448).astype(np.float32)
    codes = oracle.e4m3_encode(w)
    sc = _edge_scales(rng, ((rows + 31) // 32, k // 32))
    codes[7, :32] = 0  # row 7's first block (scale byte 255): a zero sum times +Inf, NaN
    x = oracle.act_quant(data.activation(1, k, seed=k).float().numpy(), 32, True)[2][0]
    want = oracle.gemv_fp8_e8m0_engine(codes, sc, x)
    assert np.isnan(want[7]) and np.isinf(want).any() and (want == 0).any()
    y = torch.empty(rows, device=gpu)
    ops.stbl_gemv_fp8(y, torch.from_numpy(codes).to(gpu), torch.from_numpy(sc).to(gpu), torch.from_numpy(x).to(gpu),
                      rows, k, 1)
    _assert_special_rows(np_(y).astype(np.float64), want)


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("rows,k,n", [(256, 1024, 16), (2048, 7168, 3), (128, 1024, 64)])
def test_gemv_batch(gpu, fmt, rows, k, n):
    # same-shape GEMVs in one launch (stbl_gemv_mxfp4_batch's batching, v2 formats), M = 2: 16 small
    # matrices (4-row tiles for FP4, its scales as dwords from each matrix; 2-row tiles for FP8), 3
    # large ones (8-row tiles), and the largest v2 batch, 64 matrices (8-row tiles for FP4, 4 for FP8)
    m = 2
    q = oracle.quant_fp4 if fmt == 0 else oracle.quant_fp8_b128
    ref = oracle.gemv_fp4 if fmt == 0 else oracle.gemv_fp8_b128
    cs, ss, xs, wants = [], [], [], []
    for j in range(n):
        c, s = q(data.weight(rows, k, seed=500 + j).numpy())
        x = data.activation(m, k, seed=600 + j)
        wants.append(ref(c, s, x.float().numpy()))
        cs.append(torch.from_numpy(c).to(gpu))
        ss.append(torch.from_numpy(s).to(gpu))
        xs.append(x.to(gpu))
    ys = ops.gemv_batch(cs, ss, xs, fmt, out_f32=True)
    ys16 = ops.gemv_batch(cs, ss, xs, fmt)
    for y, y16, want in zip(ys, ys16, wants):
        assert_gemv(np_(y), np_(y16), want)


@pytest.mark.parametrize("fmt,rows,k", [(0, 1100, 7168), (0, 4100, 2048), (0, 5130, 2304), (1, 4102, 2048), (1, 2052, 7168)])
def test_gemv_batch_ragged_rows_eight_row_tiles(gpu, fmt, rows, k):
    # one-token batches of 16 large matrices: FP4 16 x 1100 rows at K = 7168 and 16 x 5130 at K = 2304
    # (a second wave of 8 chunks) take 16-row tiles, 16 x 4100 at K = 2048 8-row tiles; FP8 16 x 4102
    # at K = 2048 4-row tiles, 16 x 2052 at K = 7168 8-row tiles. Each row count leaves the last tile
    # partly past the matrix (1100 = 68 x 16 + 12, 5130 = 320 x 16 + 10, 4100 = 512 x 8 + 4, 4102 =
    # 1025 x 4 + 2, 2052 = 256 x 8 + 4)
    n = 16
    q = oracle.quant_fp4 if fmt == 0 else oracle.quant_fp8_b128
    ref = oracle.gemv_fp4 if fmt == 0 else oracle.gemv_fp8_b128
    cs, ss, xs, wants = [], [], [], []
    for j in range(n):
        c, s = q(data.weight(rows, k, seed=700 + j).numpy())
        x = data.activation(1, k, seed=800 + j)
        wants.append(ref(c, s, x.float().numpy()))
        cs.append(torch.from_numpy(c).to(gpu))
        ss.append(torch.from_numpy(s).to(gpu))
        xs.append(x.to(gpu))
    ys = ops.gemv_batch(cs, ss, xs, fmt, out_f32=True)
    ys16 = ops.gemv_batch(cs, ss, xs, fmt)
    for y, y16, want in zip(ys, ys16, wants):
        assert_gemv(np_(y), np_(y16), want)


@pytest.mark.parametrize("rows,k,round_out", [(256, 7168, 0), (256, 5120, 0), (100, 1001, 0), (64, 2048, 1)])
def test_stbl_gemv_f32(gpu, rows, k, round_out):
    # the router's fp32 logits GEMV (stbl/kernels.cu:206-214); the reference's own check uses 1e-5
    # (stbl/test_kernels.py:126-130). k = 1001 takes the unaligned one-float-at-a-time path.
    w = data.normal((rows, k), 0.02, seed=rows + k)
    x = data.normal((k,), 1.0, seed=k)
    want = oracle.gemm(x.numpy()[None], w.numpy())[0]
    y = torch.empty(rows, device=gpu)
    ops.stbl_gemv_f32(y, w.to(gpu), x.to(gpu), rows, k, round_out)
    got = np_(y)
    if round_out:
        assert np.array_equal(got, oracle.bf16_round(got))
        assert np.max(np.abs(got - want)) <= np.max(np.abs(want)) * (1e-5 + 2.0 ** -8)
    else:
        assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


@pytest.mark.parametrize("rows,k,round_out,group_rows", [(4096, 5120, 1, 0), (8192, 4096, 1, 1024), (100, 1001, 0, 0),
                                                         (33, 520, 0, 11), (64, 256, 0, 16)])
def test_stbl_gemv_bf16(gpu, rows, k, round_out, group_rows):
    # bf16 weights (stbl/kernels.cu:193-204): the head (4096 x 5120, stbl/bench_gemv.py:96) and the
    # block-diagonal wo_a product (8192 x 4096, groups of 1024 rows, :80-85); odd shapes take the
    # one-element path and the one-row-per-wave path (group_rows odd)
    w = data.normal((rows, k), 0.02, seed=rows + k).to(torch.bfloat16)
    xrows = (rows + group_rows - 1) // group_rows if group_rows else 1
    x = data.normal((xrows, k), 1.0, seed=k + 1)
    wf, xf = w.float().numpy(), x.numpy()
    want = np.array([oracle.gemm(xf[(r // group_rows) if group_rows else 0][None], wf[r:r + 1])[0, 0]
                     for r in range(rows)]) if rows * k <= 2 ** 20 else None
    if want is None:
        want = np.concatenate([oracle.gemm(xf[g][None], wf[g * (group_rows or rows):(g + 1) * (group_rows or rows)])[0]
                               for g in range(xrows)])
    y = torch.empty(rows, device=gpu)
    ops.stbl_gemv_bf16(y, w.to(gpu), x.to(gpu), rows, k, round_out, group_rows)
    got = np_(y)
    if round_out:
        assert np.array_equal(got, oracle.bf16_round(got))
        assert np.max(np.abs(got - want)) <= np.max(np.abs(want)) * (1e-5 + 2.0 ** -8)
    else:
        assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


def test_gemv_from_concurrent_threads_and_streams(gpu):
    # four host threads, each on its own stream, run FP4 and FP8 GEMVs of their own matrices at once;
    # every result is bit-identical to the same call made alone (the entry points keep no shared state
    # beyond a per-device CU count and per-thread error slots)
    import threading

    rows, k = 2048, 7168
    jobs = []
    for i in range(4):
        c4, s4, d4, e4 = _fp4(gpu, rows, k, seed=40 + i)
        c8, s8, d8, e8 = _fp8(gpu, rows, k, seed=50 + i)
        jobs.append((d4, e4, d8, e8, data.activation(2, k, seed=60 + i).to(gpu)))
    alone = [(ops.gemv_fp4(d4, e4, x), ops.gemv_fp8(d8, e8, x)) for d4, e4, d8, e8, x in jobs]
    torch.cuda.synchronize()
    got = [None] * 4
    errors = []

    def work(i):
        try:
            d4, e4, d8, e8, x = jobs[i]
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                out = []
                for _ in range(20):
                    out = [ops.gemv_fp4(d4, e4, x), ops.gemv_fp8(d8, e8, x)]
            s.synchronize()
            got[i] = out
        except Exception as e:  # reported below
            errors.append(repr(e))

    ts = [threading.Thread(target=work, args=(i,)) for i in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors
    for (a4, a8), (g4, g8) in zip(alone, got):
        assert torch.equal(a4, g4) and torch.equal(a8, g8)


@pytest.mark.parametrize("seed", [11, 12])
def test_random_shapes_every_gemv_entry_point(gpu, seed):
    # 40 random shapes per seed over the v2 FP4 / FP8 GEMVs (1-4 tokens, bf16 or fp32 output) and
    # the reference ABI's GGUF single / batch (fp32 or quantized x) and FP8 E8M0 GEMVs, each against
    # the oracle; every shape the entry points accept (k a multiple of the format's chunk, k % 256
    # for GGUF) picks its own tile plan
    rng = np.random.default_rng(seed)
    for t in range(40):
        kind = ("fp4", "fp8", "gguf1", "gguf_b", "fp8e8m0")[t % 5]
        rows = int(rng.integers(1, 1500))
        if kind in ("fp4", "fp8"):
            k = int(32 * rng.integers(1, 160)) if kind == "fp4" else int(16 * rng.integers(1, 320))
            m, f32 = int(rng.integers(1, 5)), bool(rng.integers(0, 2))
            w = data.weight(rows, k, seed=seed * 100 + t).numpy()
            x = data.activation(m, k, seed=seed * 100 + t + 1)
            if kind == "fp4":
                c, s = oracle.quant_fp4(w)
                want = oracle.gemv_fp4(c, s, x.float().numpy())
                got = ops.gemv_fp4(torch.from_numpy(c).to(gpu), torch.from_numpy(s).to(gpu), x.to(gpu), out_f32=f32)
            else:
                c, s = oracle.quant_fp8_b128(w)
                want = oracle.gemv_fp8_b128(c, s, x.float().numpy())
                got = ops.gemv_fp8(torch.from_numpy(c).to(gpu), torch.from_numpy(s).to(gpu), x.to(gpu), out_f32=f32)
            g = np_(got.float())
            assert_gemv(g, None if f32 else g, want, tol=1e-5 if f32 else 2.0 ** -8)
        elif kind in ("gguf1", "gguf_b"):
            k, n = int(256 * rng.integers(1, 24)), 1 if kind == "gguf1" else int(rng.integers(2, 17))
            quant = bool(rng.integers(0, 2))
            ys, ws, xs, wants = [], [], [], []
            for j in range(n):
                codes = rng.integers(0, 256, (rows, k // 2), dtype=np.uint8)
                sc = rng.integers(118, 126, (rows, k // 32), dtype=np.uint8)
                x = data.activation(1, k, seed=seed * 1000 + t * 17 + j).float().numpy()[0]
                if quant:
                    x = oracle.act_quant(x[None], 32, True)[2][0]
                wants.append(oracle.gemv_fp4(codes, sc, x[None])[0])
                ws.append(torch.from_numpy(oracle.ocp_to_gguf17(codes, sc)).to(gpu))
                xs.append(torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(gpu))
                ys.append(torch.empty(rows, device=gpu))
            if n == 1:
                ops.stbl_gemv_mxfp4(ys[0], ws[0], xs[0], rows, k)
            else:
                ops.stbl_gemv_mxfp4_batch(ys, ws, xs, rows, k)
            for j in range(n):
                assert_gemv(np_(ys[j]), np_(ys[j]), wants[j], tol=2.0 ** -8)
        else:
            k = int(32 * rng.integers(1, 256))
            w = np.clip(rng.standard_normal((rows, k)) * 100, -448, 448).astype(np.float32)
            codes = oracle.e4m3_encode(w)
            sc = rng.integers(113, 121, ((rows + 31) // 32, k // 32), dtype=np.uint8)
            x = oracle.act_quant(data.activation(1, k, seed=seed * 100 + t).float().numpy(), 32, True)[2][0]
            want = oracle.gemv_fp8_e8m0_engine(codes, sc, x)
            y = torch.empty(rows, device=gpu)
            ops.stbl_gemv_fp8(y, torch.from_numpy(codes).to(gpu), torch.from_numpy(sc).to(gpu),
                              torch.from_numpy(x).to(gpu), rows, k, 1)
            assert_gemv(np_(y), np_(y), want, tol=2.0 ** -8)


@pytest.mark.parametrize("fmt,rows,k", [(0, 2052, 7168), (1, 2060, 4096)])
@pytest.mark.parametrize("m", [2, 3, 4])
def test_gemv_multi_token_8_row_tiles(gpu, fmt, rows, k, m):
    # 2-4 tokens over FP4 rows of 4+ waves take 8-row tiles when those fill every CU (2052 x 7168: the
    # last tile holds 4 rows); FP8 rows of 4 waves take 8-row tiles at 2 tokens (2060 x 4096: 4 rows
    # in the last) and 4-row tiles at 3-4 tokens, where 8 rows would give a CU fewer than two
    q, ref = (oracle.quant_fp4, oracle.gemv_fp4) if fmt == 0 else (oracle.quant_fp8_b128, oracle.gemv_fp8_b128)
    codes, scales = q(data.weight(rows, k, seed=rows + m).numpy())
    x = data.activation(m, k, seed=k + m)
    want = ref(codes, scales, x.float().numpy())
    fn = ops.gemv_fp4 if fmt == 0 else ops.gemv_fp8
    dc, ds = torch.from_numpy(codes).to(gpu), torch.from_numpy(scales).to(gpu)
    y32 = fn(dc, ds, x.to(gpu), out_f32=True)
    y16 = fn(dc, ds, x.to(gpu))
    assert tuple(y16.shape) == (m, rows)
    assert_gemv(np_(y32), np_(y16), want)
