"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each oracle function is checked against (a) the golden vectors of tests/golden/golden.json, which
restate the reference's own inline known-answer tests (ref/test_kernel.py:12-57) and the closed forms
the path depends on, computed by exact rational arithmetic and brute force without the oracle, and
(b) library routines that fix the same rounding (torch's float8/bfloat16 casts, numpy float64 matrix
products). A few tests plant a plausible mistake in an oracle input and require that the golden
vectors catch it.
"""

import base64
import json
import math
import os

import numpy as np
import pytest
import torch

import oracle

G = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "golden.json")))


def hexf(s):
    return float.fromhex(s)


def b64(s, dtype):
    return np.frombuffer(base64.b64decode(s), dtype=np.dtype(dtype).newbyteorder("<")).astype(dtype)


def f32(vals):
    return np.array(vals, dtype=np.float32)


# ---- scalar codecs ---------------------------------------------------------------------------------

def test_e4m3_decode_all_codes():
    want = np.array([np.nan if v is None else hexf(v) for v in G["e4m3_table"]], np.float32)
    got = oracle.e4m3_decode(np.arange(256))
    assert np.array_equal(got, want, equal_nan=True)
    # and as torch reads float8_e4m3fn bytes
    lib = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(got, lib, equal_nan=True)


def test_e4m3_encode_golden_rne():
    for xh, code in G["e4m3_round"]:
        assert oracle.e4m3_encode(f32([hexf(xh)]))[0] == code, xh


def test_e4m3_encode_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-4, 3, 20000),
        np.linspace(-448, 448, 20001, dtype=np.float32),
        f32([0.0, -0.0, 2.0 ** -10, -(2.0 ** -10), 2.0 ** -9, 3 * 2.0 ** -11, 2.0 ** -7 * 1.0625]),
    ]).astype(np.float32)
    x = np.clip(x, -448, 448)
    got = oracle.e4m3_encode(x)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(got, want)


def test_pow2_ceil_kat():
    # ref/test_kernel.py:12-15
    for xh, wh in G["pow2_ceil"]:
        assert oracle.pow2_ceil(f32([hexf(xh)]))[0] == np.float32(hexf(wh))


def test_e2m1_table_and_codes():
    tab = oracle.e2m1_table()
    assert tab.tolist() == [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]
    assert np.array_equal(np.signbit(tab), np.arange(16) >= 8)
    for c in range(16):
        assert oracle.fp4_code(tab[c:c + 1])[0] == c


def test_fp4_round_ties_to_even():
    # ref/test_kernel.py:18-23 sweep, brute-forced in the fixture
    x, want = b64(G["fp4_round"]["x"], np.float32), b64(G["fp4_round"]["want"], np.float32)
    got = oracle.round_fp4(x)
    assert np.array_equal(got, want)


def test_e8m0_decode_matches_torch():
    got = oracle.e8m0_decode(np.arange(256))
    want = torch.arange(256, dtype=torch.uint8).view(torch.float8_e8m0fnu).float().numpy()
    assert np.array_equal(got, want, equal_nan=True)


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(100000) * 10.0 ** rng.integers(-30, 30, 100000)).astype(np.float32)
    x = np.concatenate([x, f32([0.0, -0.0, np.inf, -np.inf, 1 + 2 ** -8, 1 + 3 * 2 ** -8, 3.0e38])])
    got = oracle.bf16_round(x)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, want)


# ---- act_quant / weight quantizers ---------------------------------------------------------------

def test_act_quant_golden():
    # ref/test_kernel.py:26-35 closed form, act_quant(x, 32, "ue8m0")
    a = G["act_quant"]
    x = f32([hexf(v) for v in a["x"]]).reshape(a["rows"], a["n"])
    codes, scales, deq = oracle.act_quant(x, a["block"], True)
    assert np.array_equal(scales.ravel(), f32([hexf(v) for v in a["scales"]]))
    assert codes.ravel().tolist() == a["codes"]
    assert np.array_equal(deq.ravel(), f32([hexf(v) for v in a["deq"]]))


def test_act_quant_block128_non_pow2_matches_torch_casts():
    # scale_fmt=None path: s = amax * fp32(1/448), y = e4m3(clamp(x / s)); restated with torch casts
    rng = np.random.default_rng(2)
    x = torch.from_numpy((rng.standard_normal((4, 512)) * 3).astype(np.float32)).to(torch.bfloat16).float()
    codes, scales, _ = oracle.act_quant(x.numpy(), 128, False)
    xf = x.view(4, 4, 128)
    amax = xf.abs().amax(-1).clamp_min(1e-4)
    s = amax * torch.tensor(1.0 / 448.0, dtype=torch.float32)
    y = (xf / s.unsqueeze(-1)).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    assert np.array_equal(scales, s.numpy())
    assert np.array_equal(codes, y.view(4, 512).numpy())


def test_quant_fp4_golden():
    q = G["quant_fp4"]
    w = f32([hexf(v) for v in q["w"]]).reshape(q["rows"], q["k"])
    codes, scales = oracle.quant_fp4(w)
    assert codes.ravel().tolist() == q["codes"]
    assert scales.ravel().tolist() == q["scales"]


def test_quant_fp4_roundtrip_bound():
    # every value lands on the grid point nearest to w/s: |deq - w| <= s * half step
    w = np.random.default_rng(3).standard_normal((8, 256)).astype(np.float32) * np.float32(0.02)
    codes, scales = oracle.quant_fp4(w)
    deq = oracle.dequant_fp4(codes, scales)
    s = np.repeat(oracle.e8m0_decode(scales), 32, axis=1)
    half = np.where(np.abs(deq / s) < 2, 0.25, np.where(np.abs(deq / s) < 4, 0.5, 1.0))
    assert np.all(np.abs(deq - w) <= s * half + 1e-12)


def test_quant_fp8_b128_golden():
    q = G["quant_fp8_b128"]
    w = b64(q["w"], np.float32).reshape(q["rows"], q["k"])
    codes, scales = oracle.quant_fp8_b128(w)
    assert np.array_equal(codes.ravel(), b64(q["codes"], np.uint8))
    assert np.array_equal(scales.ravel(), b64(q["scales"], np.float32))


# ---- dequant / layouts / GEMV ----------------------------------------------------------------------

def _gemv_fp4_case():
    g = G["gemv_fp4"]
    n, k, m = g["n"], g["k"], g["m"]
    codes = np.array(g["codes"], np.uint8).reshape(n, k // 2)
    scales = np.array(g["scales"], np.uint8).reshape(n, k // 32)
    x = f32([hexf(v) for v in g["x"]]).reshape(m, k)
    y = np.array([hexf(v) for v in g["y"]]).reshape(m, n)
    return codes, scales, x, y


def test_gemv_fp4_exact_golden():
    codes, scales, x, y = _gemv_fp4_case()
    assert np.array_equal(oracle.gemv_fp4(codes, scales, x), y)  # exact: products and sums fit double
    deq = oracle.dequant_fp4(codes, scales)
    assert np.array_equal(oracle.gemm(x, deq), y)


def test_gemv_fp4_catches_swapped_nibbles():
    codes, scales, x, y = _gemv_fp4_case()
    swapped = ((codes >> 4) | (codes << 4)).astype(np.uint8)
    assert not np.array_equal(oracle.gemv_fp4(swapped, scales, x), y)


def test_gguf17_repack_and_dequant():
    codes, scales, x, y = _gemv_fp4_case()
    blocks = oracle.ocp_to_gguf17(codes, scales)
    assert blocks.ravel().tolist() == G["gguf17"]
    n, k = codes.shape[0], codes.shape[1] * 2
    assert np.array_equal(oracle.dequant_gguf17(blocks, n, k), oracle.dequant_fp4(codes, scales))


def test_e8m0_engine_decode():
    # stbl/kernels.cu:32: the byte as an fp32 exponent field. 1..254 agree with E8M0 (2^(s-127));
    # 0 and 255 are 0.0 and +Inf where E8M0 reads 2^-127 and NaN
    s = np.arange(256, dtype=np.uint8)
    got = oracle.e8m0_engine(s)
    assert got[0] == 0.0 and got[255] == np.inf and got[127] == 1.0
    assert np.array_equal(got[1:255], 2.0 ** (np.arange(1, 255) - 127.0))
    assert np.array_equal(got[1:255], oracle.e8m0_decode(s)[1:255].astype(np.float64))


def _engine_rows(rng, n, k):
    codes = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    scales = rng.integers(100, 140, (n, k // 32), dtype=np.uint8)
    x = rng.standard_normal(k).astype(np.float32)
    return codes, scales, x


def test_gemv_gguf_engine_matches_fp4_oracle_on_ordinary_scales():
    # with scale bytes 1..254 the engine's decode is E8M0's: the two restatements (block sums times
    # the scale here, scaled products in gemv_fp4) agree to double rounding
    rng = np.random.default_rng(30)
    n, k = 24, 512
    codes, scales, x = _engine_rows(rng, n, k)
    scales[0, 0], scales[1, 3] = 1, 200  # far scales; 254 would overflow gemv_fp4's fp32 products
    blocks = oracle.ocp_to_gguf17(codes, scales)
    np.testing.assert_allclose(oracle.gemv_gguf_engine(blocks, x, n, k), oracle.gemv_fp4(codes, scales, x[None])[0],
                               rtol=1e-12, atol=0)


def test_gemv_gguf_engine_edge_scale_bytes():
    # closed forms: scale byte 0 takes a block to exactly 0 (NaN if x there is infinite); 255 takes
    # it to +-Inf by the sign of the block's sum (NaN for a zero sum). A block of +1 and -0.5 codes
    # whose sum is positive must give +Inf, not the NaN that scaling each product first would give.
    n, k = 6, 64
    codes = np.full((n, k // 2), 0x22, np.uint8)  # every element +1.0
    scales = np.full((n, k // 32), 127, np.uint8)
    x = np.ones(k, np.float32)
    scales[0, :] = 0          # row 0: exactly 0
    scales[1, 1] = 255        # row 1: block sum 32 -> +Inf
    codes[2, 16:] = 0xaa      # row 2, block 1: every element -1.0 ...
    scales[2, 1] = 255        # ... -> -Inf
    codes[3, 16:] = 0x00      # row 3, block 1: zero codes times Inf -> NaN
    scales[3, 1] = 255
    codes[4, 16:] = 0x92      # row 4, block 1: +1.0 and -0.5 alternating, sum 8
    scales[4, 1] = 255
    scales[5, 1] = 0          # row 5: block 1 times 0.0, block 0 kept: 32
    xi = x.copy()
    blocks = oracle.ocp_to_gguf17(codes, scales)
    y = oracle.gemv_gguf_engine(blocks, xi, n, k)
    assert y[0] == 0.0 and y[1] == np.inf and y[2] == -np.inf and np.isnan(y[3]) and y[4] == np.inf
    assert y[5] == 32.0
    xi[40] = np.inf           # an infinite x in row 5's zero-scaled block: Inf * 1 * 0.0 = NaN
    assert np.isnan(oracle.gemv_gguf_engine(blocks, xi, n, k)[5])


def test_gemv_fp8_e8m0_engine():
    # ordinary scale bytes: the dequantized product in double; edge bytes: the closed forms above
    rng = np.random.default_rng(31)
    n, k = 64, 128
    codes = rng.integers(0, 256, (n, k), dtype=np.uint8)
    codes[(codes & 127) == 127] = 0  # no NaN codes
    scales = rng.integers(110, 140, (n // 32, k // 32), dtype=np.uint8)
    x = rng.standard_normal(k).astype(np.float32)
    want = oracle.dequant_fp8_e8m0_b32(codes, scales).astype(np.float64) @ x.astype(np.float64)
    np.testing.assert_allclose(oracle.gemv_fp8_e8m0_engine(codes, scales, x), want, rtol=1e-12, atol=1e-300)
    codes[:] = 0x38  # e4m3 1.0
    scales[:] = 127
    scales[0, 0], scales[1, 2] = 0, 255
    y = oracle.gemv_fp8_e8m0_engine(codes, scales, np.ones(k, np.float32))
    assert np.all(y[:32] == 96.0) and np.all(y[32:] == np.inf)


def test_dequant_fp4_matches_torch_formula():
    # ref/kernel.py:98-101 evaluated with torch: table[nibble] * e8m0 scale, one fp32 product
    rng = np.random.default_rng(4)
    codes = rng.integers(0, 256, (16, 64), dtype=np.uint8)
    scales = rng.integers(100, 140, (16, 4), dtype=np.uint8)
    scales[0, 0], scales[1, 1] = 0, 254
    raw = torch.from_numpy(codes)
    table = torch.tensor(oracle.e2m1_table())
    vals = torch.stack([table[(raw & 15).long()], table[(raw >> 4).long()]], -1).view(16, 128)
    sc = torch.from_numpy(scales).view(torch.float8_e8m0fnu).float()
    want = (vals.view(16, 4, 32) * sc.view(16, 4, 1)).view(16, 128).numpy()
    assert np.array_equal(oracle.dequant_fp4(codes, scales), want)


def test_dequant_fp8_matches_torch_formula():
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 256, (130, 260), dtype=np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0  # no NaN codes (the quantizer never writes them)
    scales = rng.random((2, 3)).astype(np.float32) * np.float32(0.01)
    b = torch.from_numpy(codes).view(torch.float8_e4m3fn)
    sb = torch.from_numpy(scales).repeat_interleave(128, 0)[:130].repeat_interleave(128, 1)[:, :260]
    want = (b.float() * sb).numpy()  # ref/kernel.py:89-90
    assert np.array_equal(oracle.dequant_fp8_b128(codes, scales), want)
    e8 = rng.integers(110, 130, (5, 8), dtype=np.uint8)
    c2 = codes[:130, :256]
    s2 = torch.from_numpy(e8).view(torch.float8_e8m0fnu).float().repeat_interleave(32, 0)[:130].repeat_interleave(32, 1)
    want2 = (torch.from_numpy(np.ascontiguousarray(c2)).view(torch.float8_e4m3fn).float() * s2).numpy()
    assert np.array_equal(oracle.dequant_fp8_e8m0_b32(c2, e8), want2)


def test_gemv_fp8_b128_exact_golden():
    q = G["quant_fp8_b128"]
    codes = b64(q["codes"], np.uint8).reshape(q["rows"], q["k"])
    scales = b64(q["scales"], np.float32).reshape(2, 3)
    x = b64(G["gemv_fp8_b128"]["x"], np.float32)
    y = np.array([hexf(v) for v in G["gemv_fp8_b128"]["y"]])
    got = oracle.gemv_fp8_b128(codes, scales, x)[0]
    # exact products summed in double: differs from the exact rational sum by double rounding only
    assert np.max(np.abs(got - y)) <= 1e-12 * np.max(np.abs(y))


def test_gemm_matches_numpy():
    rng = np.random.default_rng(6)
    a = rng.standard_normal((3, 100)).astype(np.float32)
    w = rng.standard_normal((7, 100)).astype(np.float32)
    want = a.astype(np.float64) @ w.astype(np.float64).T
    assert np.allclose(oracle.gemm(a, w), want, rtol=1e-13, atol=1e-13)


def test_fp8_gemm_brute_force():
    # ref/test_kernel.py:48-57: act_quant(a, 32, ue8m0) then fp8_gemm with 2^-3 weight scales
    rng = np.random.default_rng(7)
    a = torch.from_numpy(rng.standard_normal((5, 64)).astype(np.float32)).to(torch.bfloat16).float().numpy()
    b = rng.standard_normal((40, 64)).astype(np.float32)
    aq, as_, _ = oracle.act_quant(a, 32, True)
    bq = oracle.e4m3_encode(np.clip(b * 8, -448, 448))
    A = (oracle.e4m3_decode(aq).reshape(5, 2, 32) * as_[..., None]).reshape(5, 64)
    got = oracle.gemm(A, oracle.e4m3_decode(bq) * np.float32(2.0 ** -3))
    want = A.astype(np.float64) @ (oracle.e4m3_decode(bq).astype(np.float64) * 2.0 ** -3).T
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


# ---- epilogues / router ------------------------------------------------------------------------------

def test_swiglu_golden():
    for gh, uh, wh, lim, oh in G["swiglu"]:
        got = oracle.swiglu(f32([hexf(gh)]), f32([hexf(uh)]), hexf(wh), lim)[0]
        assert got == np.float32(hexf(oh)), (gh, uh)


def test_swiglu_matches_torch_silu():
    # stbl/test_kernels.py:200-207: (w * (silu(clamp(g, max=10)) * clamp(u, +-10))).to(bf16), tol 1e-2
    rng = np.random.default_rng(8)
    g = torch.from_numpy((rng.standard_normal(2304) * 4).astype(np.float32)).to(torch.bfloat16).float()
    u = torch.from_numpy((rng.standard_normal(2304) * 4).astype(np.float32)).to(torch.bfloat16).float()
    want = (0.37 * (torch.nn.functional.silu(g.clamp(max=10.0)) * u.clamp(-10, 10))).to(torch.bfloat16).float()
    got = oracle.swiglu(g.numpy(), u.numpy(), 0.37, 10.0)
    assert np.max(np.abs(got - want.numpy())) <= 1e-2 * np.max(np.abs(want.numpy()))


def test_route_golden():
    r = G["route"]
    logits = f32([hexf(v) for v in r["logits"]]).reshape(r["t"], r["e"])
    _, ids, w = oracle.route(logits, r["topk"])
    assert ids.tolist() == r["ids"]
    # the fixture's sigmoid used numpy's float32 exp, the oracle libm's expf: both faithful, so the
    # weights may differ in the last bit or two
    want = f32([[hexf(v) for v in row] for row in r["weights"]])
    assert np.allclose(w, want, rtol=4 * 2.0 ** -24, atol=0)


def test_route_bias_and_scale():
    logits = f32([[0.0, 1.0, 2.0, 3.0]])
    bias = f32([10.0, 0.0, 0.0, 0.0])
    _, ids, w = oracle.route(logits, 2, bias=bias, route_scale=2.5)
    assert ids.tolist() == [[0, 3]]  # the bias selects, the unbiased score weighs
    s = 1 / (1 + np.exp(-np.array([0.0, 3.0], np.float32)))
    assert np.allclose(w[0], s / s.sum() * 2.5, rtol=1e-6)


def test_route_score_sqrt_softplus():
    # stbl/kernels.cu:436-442: sqrt(x > 20 ? x : log1p(exp(x))), fp32; checked against float64 within
    # 2 ulp over [-30, 40], and the threshold itself: 20 takes log1p(exp), above 20 the identity
    xs = np.concatenate([np.linspace(-30, 40, 7001), [20.0, np.nextafter(np.float32(20), 30), 19.99]]).astype(np.float32)
    got = np.array([oracle.route_score(float(v), 1) for v in xs], np.float32)
    x64 = xs.astype(np.float64)
    want = np.sqrt(np.where(x64 > 20, x64, np.log1p(np.exp(x64))))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 2 * ulp)
    assert oracle.route_score(20.0, 1) == np.float32(np.sqrt(np.log1p(np.exp(20.0))))
    above = np.nextafter(np.float32(20), np.float32(30))
    assert oracle.route_score(float(above), 1) == np.sqrt(above)
    assert oracle.route_score(0.0, 0) == 0.5


def test_route_sqrt_softplus_brute_force():
    rng = np.random.default_rng(21)
    t, e, k = 3, 64, 6
    logits = (rng.standard_normal((t, e)) * 3).astype(np.float32)
    logits[1, 5] = logits[1, 9]  # an exact tie: the lower id first
    bias = (rng.standard_normal(e) * 0.1).astype(np.float32)
    sc, ids, w = oracle.route(logits, k, bias=bias, route_scale=2.5, score_fn=oracle.SCORE_SQRT_SOFTPLUS)
    for i in range(t):
        want_sc = np.array([oracle.route_score(float(v), 1) for v in logits[i]], np.float32)
        assert np.array_equal(sc[i], want_sc)
        key = want_sc + bias
        order = sorted(range(e), key=lambda j: (-key[j], j))[:k]
        assert ids[i].tolist() == order
        tot = np.float32(0)
        for j in order:
            tot = np.float32(tot + want_sc[j])
        ww = (want_sc[order] / np.float32(tot + np.float32(1e-20))) * np.float32(2.5)
        assert np.array_equal(w[i], ww.astype(np.float32))


def test_route_nan_keys_rank_last():
    # NaN logits (a NaN hidden state) give NaN keys: they rank below every number, so a token with
    # fewer numeric keys than k takes the lowest unused ids next (ties to the lower id); weights
    # that sum a NaN score come out NaN. Checked by brute force over (key or -inf, id).
    rng = np.random.default_rng(25)
    t, e, k = 3, 40, 8
    logits = rng.standard_normal((t, e)).astype(np.float32)
    logits[0, [3, 7, 11]] = np.nan           # three NaN keys among numeric ones
    logits[1, :] = np.nan
    logits[1, [30, 5, 17, 22, 9]] = [2.0, -1.0, 0.5, 0.5, 3.0]  # five numeric keys, one tie
    logits[2, :] = np.nan                    # no numeric key at all
    sc, ids, w = oracle.route(logits, k)
    for i in range(t):
        key = [(-np.float64(sc[i, j]) if not np.isnan(sc[i, j]) else np.inf, j) for j in range(e)]
        assert ids[i].tolist() == [j for _, j in sorted(key)[:k]]
    assert ids[1].tolist() == [9, 30, 17, 22, 5, 0, 1, 2]
    assert ids[2].tolist() == list(range(k))
    assert np.all(np.isfinite(w[0]))  # its 8 best keys are numeric
    assert np.all(np.isnan(w[1])) and np.all(np.isnan(w[2]))


def test_quant_fp8_e8m0_b32_properties():
    rng = np.random.default_rng(22)
    rows, k = 70, 96  # a partial last row block
    w = (rng.standard_normal((rows, k)) * 0.02).astype(np.float32)
    w[0:32, 0:32] = 0  # an all-zero block takes the 1e-4 floor
    w[32:64, 32:64] *= 1e4
    codes, sc = oracle.quant_fp8_e8m0_b32(w)
    assert sc.shape == (3, 3)
    for bi in range(3):
        for bj in range(3):
            blk = w[32 * bi:32 * bi + 32, 32 * bj:32 * bj + 32]
            t = np.float32(max(np.abs(blk).max(), np.float32(1e-4)) * np.float32(1 / 448))
            s = 2.0 ** np.ceil(np.log2(np.float64(t)))  # pow2_ceil by log2 of the fp32 value
            assert sc[bi, bj] == 127 + int(np.log2(s))
            q = np.clip(blk / np.float32(s), -448, 448).astype(np.float32)
            assert np.array_equal(codes[32 * bi:32 * bi + 32, 32 * bj:32 * bj + 32], oracle.e4m3_encode(q))
    # round trip: half an e4m3 step (2^-4 relative), or half the subnormal step 2^-9 * s
    deq = oracle.dequant_fp8_e8m0_b32(codes, sc)
    s_el = np.repeat(np.repeat(2.0 ** (sc.astype(np.int32) - 127), 32, 0)[:rows], 32, 1)
    assert np.all(np.abs(deq - w) <= np.abs(w) * 2.0 ** -4 + 2.0 ** -10 * s_el)


# ---- expert FFN / MoE composition ----------------------------------------------------------------------

def _fp4_slot(rng, dim, inter):
    parts = []
    mats = []
    for rows, k in ((inter, dim), (inter, dim), (dim, inter)):
        w = rng.standard_normal((rows, k)).astype(np.float32) * np.float32(0.02)
        c, s = oracle.quant_fp4(w)
        parts += [c.ravel(), s.ravel()]
        mats.append(oracle.dequant_fp4(c, s))
    return np.concatenate(parts), mats


def _ffn_numpy(mats, x, w, official, limit=0.0):
    """stbl/model.cu:536-539 composition with dense float64 products: g, u rounded to bf16, SwiGLU
    with the route weight (g capped at limit, u clamped to +-limit when limit > 0,
    stbl/kernels.cu:444-459), optional act_quant of the input and of the SwiGLU output, bf16 output."""
    wg, wu, wd = mats
    if official:
        x = oracle.act_quant(x[None], 32, True)[2][0]
    g = oracle.bf16_round((wg.astype(np.float64) @ x.astype(np.float64)).astype(np.float32))
    u = oracle.bf16_round((wu.astype(np.float64) @ x.astype(np.float64)).astype(np.float32))
    if limit > 0:
        g, u = np.minimum(g, np.float32(limit)), np.clip(u, -np.float32(limit), np.float32(limit))
    gt = torch.from_numpy(g)
    h = ((gt / (1 + torch.exp(-gt))) * torch.from_numpy(u) * w).to(torch.bfloat16).float().numpy()
    if official:
        h = oracle.act_quant(h[None], 32, True)[2][0]
    return oracle.bf16_round((wd.astype(np.float64) @ h.astype(np.float64)).astype(np.float32))


@pytest.mark.parametrize("official", [False, True])
def test_expert_ffn_fp4_composition(official):
    rng = np.random.default_rng(9)
    dim, inter = 256, 128
    slot, mats = _fp4_slot(rng, dim, inter)
    x = oracle.bf16_round(rng.standard_normal(dim).astype(np.float32))
    got = oracle.expert_ffn_fp4(slot, dim, inter, x, 0.7, 0.0, official)
    want = _ffn_numpy(mats, x, 0.7, official)
    # bf16 outputs of the same exact products: at most one bf16 step apart (summation order only)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-30)
    assert np.mean(got == want) > 0.9


def test_moe_fp4_sum_order():
    rng = np.random.default_rng(10)
    dim, inter, topk = 128, 64, 3
    slots = [_fp4_slot(rng, dim, inter) for _ in range(4)]
    x = oracle.bf16_round(rng.standard_normal((2, dim)).astype(np.float32))
    picks = [[0, 2, 1], [3, 0, 2]]
    wts = np.array([[0.5, 0.3, 0.2], [0.6, 0.25, 0.15]], np.float32)
    y = oracle.moe_fp4([[slots[e][0] for e in row] for row in picks], wts, slots[3][0], dim, inter, x)
    for t in range(2):
        acc = np.zeros(dim, np.float32)
        for p, e in enumerate(picks[t]):
            acc = acc + oracle.expert_ffn_fp4(slots[e][0], dim, inter, x[t], wts[t, p])
        acc = acc + oracle.expert_ffn_fp4(slots[3][0], dim, inter, x[t], 1.0)
        assert np.array_equal(y[t], oracle.bf16_round(acc))


@pytest.mark.parametrize("official", [False, True])
def test_expert_ffn_deq_equals_fp4_path(official):
    # the format-independent composition on dequantized matrices against the pinned FP4 one
    rng = np.random.default_rng(23)
    dim, inter = 256, 128
    slot, mats = _fp4_slot(rng, dim, inter)
    x = oracle.bf16_round(rng.standard_normal(dim).astype(np.float32))
    a = oracle.expert_ffn_fp4(slot, dim, inter, x, 0.7, 3.0, official)
    b = oracle.expert_ffn_deq(*mats, x, 0.7, 3.0, official)
    assert np.all(np.abs(a - b) <= np.abs(a) * 2.0 ** -7 + 1e-30)
    assert np.mean(a == b) > 0.99


def test_moe_deq_equals_fp4_path():
    rng = np.random.default_rng(24)
    dim, inter = 128, 64
    slots = [_fp4_slot(rng, dim, inter) for _ in range(4)]
    x = oracle.bf16_round(rng.standard_normal((2, dim)).astype(np.float32))
    picks = [[0, 2, 1], [3, 0, 2]]
    wts = np.array([[0.5, 0.3, 0.2], [0.6, 0.25, 0.15]], np.float32)
    a = oracle.moe_fp4([[slots[e][0] for e in row] for row in picks], wts, slots[3][0], dim, inter, x, 2.0, True)
    b = oracle.moe_deq([[slots[e][1] for e in row] for row in picks], wts, slots[3][1], x, 2.0, True)
    assert np.all(np.abs(a - b) <= np.abs(a) * 2.0 ** -7 + 1e-30)
    assert np.mean(a == b) > 0.99


def _fp8_parts(rng, dim, inter):
    """(gate, up, down) as (e4m3 codes, fp32 128x128 scales) from the oracle's quantizer, and their
    dequantized matrices. Each 128x128 block gets its own magnitude, so every block scale matters."""
    parts, mats = [], []
    for rows, k in ((inter, dim), (inter, dim), (dim, inter)):
        w = rng.standard_normal((rows, k)).astype(np.float32) * np.float32(0.02)
        gain = rng.uniform(0.25, 4.0, ((rows + 127) // 128, (k + 127) // 128)).astype(np.float32)
        w *= np.repeat(np.repeat(gain, 128, 0), 128, 1)[:rows, :k]
        c, s = oracle.quant_fp8_b128(w)
        parts.append((c, s))
        mats.append(oracle.dequant_fp8_b128(c, s))
    return parts, mats


@pytest.mark.parametrize("official,limit", [(False, 0.0), (True, 0.0), (False, 0.25), (True, 0.25)])
def test_expert_ffn_fp8_composition(official, limit):
    # orc_expert_ffn_fp8 (FP8 weights with 128x128 fp32 block scales) against the dense float64
    # composition of stbl/model.cu:536-539 on its dequantized matrices, and against the
    # format-independent composition; limit 0.25 caps g and clamps u in most rows
    rng = np.random.default_rng(31)
    dim, inter = 384, 256
    parts, mats = _fp8_parts(rng, dim, inter)
    x = oracle.bf16_round(rng.standard_normal(dim).astype(np.float32))
    got = oracle.expert_ffn_fp8(*parts, dim, inter, x, 0.7, limit, official)
    want = _ffn_numpy(mats, x, 0.7, official, limit)
    close = lambda a, b: np.abs(a - b) <= np.abs(b) * 2.0 ** -7 + 1e-30
    assert np.all(close(got, want))
    assert np.mean(got == want) > 0.9
    deq = oracle.expert_ffn_deq(*mats, x, 0.7, limit, official)
    assert np.all(close(got, deq))
    assert np.mean(got == deq) > 0.99
    # a planted mistake, gate and up passed swapped, fails that bar
    bad = oracle.expert_ffn_fp8(parts[1], parts[0], parts[2], dim, inter, x, 0.7, limit, official)
    assert np.mean(close(bad, want)) < 0.5


@pytest.mark.parametrize("official,limit", [(False, 0.0), (True, 0.0), (False, 0.25)])
def test_expert_ffn_fp8_intermediate_exact(official, limit):
    # A down matrix that dequantizes to the identity (e4m3 code 0x38 = 1.0 on the diagonal, block
    # scales 1) makes the raw output the SwiGLU intermediate itself, so it is checked bit for bit:
    # g and u each rounded to bf16, the SwiGLU of stbl/kernels.cu:444-459 with the route weight
    # (pinned on its own), and in official mode act_quant(h, 32) (stbl/model.cu:538)
    rng = np.random.default_rng(32)
    dim = inter = 256
    parts, mats = _fp8_parts(rng, dim, inter)
    eye = np.zeros((dim, inter), np.uint8)
    np.fill_diagonal(eye, 0x38)
    parts[2] = (eye, np.ones((2, 2), np.float32))
    assert np.array_equal(oracle.dequant_fp8_b128(*parts[2]), np.eye(dim, dtype=np.float32))
    x = oracle.bf16_round(rng.standard_normal(dim).astype(np.float32) * 2)
    _, h = oracle.expert_ffn_fp8(*parts, dim, inter, x, 0.7, limit, official, raw=True)
    h = h.astype(np.float32)
    xin = oracle.act_quant(x[None], 32, True)[2][0] if official else x
    gsum, usum = (m.astype(np.float64) @ xin.astype(np.float64) for m in mats[:2])
    g, u = (oracle.bf16_round(v.astype(np.float32)) for v in (gsum, usum))

    def swiglu_h(g, u, w):
        out = oracle.swiglu(g, u, w, limit)
        return oracle.act_quant(out[None], 32, True)[2][0] if official else out

    assert np.array_equal(h, swiglu_h(g, u, 0.7))
    if not official:  # (act_quant's 3-bit mantissa would hide the smaller mistakes)
        # each planted mistake changes the intermediate: g not rounded to bf16, gate and up
        # swapped, the route weight dropped
        assert np.mean(h != swiglu_h(gsum.astype(np.float32), u, 0.7)) > 0.05
        assert np.mean(h != swiglu_h(u, g, 0.7)) > 0.5
        assert np.mean(h != swiglu_h(g, u, 1.0)) > 0.5


def test_fp4_gemm_torch_matches_the_c_restatement():
    # the timed CPU baseline (ref/kernel.py:94-102's torch method) against the pinned C GEMV:
    # the same exact products in another summation order, rounded to bf16
    rng = np.random.default_rng(26)
    n, k = 96, 512
    codes = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    sc = rng.integers(118, 130, (n, k // 32), dtype=np.uint8)
    x = oracle.bf16_round(rng.standard_normal((2, k)).astype(np.float32))
    got = oracle.fp4_gemm_torch(torch.from_numpy(x), torch.from_numpy(codes), torch.from_numpy(sc)).float().numpy()
    want = oracle.gemv_fp4(codes, sc, x)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -7 + 1e-30)
    assert np.mean(got == oracle.bf16_round(want.astype(np.float32))) > 0.95


# ---- expert LRU bookkeeping ------------------------------------------------------------------------------

def test_lru_simulate_hand_case():
    # 2 slots. step 1: 1, 2 miss into slots 0, 1. step 2: 2 hit; 3 misses and evicts 1 (LRU).
    # step 3: ids 1, 3: 3 is touched first, so 1's miss evicts 2, not 3.
    out = oracle.lru_simulate([[1, 2], [2, 3], [1, 3]], 2)
    assert out[0] == ([False, False], [0, 1], [])
    assert out[1] == ([True, False], [1, 0], [1])
    assert out[2] == ([False, True], [1, 0], [2])


def test_lru_simulate_brute_force():
    rng = np.random.default_rng(11)
    steps = [list(rng.choice(12, size=3, replace=False)) for _ in range(200)]
    out = oracle.lru_simulate(steps, 5)
    last_use, cached = {}, set()
    clock = 0
    for ids, (hits, _, _) in zip(steps, out):
        clock += 1
        for e in ids:
            if e in cached:
                last_use[e] = clock  # touched before any miss of this step
        for e, hit in zip(ids, hits):
            assert hit == (e in cached)
            clock += 1
            if not hit:
                if len(cached) == 5:
                    victim = min(cached, key=lambda v: last_use[v])
                    cached.remove(victim)
                cached.add(e)
            last_use[e] = clock
