"""GPU parity of the expert FFN, the routed MoE layer, the router and the expert cache.

Oracle: stbl_oracle.c's expert FFN / MoE composition (stbl/model.cu:505-592), router
(stbl/model.cu:444-451, sigmoid or the engine's sqrt-softplus) and oracle.lru_simulate
(stbl/model.cu:347-422, 497-507).
Bar: the unrounded down product within 1e-3 of the oracle (max error over max output); bf16 outputs at most one bf16
step from the oracle's, flips rare (an intermediate bf16 rounding of g or u may flip when the two
sums differ in their last fp32 bits). Router ids exact; route weights within a few fp32 ulps (the
sigmoid's exp is a library routine on both sides).
"""

import numpy as np
import pytest
import torch

import oracle
from stblarge_amd import _lib, data, ops
from stblarge_amd.moe import ExpertCache, MoELayer
from util import assert_gemv, assert_moe_sum, bf16_ulps, np_, read_device

pytestmark = pytest.mark.gpu


def make_expert(fmt, dim, inter, seed, gpu):
    """Seeded N(0, 0.02) gate/up/down quantized on the GPU into one slot; also the numpy parts."""
    ws = [data.weight(inter, dim, seed), data.weight(inter, dim, seed + 1), data.weight(dim, inter, seed + 2)]
    slot = ops.quant_expert(*[w.to(gpu) for w in ws], fmt)
    parts = [np_(v) for v in ops.slot_views(slot, fmt, dim, inter)]
    return slot, parts


def oracle_ffn(fmt, parts, dim, inter, x, w, limit, official):
    if fmt == ops.FP4:
        packed = np.concatenate([p.ravel() for p in parts])
        return oracle.expert_ffn_fp4(packed, dim, inter, x, w, limit, official, raw=True)
    g, u, d = (parts[0], parts[1]), (parts[2], parts[3]), (parts[4], parts[5])
    return oracle.expert_ffn_fp8(g, u, d, dim, inter, x, w, limit, official, raw=True)


@pytest.mark.parametrize("fmt", [ops.FP4, ops.FP8])
@pytest.mark.parametrize("dim,inter", [(512, 256), (7168, 2048)])
@pytest.mark.parametrize("official", [False, True])
def test_expert_ffn(gpu, fmt, dim, inter, official):
    slot, parts = make_expert(fmt, dim, inter, seed=dim + fmt, gpu=gpu)
    m = 1 if dim == 7168 else 3
    x = data.activation(m, dim, seed=7)
    w, limit = (1.0, 0.0) if dim == 7168 else (0.37, 10.0)
    y16 = np_(ops.expert_ffn(slot, x.to(gpu), fmt, dim, inter, w, limit, official))
    y32 = np_(ops.expert_ffn(slot, x.to(gpu), fmt, dim, inter, w, limit, official, out_f32=True))
    for t in range(m):
        o, raw = oracle_ffn(fmt, parts, dim, inter, x[t].float().numpy(), w, limit, official)
        assert np.array_equal(oracle.bf16_round(raw.astype(np.float32)), o)
        assert_gemv(y32[t], y16[t], raw)


@pytest.mark.parametrize("fmt,dim,inter", [(ops.FP4, 160, 96), (ops.FP4, 16384, 64), (ops.FP8, 384, 640),
                                            (ops.FP8, 8192, 128)])
def test_expert_ffn_ragged_and_maximum_dims(gpu, fmt, dim, inter):
    # dims that fill no row tile (160 = 5 x 32, 96 = 3 x 32; FP8 3 and 5 scale blocks), and the
    # largest K each GEMV of the FFN takes (gate/up over dim = 16384 FP4 / 8192 FP8 elements)
    slot, parts = make_expert(fmt, dim, inter, seed=dim + inter, gpu=gpu)
    x = data.activation(2, dim, seed=9)
    y16 = np_(ops.expert_ffn(slot, x.to(gpu), fmt, dim, inter, 0.61, 7.0, False))
    y32 = np_(ops.expert_ffn(slot, x.to(gpu), fmt, dim, inter, 0.61, 7.0, False, out_f32=True))
    for t in range(2):
        _, raw = oracle_ffn(fmt, parts, dim, inter, x[t].float().numpy(), 0.61, 7.0, False)
        assert_gemv(y32[t], y16[t], raw)


def test_expert_ffn_m4_matches_m1(gpu):
    dim, inter = 1024, 512
    slot, _ = make_expert(ops.FP4, dim, inter, seed=3, gpu=gpu)
    x = data.activation(4, dim, seed=4).to(gpu)
    y4 = ops.expert_ffn(slot, x, ops.FP4, dim, inter, out_f32=True)
    for t in range(4):
        y1 = ops.expert_ffn(slot, x[t:t + 1].contiguous(), ops.FP4, dim, inter, out_f32=True)
        assert torch.equal(y4[t], y1[0])  # same rows, same lanes, same order


@pytest.mark.parametrize("t", [1, 4])
@pytest.mark.parametrize("official", [False, True])
def test_moe_experts_fp4(gpu, t, official):
    dim, inter, topk, n = 512, 256, 4, 6
    experts = [make_expert(ops.FP4, dim, inter, seed=100 + 3 * i, gpu=gpu) for i in range(n)]
    rng = np.random.default_rng(t)
    pick = [list(rng.choice(n - 1, size=topk, replace=False)) for _ in range(t)]  # slot n-1 is the shared one
    w = rng.random((t, topk)).astype(np.float32)
    x = data.activation(t, dim, seed=9)
    y = np_(ops.moe_experts(x.to(gpu), [e[0] for e in experts], pick, w.tolist(), ops.FP4, dim, inter, shared=n - 1,
                            official=official))
    packed = [np.concatenate([p.ravel() for p in e[1]]) for e in experts]
    want = oracle.moe_fp4([[packed[i] for i in row] for row in pick], w, packed[n - 1], dim, inter, x.float().numpy(),
                          official=official)
    u = bf16_ulps(y, want)
    assert u.max() <= 1 and u.mean() < 0.02, (u.max(), u.mean())


@pytest.mark.parametrize("v41", [False, True])
def test_moe_one_token_equals_two_identical_tokens(gpu, v41):
    # one token runs the single-token kernels, the same token twice the two-token ones: every token's
    # sums use the same lanes in the same order, so the results agree bit for bit
    dim, inter, topk, n = (5120, 2304, 6, 8) if v41 else (1024, 512, 4, 6)
    sfmt = ops.FP8_E8M0 if v41 else ops.FP4
    experts = [make_expert(ops.FP4, dim, inter, seed=700 + 3 * i, gpu=gpu) for i in range(n - 1)]
    experts.append(make_expert(sfmt, dim, inter, seed=790, gpu=gpu))
    pick = [[3, 0, 5, 1, 2, 4][:topk]]
    w = [[0.3, 0.25, 0.2, 0.1, 0.1, 0.05][:topk]]
    x = data.activation(1, dim, seed=71).to(gpu)
    kw = dict(shared=n - 1, limit=10.0, official=v41, shared_fmt=sfmt)
    y1 = ops.moe_experts(x, [e[0] for e in experts], pick, w, ops.FP4, dim, inter, **kw)
    y2 = ops.moe_experts(torch.cat([x, x]), [e[0] for e in experts], pick * 2, w * 2, ops.FP4, dim, inter, **kw)
    assert torch.equal(y1[0], y2[0]) and torch.equal(y1[0], y2[1])


@pytest.mark.parametrize("fmt,dim,inter,topk,official,out_f32", [(ops.FP4, 7168, 2048, 8, False, False),
                                                                  (ops.FP4, 1024, 512, 4, True, True),
                                                                  (ops.FP8, 1024, 1024, 6, False, False),
                                                                  (ops.FP4, 2048, 1024, 15, False, True)])
def test_moe_one_token_one_call_matches_two_phases(gpu, fmt, dim, inter, topk, official, out_f32):
    # one token through one call and through the two-phase call (half the slots "ready" first, the
    # rest and the combine second): every expert output has its own rows and the combine adds them
    # in top-k order either way, so the outputs agree bit for bit (C4's 7168 x 2048 top-8 + shared,
    # also checked against the oracle; 15 + 1 experts; FP8 128x128 weights; fp32 output)
    n = topk + 2
    experts = [make_expert(fmt, dim, inter, seed=900 + 5 * i, gpu=gpu) for i in range(n)]
    slots = [e[0] for e in experts]
    rng = np.random.default_rng(topk)
    pick = [[int(v) for v in rng.choice(n - 1, size=topk, replace=False)]]
    w = [list((rng.random(topk) / topk).astype(np.float32))]
    x = data.activation(1, dim, seed=topk).to(gpu)
    kw = dict(shared=n - 1, limit=10.0, official=official, out_f32=out_f32)
    y = ops.moe_experts(x, slots, pick, w, fmt, dim, inter, **kw)
    work = torch.empty(ops.moe_work_bytes(1, topk, dim, inter), dtype=torch.uint8, device=gpu)
    y2 = torch.full_like(y, float("nan"))
    ready = [i % 2 == 0 for i in range(n)]
    for phase in (1, 2):
        ops.moe_experts(x, slots, pick, w, fmt, dim, inter, work=work, out=y2, slot_ready=ready, phase=phase, **kw)
    assert torch.equal(y, y2)
    if fmt == ops.FP4 and dim == 7168:
        packed = [np.concatenate([p.ravel() for p in e[1]]) for e in experts]
        want = oracle.moe_fp4([[packed[i] for i in pick[0]]], np.array(w, np.float32), packed[n - 1], dim, inter,
                              x.float().cpu().numpy(), limit=10.0)
        u = bf16_ulps(np_(y), want)
        assert u.max() <= 1 and u.mean() < 0.02, (u.max(), u.mean())


@pytest.mark.parametrize("dim,inter", [(1024, 512), (7168, 2048)])
def test_moe_token_classes_in_one_launch_match_one_token_calls(gpu, dim, inter):
    # four tokens whose experts take one, two and four tokens (the shared expert every token): the
    # jobs of all three classes share one gate/up and one down launch, and each token's output must
    # equal, bit for bit, a call with that token alone (one-token kernels; each token's sums use the
    # same lanes in the same order); the first shape is also checked against the oracle
    topk, n = 6, 14
    experts = [make_expert(ops.FP4, dim, inter, seed=1300 + 3 * i, gpu=gpu) for i in range(n)]
    slots = [e[0] for e in experts]
    pick = [[0, 1, 2, 3, 4, 5], [0, 1, 7, 8, 9, 10], [0, 11, 12, 6, 2, 3], [0, 7, 11, 12, 8, 9]]
    w = [[0.3, 0.2, 0.15, 0.15, 0.1, 0.1]] * 4
    x = data.activation(4, dim, seed=131).to(gpu)
    kw = dict(shared=n - 1, limit=10.0)
    y = ops.moe_experts(x, slots, pick, w, ops.FP4, dim, inter, **kw)
    for t in range(4):
        y1 = ops.moe_experts(x[t:t + 1], slots, pick[t:t + 1], w[t:t + 1], ops.FP4, dim, inter, **kw)
        assert torch.equal(y[t], y1[0]), f"token {t}"
    if dim == 1024:
        packed = [np.concatenate([p.ravel() for p in e[1]]) for e in experts]
        wn, xf = np.array(w, np.float32), x.float().cpu().numpy()
        want = oracle.moe_fp4([[packed[i] for i in row] for row in pick], wn, packed[n - 1], dim, inter, xf, limit=10.0)
        terms = np.zeros((4, dim))
        for i, row in enumerate(pick):
            for p, e in enumerate(row + [n - 1]):
                terms[i] += np.abs(oracle.expert_ffn_fp4(packed[e], dim, inter, xf[i], wn[i, p] if p < topk else 1.0,
                                                         limit=10.0))
        assert_moe_sum(np_(y), want, terms)


def test_moe_experts_shared_token_groups(gpu):
    # six tokens all routed to the same two experts: jobs of <= 4 tokens are split (4 + 2)
    dim, inter, topk = 256, 128, 2
    experts = [make_expert(ops.FP4, dim, inter, seed=200 + 3 * i, gpu=gpu) for i in range(2)]
    t = 6
    pick = [[0, 1] if i % 2 else [1, 0] for i in range(t)]
    w = np.full((t, topk), 0.5, np.float32)
    x = data.activation(t, dim, seed=11)
    y = np_(ops.moe_experts(x.to(gpu), [e[0] for e in experts], pick, w.tolist(), ops.FP4, dim, inter))
    packed = [np.concatenate([p.ravel() for p in e[1]]) for e in experts]
    want = oracle.moe_fp4([[packed[i] for i in row] for row in pick], w, None, dim, inter, x.float().numpy())
    assert bf16_ulps(y, want).max() <= 1


def test_moe_experts_maximum_tokens_and_topk(gpu):
    # the largest step a launch takes: 16 tokens x top-16 over 17 routed experts plus a shared one,
    # so most experts get 14-16 tokens (jobs of 4 + 4 + 4 + 1..4)
    dim, inter, topk, n = 256, 128, 16, 18
    experts = [make_expert(ops.FP4, dim, inter, seed=300 + 3 * i, gpu=gpu) for i in range(n)]
    rng = np.random.default_rng(16)
    t = 16
    pick = [list(rng.choice(n - 1, size=topk, replace=False)) for _ in range(t)]
    w = (rng.random((t, topk)) / topk).astype(np.float32)
    x = data.activation(t, dim, seed=13)
    y = np_(ops.moe_experts(x.to(gpu), [e[0] for e in experts], pick, w.tolist(), ops.FP4, dim, inter, shared=n - 1))
    packed = [np.concatenate([p.ravel() for p in e[1]]) for e in experts]
    want = oracle.moe_fp4([[packed[i] for i in row] for row in pick], w, packed[n - 1], dim, inter, x.float().numpy())
    u = bf16_ulps(y, want)
    assert u.max() <= 1 and u.mean() < 0.02, (u.max(), u.mean())


def deq_parts(fmt, parts):
    """(gate, up, down) dequantized fp32 from a slot's six parts."""
    out = []
    for c, sc in zip(parts[0::2], parts[1::2]):
        if fmt == ops.FP4:
            out.append(oracle.dequant_fp4(c, sc))
        elif fmt == ops.FP8:
            out.append(oracle.dequant_fp8_b128(c, sc))
        else:
            out.append(oracle.dequant_fp8_e8m0_b32(c, sc))
    return out


@pytest.mark.parametrize("fmt", [ops.FP4, ops.FP8])
@pytest.mark.parametrize("limit", [10.0, 0.0])
def test_expert_ffn_official_non_finite_inputs(gpu, fmt, limit):
    # the official numerics quantize x and h in registers with the engine's rules
    # (stbl/kernels.cu:56-63): in a token whose x holds an infinity, that block's values become
    # 0 * Inf = NaN and so do its gate and up sums; the SwiGLU clamps turn NaN into the limits
    # (fminf / fmaxf, stbl/kernels.cu:452-458), and without a limit the NaN h is left out of its
    # blocks' maxima and each NaN clamps to -448 times the smallest scale in h's act_quant. Either
    # way the token comes out finite, as the oracle's does; a NaN element of x only clamps to -448
    # times its block's scale. Every token meets the oracle's bar.
    dim, inter = 1024, 512
    slot, parts = make_expert(fmt, dim, inter, seed=333 + fmt, gpu=gpu)
    x = data.activation(3, dim, seed=334)
    x[0, 100] = float("inf")
    x[1, 200] = float("nan")
    y16 = np_(ops.expert_ffn(slot, x.to(gpu), fmt, dim, inter, 0.5, limit, True))
    y32 = np_(ops.expert_ffn(slot, x.to(gpu), fmt, dim, inter, 0.5, limit, True, out_f32=True))
    for t in range(3):
        _, raw = oracle_ffn(fmt, parts, dim, inter, x[t].float().numpy(), 0.5, limit, True)
        assert np.isfinite(raw).all()
        assert_gemv(y32[t], y16[t], raw)


@pytest.mark.parametrize("dim,inter", [(512, 256), (5120, 2304)])
@pytest.mark.parametrize("official", [False, True])
def test_expert_ffn_fp8_e8m0(gpu, dim, inter, official):
    # the reference engine's FP8 layout (E8M0 per 32x32, stbl/kernels.cu:98-103) as an expert slot
    slot, parts = make_expert(ops.FP8_E8M0, dim, inter, seed=dim + 40, gpu=gpu)
    x = data.activation(2, dim, seed=41)
    y16 = np_(ops.expert_ffn(slot, x.to(gpu), ops.FP8_E8M0, dim, inter, 0.6, 10.0, official))
    y32 = np_(ops.expert_ffn(slot, x.to(gpu), ops.FP8_E8M0, dim, inter, 0.6, 10.0, official, out_f32=True))
    mats = deq_parts(ops.FP8_E8M0, parts)
    for t in range(2):
        o, raw = oracle.expert_ffn_deq(*mats, x[t].float().numpy(), 0.6, 10.0, official, raw=True)
        assert_gemv(y32[t], y16[t], raw)


def _ffn_with_h(slot, x, fmt, dim, inter, w, limit, official, out_f32):
    """stbl_amd_expert_ffn through the C-ABI with a work buffer of the test's own, which holds the
    SwiGLU intermediates h (bf16 [m][inter], before the official act_quant) after the call."""
    m = x.shape[0]
    y = torch.empty((m, dim), dtype=torch.float32 if out_f32 else torch.bfloat16, device=x.device)
    work = torch.zeros(m * inter, dtype=torch.bfloat16, device=x.device)
    _lib.check(_lib.load().stbl_amd_expert_ffn(fmt, ops._ptr(y), ops._ptr(slot), ops._ptr(x), m, dim, inter, float(w),
                                               float(limit), int(official), int(out_f32), ops._ptr(work),
                                               ops._stream()), "expert_ffn")
    return np_(y), np_(work).reshape(m, inter)


def _h_candidates(g, u, abs_g, abs_u, w, limit):
    """Every value the SwiGLU intermediate bf16(silu(g) * u * w) may take when the gate and up sums
    carry the rounding of an fp32 accumulation in some order: each exact sum (double) moves by up to
    2^-17 of its sum of absolute terms (128 fp32 rounding units; a kernel's sum of one output passes
    through fewer than 50 fp32 additions), so it rounds to either bf16 neighbour where a rounding
    midpoint lies that close; and the product moves by 2^-20 of itself (expf is a library routine on
    either side). That worst-case band admits both neighbours for about half the elements at K = 5120
    to 7168 (a sixth at K = 256), so it only bounds where a difference may sit; the test also caps
    the elements that differ from the exact oracle's h. Returns the candidate arrays (the exact
    oracle's first)."""
    cands = [oracle.swiglu(oracle.bf16_round(g.astype(np.float32)), oracle.bf16_round(u.astype(np.float32)), w, limit)]
    for gs in (-1.0, 1.0):
        for us in (-1.0, 1.0):
            gb = oracle.bf16_round((g + gs * 2.0 ** -17 * abs_g).astype(np.float32))
            ub = oracle.bf16_round((u + us * 2.0 ** -17 * abs_u).astype(np.float32))
            for ws in (1 - 2.0 ** -20, 1 + 2.0 ** -20):
                cands.append(oracle.swiglu(gb, ub, w * ws, limit))
    return cands


# (format, dim, inter, tokens, route weight, limit, official, weight seed, x seed, x row): random
# configurations, and two that a longer randomized run found, where one gate sum lies at a bf16
# rounding midpoint (0 and 19 fp32 units from it) and the GPU's h takes the other neighbour, which
# moves a few percent of the outputs by up to 6 bf16 steps through the down product
_STAGE_CASES = [
    (ops.FP8, 256, 512, 1, 1.0, 7.0, True, 9001, 1, 0),
    (ops.FP4, 768, 384, 1, 0.5595918297767639, 0.0, False, 6203, 12, 1),
    (ops.FP4, 7168, 2048, 1, 1.0, 0.0, False, 11, 11, 0),
    (ops.FP4, 1024, 512, 4, 0.37, 7.0, True, 12, 12, 0),
    (ops.FP8, 2048, 1024, 3, 0.8, 0.0, True, 13, 13, 0),
    (ops.FP8_E8M0, 5120, 2304, 1, 1.0, 10.0, True, 14, 14, 0),
    (ops.FP8_E8M0, 768, 256, 2, 0.25, 0.0, False, 15, 15, 0),
    (ops.FP4, 512, 128, 3, 0.6, 10.0, False, 16, 16, 0),
]


@pytest.mark.parametrize("case", range(len(_STAGE_CASES)))
def test_expert_ffn_stage_by_stage(gpu, case):
    # The FFN checked one stage at a time, so that no intermediate rounding can hide in a tolerance:
    # (1) h (read from the work buffer) equals the exact oracle's h except in at most 1% of its
    # elements, each of which is one of the values the gate/up sums admit under fp32 accumulation
    # (_h_candidates: a gate sum one bf16 step over moves h by one or two steps); (2) the down product
    # of the GPU's own h (act_quant'ed as the official numerics do) meets the GEMV bar, fp32 within
    # 1e-3 and bf16 outputs at most one step from the exact product. (stbl/model.cu:516-547,
    # stbl/kernels.cu:444-464)
    fmt, dim, inter, m, w, limit, official, wseed, xseed, row = _STAGE_CASES[case]
    slot, parts = make_expert(fmt, dim, inter, seed=wseed, gpu=gpu)
    gw, uw, dw = deq_parts(fmt, parts)
    x = data.activation(max(m, row + 1), dim, seed=xseed)[row:row + m]
    y16, h = _ffn_with_h(slot, x.to(gpu), fmt, dim, inter, w, limit, official, False)
    y32, h2 = _ffn_with_h(slot, x.to(gpu), fmt, dim, inter, w, limit, official, True)
    assert np.array_equal(h, h2)
    xs = x.float().numpy()
    xb = oracle.act_quant(xs, 32, True)[2] if official else xs
    g, u = oracle.gemm(xb, gw), oracle.gemm(xb, uw)
    abs_g, abs_u = oracle.gemm(np.abs(xb), np.abs(gw)), oracle.gemm(np.abs(xb), np.abs(uw))
    cands = _h_candidates(g, u, abs_g, abs_u, w, limit)
    diff = h != cands[0]
    assert diff.mean() <= 0.01, f"{diff.mean():.4f} of h values differ from the oracle's"
    ok = np.zeros(h.shape, bool)
    for c in cands:
        ok |= h == c
    assert ok.all(), f"{int((~ok).sum())} h values outside what the gate/up sums admit"
    hq = oracle.act_quant(h, 32, True)[2] if official else h
    raw = oracle.gemm(hq, dw)
    for t in range(m):
        assert_gemv(y32[t], y16[t], raw[t])


def test_moe_experts_routed_picks_of_the_shared_slot_and_phases(gpu):
    # 16 tokens x top-16 whose picks repeat the shared slot (FP8 E8M0, the routed experts FP4): the
    # shared format's jobs, up to one per 4 of the 272 (token, pick) pairs, run in launches of their
    # own. Checked against the oracle, and the two-phase call (slots 1 and 3 "ready") against one call.
    dim, inter, topk, t = 256, 128, 16, 16
    routed = [make_expert(ops.FP4, dim, inter, seed=820 + 3 * i, gpu=gpu) for i in range(3)]
    shared = make_expert(ops.FP8_E8M0, dim, inter, seed=850, gpu=gpu)
    slots = [r[0] for r in routed] + [shared[0]]
    rng = np.random.default_rng(85)
    pick = [[int(v) for v in rng.choice([0, 1, 2, 3, 3, 3], size=topk)] for _ in range(t)]
    w = (rng.random((t, topk)) / topk).astype(np.float32)
    x = data.activation(t, dim, seed=86)
    kw = dict(shared=3, shared_fmt=ops.FP8_E8M0, limit=10.0)
    y = ops.moe_experts(x.to(gpu), slots, pick, w.tolist(), ops.FP4, dim, inter, **kw)
    mats = [deq_parts(ops.FP4, r[1]) for r in routed] + [deq_parts(ops.FP8_E8M0, shared[1])]
    want = oracle.moe_deq([[mats[i] for i in row] for row in pick], w, mats[3], x.float().numpy(), limit=10.0)
    u = bf16_ulps(np_(y), want)
    assert u.max() <= 1 and u.mean() < 0.02, (u.max(), u.mean())
    ready = [False, True, False, True]
    work = torch.empty(ops.moe_work_bytes(t, topk, dim, inter), dtype=torch.uint8, device=gpu)
    y2 = torch.full((t, dim), float("nan"), dtype=torch.bfloat16, device=gpu)
    for phase in (1, 2):
        ops.moe_experts(x.to(gpu), slots, pick, w.tolist(), ops.FP4, dim, inter, work=work, out=y2, slot_ready=ready,
                        phase=phase, **kw)
    assert torch.equal(y, y2)


@pytest.mark.parametrize("t", [1, 4])
def test_moe_v41_semantics(gpu, t):
    # the reference engine's MoE at V4.1 shapes (stbl/bench_gemv.py:15): dim 5120, inter 2304, top-6,
    # FP4 routed experts + an FP8 E8M0 shared expert, official numerics (act_quant of x and of the
    # SwiGLU output, stbl/model.cu:510,538), sqrt-softplus router with bias, SwiGLU limit 10
    dim, inter, topk, n = 5120, 2304, 6, 8
    experts = [make_expert(ops.FP4, dim, inter, seed=400 + 3 * i, gpu=gpu) for i in range(n)]
    shared = make_expert(ops.FP8_E8M0, dim, inter, seed=490, gpu=gpu)
    logits = data.zipf_logits(t, n, seed=43) * 2
    bias = data.normal((n,), 0.05, seed=44)
    ids, w = ops.route(logits.to(gpu), topk, bias.to(gpu), route_scale=2.5, score_fn=ops.SCORE_SQRT_SOFTPLUS)
    _, oids, ow = oracle.route(logits.numpy(), topk, bias.numpy(), 2.5, score_fn=oracle.SCORE_SQRT_SOFTPLUS)
    assert np_(ids).tolist() == oids.tolist()
    assert np.allclose(np_(w), ow, rtol=8 * 2.0 ** -24, atol=0)
    x = data.activation(t, dim, seed=45)
    slots = [e[0] for e in experts] + [shared[0]]
    y = np_(ops.moe_experts(x.to(gpu), slots, oids.tolist(), ow.tolist(), ops.FP4, dim, inter, shared=n, limit=10.0,
                            official=True, shared_fmt=ops.FP8_E8M0))
    mats = [deq_parts(ops.FP4, e[1]) for e in experts]
    want = oracle.moe_deq([[mats[i] for i in row] for row in oids], ow, deq_parts(ops.FP8_E8M0, shared[1]),
                          x.float().numpy(), limit=10.0, official=True)
    u = bf16_ulps(y, want)
    assert u.max() <= 1 and u.mean() < 0.02, (u.max(), u.mean())


def test_route_sqrt_softplus(gpu):
    t, e, topk = 4, 256, 6
    logits = data.zipf_logits(t, e, seed=15) * 4  # spans both sides of the softplus threshold (20)
    bias = data.normal((e,), 0.01, seed=16)
    ids, w, sc = ops.route(logits.to(gpu), topk, bias.to(gpu), route_scale=2.5, want_scores=True,
                           score_fn=ops.SCORE_SQRT_SOFTPLUS)
    osc, oids, ow = oracle.route(logits.numpy(), topk, bias.numpy(), 2.5, score_fn=oracle.SCORE_SQRT_SOFTPLUS)
    assert np_(ids).tolist() == oids.tolist()
    # scores at the reference's own bar for this kernel, max |d| <= 1e-6 max |score|
    # (stbl/test_kernels.py:208-211, the check metric of :47-52): for logits near -30 the device's
    # expf differs from the host's by ~10 ulp of a value ~1e-13, invisible next to the selected scores
    assert np.max(np.abs(np_(sc) - osc)) <= 1e-6 * np.max(np.abs(osc))
    assert np.allclose(np_(w), ow, rtol=8 * 2.0 ** -24, atol=0)


def test_route_scores_over_the_logit_range(gpu):
    # both score functions at 4001 logits over fp32's whole exp range [-87, 87]: the device scores
    # within 3 fp32 ulps of the oracle's (host libm, within 1 ulp of exact; the device's are within
    # 1.6). The library is built so that the compiler's expf / log1pf expansions keep their range
    # reduction as written; with x * log2(e) - n fused into one FMA the device sigmoid was 43 ulps
    # off at |logit| ~ 70 and 5 ulps within |logit| < 10
    lg = torch.linspace(-87, 87, 4001)
    for fn in (ops.SCORE_SIGMOID, ops.SCORE_SQRT_SOFTPLUS):
        _, _, sc = ops.route(lg[:, None].contiguous().to(gpu), 1, want_scores=True, score_fn=fn)
        osc, _, _ = oracle.route(lg[:, None].numpy(), 1, score_fn=fn)
        got, want = np_(sc)[:, 0], osc[:, 0]
        ulps = np.abs(got.astype(np.float64) - want) / np.spacing(np.abs(want)).astype(np.float64)
        assert ulps.max() <= 3, f"score_fn {fn}: {ulps.max():.1f} ulps at logit {float(lg[int(ulps.argmax())])}"


def test_stbl_sqrt_softplus(gpu):
    # the reference ABI's in-place scores (stbl/test_kernels.py:208-211: 384 values of N(0, 8), bar
    # 1e-6 of max |want|); also bit-identical to the scores stbl_amd_route reports for the same logits
    score = lambda v: np.array([oracle.route_score(float(x), oracle.SCORE_SQRT_SOFTPLUS) for x in v], np.float32)
    s = data.normal((384,), 8.0, seed=21)
    got = ops.stbl_sqrt_softplus(s.clone().to(gpu))
    want = score(s.numpy())
    assert np.max(np.abs(np_(got) - want)) <= 1e-6 * np.max(np.abs(want))
    _, _, sc = ops.route(s.view(1, 384).to(gpu), 6, want_scores=True, score_fn=ops.SCORE_SQRT_SOFTPLUS)
    assert np.array_equal(np_(sc).ravel().view(np.uint32), np_(got).view(np.uint32))
    edge = torch.tensor([-200.0, -30.0, 0.0, 19.999, 20.0, 20.001, 88.0, 1e30], dtype=torch.float32)
    got = np_(ops.stbl_sqrt_softplus(edge.clone().to(gpu)))
    want = score(edge.numpy())
    assert np.all(np.abs(got - want) <= 1e-6 * np.maximum(np.abs(want), 1.0))


def test_route(gpu):
    t, e, topk = 4, 256, 8
    logits = data.zipf_logits(t, e, seed=5)
    bias = data.normal((e,), 0.01, seed=6)
    ids, w = ops.route(logits.to(gpu), topk, bias.to(gpu), route_scale=2.5)
    _, oids, ow = oracle.route(logits.numpy(), topk, bias.numpy(), 2.5)
    assert np_(ids).tolist() == oids.tolist()
    assert np.allclose(np_(w), ow, rtol=8 * 2.0 ** -24, atol=0)
    tie = torch.zeros(2, e)
    ids, w = ops.route(tie.to(gpu), topk)
    assert np_(ids).tolist() == [list(range(topk))] * 2
    assert np.allclose(np_(w), 1.0 / topk)


# ---- expert cache ------------------------------------------------------------------------------------

def pinned_pool(n_experts, slot_bytes):
    pool = torch.empty(n_experts * slot_bytes, dtype=torch.uint8, pin_memory=True)
    view = pool.view(n_experts, slot_bytes)
    for e in range(n_experts):
        view[e].fill_(e + 1)
        view[e, :4] = torch.tensor([e, 255 - e, 7, 9], dtype=torch.uint8)
    return pool


def test_cache_lru_matches_oracle(gpu):
    n, slots, sb = 40, 6, 4096
    pool = pinned_pool(n, sb)
    cache = ExpertCache(slots, sb, pool, n)
    rng = np.random.default_rng(0)
    steps = [list(rng.choice(n, size=4, replace=False)) for _ in range(200)]
    want = oracle.lru_simulate(steps, slots)
    for ids, (hits, where, _) in zip(steps, want):
        ptrs, got_hits, nmiss = cache.lookup(ids)
        assert got_hits == hits
        assert nmiss == hits.count(False)
        cache.mark_used()
        torch.cuda.synchronize()
        for e, p in zip(ids, ptrs):
            assert read_device(p, 8).tolist()[:4] == [e, 255 - e, 7, 9]
    st = cache.stats()
    assert st["hits"] + st["misses"] == 800 and st["in_use"] == slots
    assert st["refill_bytes"] == st["misses"] * sb
    cache.close()


def test_cache_lru_random_configurations(gpu):
    # 10 random caches (2-199 experts, 1-48 slots, 1-16 distinct ids a lookup, uniform or Zipf(1.1)
    # picks, 200 lookups each): hits equal oracle.lru_simulate's (stbl/model.cu:347-422) and every
    # looked-up slot holds its expert's bytes
    rng = np.random.default_rng(3)
    for case in range(10):
        n, slots, sb = int(rng.integers(2, 200)), int(rng.integers(1, 49)), 256 * int(rng.integers(16, 64))
        width = int(rng.integers(1, min(slots, n, 16) + 1))
        p = None
        if case % 2:
            p = 1.0 / np.arange(1, n + 1) ** 1.1
            p /= p.sum()
        steps = [[int(v) for v in rng.choice(n, size=int(rng.integers(1, width + 1)), replace=False, p=p)]
                 for _ in range(200)]
        cache = ExpertCache(slots, sb, pinned_pool(n, sb), n)
        for si, (ids, (hits, _, _)) in enumerate(zip(steps, oracle.lru_simulate(steps, slots))):
            ptrs, got_hits, nmiss = cache.lookup(ids)
            cache.mark_used()
            torch.cuda.synchronize()
            assert list(got_hits) == hits and nmiss == hits.count(False), f"case {case} step {si}"
            for e, q in zip(ids, ptrs):
                assert read_device(q, 8).tolist()[:4] == [e, 255 - e, 7, 9], f"case {case} step {si} expert {e}"
        st = cache.stats()
        assert st["hits"] + st["misses"] == sum(len(s) for s in steps)
        cache.close()


def test_cache_lookup_begin_end(gpu):
    # the lookup in two calls: begin maps and queues the refills and says which slots may be read at
    # once (pool tier: the hits), end makes the compute stream wait for the refills
    n, slots, sb = 12, 4, 4096
    cache = ExpertCache(slots, sb, pinned_pool(n, sb), n)
    ptrs, hits, ready, nmiss = cache.lookup_begin([0, 1])
    assert hits == [False, False] and ready == [False, False] and nmiss == 2
    with pytest.raises(Exception, match="not ended"):
        cache.lookup_begin([2])
    cache.lookup_end()
    cache.lookup_end()  # nothing open: a no-op
    cache.mark_used()
    ptrs, hits, ready, nmiss = cache.lookup_begin([1, 2, 0])
    assert hits == [True, False, True] and ready == hits and nmiss == 1
    cache.lookup_end()
    cache.mark_used()
    torch.cuda.synchronize()
    for e, p in zip([1, 2, 0], ptrs):
        assert read_device(p, 8).tolist()[:4] == [e, 255 - e, 7, 9]
    # lookahead counters (stbl/model.cu:452-460): guesses 3 and 5 are uncached when noted, 0 cached
    cache.note_guesses([3, 0, 5], layer=0)
    cache.lookup([5, 6, 0])  # 5: a cold guess, routed, a miss; 6: an unguessed miss; 0: a hit
    cache.mark_used()
    assert cache.lookahead() == {"cold_guesses": 2, "cold_guesses_routed": 1, "misses": 2, "misses_guessed": 1}
    cache.lookup([7])  # no guesses noted for this lookup: nothing counted
    cache.mark_used()
    assert cache.lookahead()["misses"] == 2
    cache.close()


def check_route(gids, gw, scores, oids, ow, bias):
    """Device router output against the oracle's. The scores' exp / log1p are library routines on
    either side and may differ in the last fp32 bit, so where the ids differ the two keys (score +
    bias, as the oracle computes them) must be a near tie, within 4 fp32 ulps: an equal pair in the
    other order, or the other one of a tie at the k-th place. Every other id matches exactly, and
    where the ids match the weights are within 8 fp32 ulps of the row's largest weight (NaN where
    the oracle's are)."""
    key = (scores + (bias if bias is not None else np.float32(0))).astype(np.float32)
    for r in range(gids.shape[0]):
        for j in np.nonzero(gids[r] != oids[r])[0]:
            a, b = key[r, gids[r, j]], key[r, oids[r, j]]
            assert abs(float(a) - float(b)) <= 4 * float(np.spacing(np.float32(max(abs(a), abs(b))))), \
                f"row {r} place {j}: id {gids[r, j]} (key {a}) against {oids[r, j]} (key {b})"
    same = gids == oids
    assert np.array_equal(np.isnan(gw)[same], np.isnan(ow)[same])
    tol = 8 * 2.0 ** -24 * np.nanmax(np.abs(ow), axis=1, keepdims=True, initial=0)
    fin = same & ~np.isnan(ow)
    assert np.all(np.abs(gw - ow)[fin] <= np.broadcast_to(tol, ow.shape)[fin])


def test_route_random(gpu):
    # 300 random routers (stbl/model.cu:430-452): 1-32 tokens, 1-1024 experts, top-1..32, both score
    # functions, bias or none, route scales; logits normal, quantized to quarters (ties), 5% NaN with
    # 2% +Inf and 2% -Inf, or far in the tails (saturated sigmoids, softplus past its threshold) --
    # checked by check_route
    rng = np.random.default_rng(31337)
    for case in range(300):
        t, e = int(rng.integers(1, 33)), int(rng.integers(1, 1025))
        topk, fn = int(rng.integers(1, min(32, e) + 1)), int(rng.integers(0, 2))
        scale = float(rng.choice([1.0, 2.5, 0.3]))
        lg = rng.normal(0, float(rng.choice([0.5, 3.0, 12.0])), (t, e)).astype(np.float32)
        if case % 4 == 1:
            lg = np.round(lg * 4) / 4
        elif case % 4 == 2:
            lg[rng.random((t, e)) < 0.05] = np.nan
            lg[rng.random((t, e)) < 0.02] = np.inf
            lg[rng.random((t, e)) < 0.02] = -np.inf
        elif case % 4 == 3:
            lg = lg * np.float32(10)
        bias = rng.normal(0, 0.01, e).astype(np.float32) if rng.random() < 0.5 else None
        ids, w = ops.route(torch.from_numpy(lg).to(gpu), topk, None if bias is None else torch.from_numpy(bias).to(gpu),
                           route_scale=scale, score_fn=fn)
        sc, oids, ow = oracle.route(lg, topk, bias, scale, score_fn=fn)
        check_route(np_(ids), np_(w), sc, oids, ow, bias)


def test_route_nan_logits(gpu):
    # NaN keys rank below every number (the oracle's rule): a token with fewer than k numeric keys
    # takes the lowest unused ids next, and NaN scores make its weights NaN
    t, e, topk = 3, 64, 8
    logits = data.zipf_logits(t, e, seed=19)
    logits[0, [3, 7, 11]] = float("nan")
    logits[1, :] = float("nan")
    logits[1, [30, 5, 17, 22, 9]] = torch.tensor([2.0, -1.0, 0.5, 0.5, 3.0])
    logits[2, :] = float("nan")
    ids, w = ops.route(logits.to(gpu), topk)
    _, oids, ow = oracle.route(logits.numpy(), topk)
    assert np_(ids).tolist() == oids.tolist()
    assert np_(ids)[2].tolist() == list(range(topk))
    got = np_(w)
    assert np.array_equal(np.isnan(got), np.isnan(ow)) and np.all(np.isnan(got[1:]))
    assert np.allclose(got[0], ow[0], rtol=8 * 2.0 ** -24, atol=0)


def test_cache_refill_failure_leaves_slot_unmapped(gpu):
    n, slots, sb = 10, 3, 4096
    cache = ExpertCache(slots, sb, pinned_pool(n, sb), n)
    cache.lookup([0, 1])
    cache.fail_refill_after(0)  # the next refill fails on the host
    with pytest.raises(Exception):
        cache.lookup([2])
    assert cache.peek(2) is None
    ptrs, hits, nmiss = cache.lookup([2])  # retried: misses again, now succeeds
    assert hits == [False] and nmiss == 1 and cache.peek(2) == ptrs[0]
    with pytest.raises(Exception):
        cache.lookup([3, 4, 5, 6])  # more experts than slots in one lookup
    cache.close()


def test_moe_layer_phase1_failure_ends_the_lookup(gpu, monkeypatch):
    # a step whose first phase (the resident experts) raises must still end the cache's open
    # lookup: the error reaches the caller and the next step's lookup and result are normal
    dim, inter, n, topk, slots = 256, 128, 8, 2, 4
    fmt = ops.FP4
    slot_bytes, _ = ops.expert_layout(fmt, dim, inter)
    pool = torch.empty(n * slot_bytes, dtype=torch.uint8, pin_memory=True)
    packed = []
    for e in range(n):
        s, parts = make_expert(fmt, dim, inter, seed=500 + 3 * e, gpu=gpu)
        pool[e * slot_bytes:(e + 1) * slot_bytes].copy_(s.cpu())
        packed.append(np.concatenate([p.ravel() for p in parts]))
    layer = MoELayer(fmt, dim, inter, pool, n, topk, slots)
    x = data.activation(1, dim, seed=5).to(gpu)
    layer.forward(x, None, route=([[0, 1]], [[0.5, 0.5]]))  # experts 0 and 1 resident
    real = ops.moe_experts

    def failing(*a, phase=0, **kw):
        if phase == 1:
            raise RuntimeError("planted phase-1 failure")
        return real(*a, phase=phase, **kw)

    monkeypatch.setattr(ops, "moe_experts", failing)
    with pytest.raises(RuntimeError, match="planted"):
        layer.forward(x, None, route=([[0, 2]], [[0.5, 0.5]]))  # 0 resident, 2 refilled: two phases
    monkeypatch.setattr(ops, "moe_experts", real)
    y = np_(layer.forward(x, None, route=([[3, 0]], [[0.75, 0.25]])))
    want = oracle.moe_fp4([[packed[3], packed[0]]], [[0.75, 0.25]], None, dim, inter, x.float().cpu().numpy())
    assert bf16_ulps(y, want).max() <= 1
    layer.close()


def test_moe_layer_end_to_end(gpu):
    dim, inter, n, topk, slots = 256, 128, 24, 3, 12  # <= 12 distinct experts per 4-token step
    fmt = ops.FP4
    slot_bytes, _ = ops.expert_layout(fmt, dim, inter)
    pool = torch.empty(n * slot_bytes, dtype=torch.uint8, pin_memory=True)
    packed = []
    for e in range(n):
        s, parts = make_expert(fmt, dim, inter, seed=300 + 3 * e, gpu=gpu)
        pool[e * slot_bytes:(e + 1) * slot_bytes].copy_(s.cpu())
        packed.append(np.concatenate([p.ravel() for p in parts]))
    shared, sparts = make_expert(fmt, dim, inter, seed=999, gpu=gpu)
    spacked = np.concatenate([p.ravel() for p in sparts])
    layer = MoELayer(fmt, dim, inter, pool, n, topk, slots, shared_slot=shared)
    hits_total = 0
    for step in range(12):
        t = 1 + step % 4
        logits = data.zipf_logits(t, n, seed=step)
        x = data.activation(t, dim, seed=50 + step)
        y = np_(layer.forward(x.to(gpu), logits.to(gpu)))
        _, oids, ow = oracle.route(logits.numpy(), topk)
        assert [list(r) for r in layer.last_route[0]] == oids.tolist()
        want = oracle.moe_fp4([[packed[i] for i in row] for row in oids], ow, spacked, dim, inter, x.float().numpy())
        assert bf16_ulps(y, want).max() <= 1
        hits_total = layer.cache.stats()["hits"]
    assert hits_total > 0
    layer.close()


def test_moe_layer_reference_engine_semantics(gpu):
    # sqrt-softplus router, FP8 E8M0 shared expert next to FP4 routed experts, official numerics
    dim, inter, n, topk, slots = 256, 128, 16, 3, 12
    slot_bytes, _ = ops.expert_layout(ops.FP4, dim, inter)
    pool = torch.empty(n * slot_bytes, dtype=torch.uint8, pin_memory=True)
    mats = []
    for e in range(n):
        s, parts = make_expert(ops.FP4, dim, inter, seed=600 + 3 * e, gpu=gpu)
        pool[e * slot_bytes:(e + 1) * slot_bytes].copy_(s.cpu())
        mats.append(deq_parts(ops.FP4, parts))
    shared, sparts = make_expert(ops.FP8_E8M0, dim, inter, seed=699, gpu=gpu)
    bias = data.normal((n,), 0.05, seed=17)
    layer = MoELayer(ops.FP4, dim, inter, pool, n, topk, slots, shared_slot=shared, bias=bias.to(gpu), route_scale=2.5,
                     limit=10.0, official=True, score_fn=ops.SCORE_SQRT_SOFTPLUS, shared_fmt=ops.FP8_E8M0)
    for step in range(6):
        t = 1 + step % 4
        logits = data.zipf_logits(t, n, seed=70 + step) * 2
        x = data.activation(t, dim, seed=80 + step)
        y = np_(layer.forward(x.to(gpu), logits.to(gpu)))
        _, oids, ow = oracle.route(logits.numpy(), topk, bias.numpy(), 2.5, score_fn=oracle.SCORE_SQRT_SOFTPLUS)
        assert [list(r) for r in layer.last_route[0]] == oids.tolist()
        want = oracle.moe_deq([[mats[i] for i in row] for row in oids], ow, deq_parts(ops.FP8_E8M0, sparts),
                              x.float().numpy(), limit=10.0, official=True)
        assert bf16_ulps(y, want).max() <= 1
    layer.close()


def test_reference_abi_moe_composition(gpu):
    # The reference engine's MoE step issued through the drop-in ABI exactly as stbl/model.cu:508-592
    # issues it (official numerics): x quantized once; the routed experts' gate and up in one
    # stbl_gemv_mxfp4_batch on GGUF blocks, stbl_swiglu_batch with the route weights,
    # stbl_act_quant_fp8, the downs in a second batch; the FP8 E8M0 shared expert through
    # stbl_gemv_fp8 (its input re-quantized as the engine's gemv() does, :236-242); then stbl_axpy of
    # every expert output in top-k order, the shared one, and stbl_round_bf16. Checked against the
    # oracle's composition and against the fused stbl_amd_moe_experts on the same experts.
    dim, inter, topk, limit = 512, 256, 3, 10.0
    experts = [make_expert(ops.FP4, dim, inter, seed=900 + 3 * i, gpu=gpu) for i in range(topk)]
    shared, sparts = make_expert(ops.FP8_E8M0, dim, inter, seed=990, gpu=gpu)
    ws = [0.52, 0.31, 0.17]
    x = data.activation(1, dim, seed=91)
    f32 = lambda n: torch.zeros(n, dtype=torch.float32, device=gpu)

    def gguf(codes, sc):
        return torch.from_numpy(oracle.ocp_to_gguf17(codes, sc)).to(gpu)

    mats = [[gguf(p[0], p[1]), gguf(p[2], p[3]), gguf(p[4], p[5])] for _, p in experts]
    xq = x.float().to(gpu).reshape(-1).clone()
    ops.stbl_act_quant_fp8(xq)
    g, u, mid, eo = f32(topk * inter), f32(topk * inter), f32(topk * inter), f32(topk * dim)
    ops.stbl_gemv_mxfp4_batch([g[j * inter:(j + 1) * inter] for j in range(topk)] +
                              [u[j * inter:(j + 1) * inter] for j in range(topk)],
                              [m[0] for m in mats] + [m[1] for m in mats], [xq] * (2 * topk), inter, dim)
    ops.stbl_swiglu_batch(mid, g, u, ws, limit, inter)
    ops.stbl_act_quant_fp8(mid)
    ops.stbl_gemv_mxfp4_batch([eo[j * dim:(j + 1) * dim] for j in range(topk)], [m[2] for m in mats],
                              [mid[j * inter:(j + 1) * inter] for j in range(topk)], dim, inter)
    sv = ops.slot_views(shared, ops.FP8_E8M0, dim, inter)
    sg, su, smid, sout = f32(inter), f32(inter), f32(inter), f32(dim)
    ops.stbl_gemv_fp8(sg, sv[0].reshape(-1), sv[1].reshape(-1), xq, inter, dim, 1)
    ops.stbl_gemv_fp8(su, sv[2].reshape(-1), sv[3].reshape(-1), xq, inter, dim, 1)
    ops.stbl_swiglu(smid, sg, su, 1.0, limit, inter)
    ops.stbl_act_quant_fp8(smid)
    ops.stbl_gemv_fp8(sout, sv[4].reshape(-1), sv[5].reshape(-1), smid, dim, inter, 1)
    y = f32(dim)
    for j in range(topk):
        ops.stbl_axpy(y, eo[j * dim:(j + 1) * dim], 1.0, dim)
    ops.stbl_axpy(y, sout, 1.0, dim)
    ops.stbl_round_bf16(y)
    got = np_(y)

    want = oracle.moe_deq([[deq_parts(ops.FP4, p) for _, p in experts]], np.array([ws], np.float32),
                          deq_parts(ops.FP8_E8M0, sparts), x.float().numpy(), limit=limit, official=True)[0]
    assert bf16_ulps(got, want).max() <= 1
    fused = np_(ops.moe_experts(x.to(gpu), [e[0] for e in experts] + [shared], [list(range(topk))], [ws], ops.FP4,
                                dim, inter, shared=topk, limit=limit, official=True, shared_fmt=ops.FP8_E8M0))[0]
    assert bf16_ulps(got, fused.astype(np.float64)).max() <= 1


def test_moe_experts_byte_scales_fallback(gpu):
    # dims whose FP4 scale rows are not a multiple of 4 bytes (160 / 32 = 5, 96 / 32 = 3): the
    # several-expert launches (4 and 8 rows per workgroup) load scales byte by byte instead of as dwords
    dim, inter, topk, n = 160, 96, 3, 5
    experts = [make_expert(ops.FP4, dim, inter, seed=400 + 3 * i, gpu=gpu) for i in range(n)]
    rng = np.random.default_rng(44)
    for t in (1, 3):
        pick = [list(rng.choice(n - 1, size=topk, replace=False)) for _ in range(t)]
        w = (rng.random((t, topk)) / topk).astype(np.float32)
        x = data.activation(t, dim, seed=45 + t)
        y = np_(ops.moe_experts(x.to(gpu), [e[0] for e in experts], pick, w.tolist(), ops.FP4, dim, inter,
                                shared=n - 1))
        packed = [np.concatenate([p.ravel() for p in e[1]]) for e in experts]
        want = oracle.moe_fp4([[packed[i] for i in row] for row in pick], w, packed[n - 1], dim, inter,
                              x.float().numpy())
        assert bf16_ulps(y, want).max() <= 1


def test_moe_random_steps_match_one_token_calls(gpu):
    # random steps of one expert format (2-16 tokens, top-1..8 of up to 12 experts, with or without a
    # shared expert): whatever launches a step's jobs take (per token class, or every class in one
    # launch), each token's output equals a call with that token alone bit for bit, since every
    # (token, expert) sum uses the same lanes in the same order
    rng = np.random.default_rng(77)
    for case in range(9):
        fmt = (ops.FP4, ops.FP8, ops.FP8_E8M0)[case % 3]
        dim, inter = int(256 * rng.integers(1, 5)), int(128 * rng.integers(1, 5))
        t, topk = int(rng.integers(2, 17)), int(rng.integers(1, 9))
        nr = int(rng.integers(topk, topk + 5))
        slots = [make_expert(fmt, dim, inter, seed=7000 + 100 * case + 3 * i, gpu=gpu)[0] for i in range(nr + 1)]
        sh = nr if rng.random() < 0.7 else -1
        pick = [[int(v) for v in rng.choice(nr, size=topk, replace=False)] for _ in range(t)]
        w = (rng.random((t, topk)) / topk).astype(np.float32).tolist()
        official = bool(rng.integers(0, 2))
        x = data.activation(t, dim, seed=700 + case).to(gpu)
        kw = dict(shared=sh, limit=7.0, official=official)
        print(f"case {case}: fmt {fmt} {dim}x{inter} t={t} topk={topk} experts={nr} shared={sh}", flush=True)
        y = ops.moe_experts(x, slots, pick, w, fmt, dim, inter, **kw)
        for ti in range(t):
            y1 = ops.moe_experts(x[ti:ti + 1], slots, pick[ti:ti + 1], w[ti:ti + 1], fmt, dim, inter, **kw)
            assert torch.equal(y[ti], y1[0]), f"case {case} token {ti}"


def test_moe_and_gemm_from_concurrent_threads_and_streams(gpu):
    # four host threads, each on its own stream, run MoE steps (FP4 routed + FP8 E8M0 shared, one and
    # four tokens: the mixed and merged launches, whose job tables are built in per-thread host
    # arrays) and M = 64 GEMMs with their own work buffers, 10 times each; every result is
    # bit-identical to the same call made alone
    import threading

    dim, inter, n, topk = 1024, 512, 8, 4
    slots = [make_expert(ops.FP4, dim, inter, seed=3100 + 3 * i, gpu=gpu)[0] for i in range(n)]
    slots.append(make_expert(ops.FP8_E8M0, dim, inter, seed=3190, gpu=gpu)[0])
    gw = data.weight(2048, 1024, seed=3200)
    gc, gs = (torch.from_numpy(a).to(gpu) for a in oracle.quant_fp4(gw.numpy()))
    rng = np.random.default_rng(31)
    jobs = []
    for i in range(4):
        t = 1 if i % 2 == 0 else 4
        pick = [[int(v) for v in rng.choice(n, size=topk, replace=False)] for _ in range(t)]
        w = (rng.random((t, topk)) / topk).astype(np.float32).tolist()
        jobs.append((data.activation(t, dim, seed=3300 + i).to(gpu), pick, w, data.activation(64, 1024, seed=3400 + i).to(gpu)))
    kw = dict(shared=n, limit=10.0, official=True, shared_fmt=ops.FP8_E8M0)
    run = lambda x, pick, w, xg: (ops.moe_experts(x, slots, pick, w, ops.FP4, dim, inter, **kw),
                                  ops.gemm(gc, gs, xg, ops.FP4, 32))
    alone = [run(*j) for j in jobs]
    torch.cuda.synchronize()
    got, errors = [None] * 4, []

    def work(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                out = None
                for _ in range(10):
                    out = run(*jobs[i])
            s.synchronize()
            got[i] = out
        except Exception as e:  # reported below
            errors.append(repr(e))

    ts = [threading.Thread(target=work, args=(i,)) for i in range(4)]
    for th in ts:
        th.start()
    for th in ts:
        th.join()
    assert not errors, errors
    for (am, ag), (gm, gg) in zip(alone, got):
        assert torch.equal(am, gm) and torch.equal(ag, gg)


def test_moe_random_configurations(gpu):
    # 24 random expert steps over the three expert formats, a shared expert of the routed format or
    # of the engine's FP8 E8M0 one, raw and official numerics, SwiGLU limit or none, 1-16 tokens,
    # top-1..8 of up to 15 routed experts, against the dequantized composition
    rng = np.random.default_rng(2024)
    for case in range(24):
        fmt = (ops.FP4, ops.FP8, ops.FP8_E8M0)[case % 3]
        sfmt = fmt if rng.random() < 0.6 else (ops.FP8_E8M0 if fmt == ops.FP4 else fmt)
        dim, inter = int(256 * rng.integers(1, 5)), int(128 * rng.integers(1, 5))
        t, topk = int(rng.integers(1, 17)), int(rng.integers(1, 9))
        nr = int(rng.integers(topk, topk + 8))
        official, limit = bool(rng.integers(0, 2)), float(rng.choice([0.0, 7.0]))
        slots, dq = [], []
        for i in range(nr):
            s, parts = make_expert(fmt, dim, inter, seed=5000 + 100 * case + 3 * i, gpu=gpu)
            slots.append(s)
            dq.append(deq_parts(fmt, parts))
        shd, sh = None, -1
        if rng.random() < 0.7:
            s, parts = make_expert(sfmt, dim, inter, seed=9000 + case, gpu=gpu)
            slots.append(s)
            shd, sh = deq_parts(sfmt, parts), len(slots) - 1
        pick = [list(rng.choice(nr, size=topk, replace=False)) for _ in range(t)]
        w = (rng.random((t, topk)) / topk).astype(np.float32)
        x = data.activation(t, dim, seed=case)
        y = np_(ops.moe_experts(x.to(gpu), slots, pick, w.tolist(), fmt, dim, inter, shared=sh, limit=limit,
                                official=official, shared_fmt=sfmt if sh >= 0 and sfmt != fmt else -1).float())
        xs = x.float().numpy()
        want = oracle.moe_deq([[dq[i] for i in row] for row in pick], w, shd, xs, limit, official)
        terms = np.zeros((t, dim))
        for ti in range(t):
            for j, e in enumerate(pick[ti]):
                terms[ti] += np.abs(oracle.expert_ffn_deq(*dq[e], xs[ti], float(w[ti, j]), limit, official))
            if shd is not None:
                terms[ti] += np.abs(oracle.expert_ffn_deq(*shd, xs[ti], 1.0, limit, official))
        assert_moe_sum(y, want, terms)
