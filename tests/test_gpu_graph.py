"""Every hot-path entry point captured in a HIP graph (torch.cuda.CUDAGraph) and replayed several
times, with the program's own eager work and synchronizations between the replays: each replay must
equal the eager result bit for bit. bench.py times the path through such graphs, and a kernel or
library call that records something a replay does not redo (a memset node, host-side state) would
show here as a wrong second replay."""

import pytest
import torch

from stblarge_amd import data, ops

pytestmark = pytest.mark.gpu


def _replays_match(fn, other):
    """fn() returns a list of output tensors; other() is unrelated eager work."""
    eager = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm the code path outside the capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        outs = fn()
    for rep in range(3):
        for t in outs:
            t.fill_(float("nan") if t.is_floating_point() else 0)  # a replay must rewrite every output
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep} differs from the eager result"
        other()
        torch.cuda.synchronize()


def test_graph_replay_gemv_batch_ffn_moe_gemm(gpu):
    rows, k = 2048, 7168
    w = data.weight(rows, k, seed=1).to(gpu)
    c4, s4 = ops.quant_fp4(w)
    c8, s8 = ops.quant_fp8_b128(w)
    x = data.activation(1, k, seed=2).to(gpu)
    x4 = data.activation(4, k, seed=3).to(gpu)
    other_x = data.activation(1, k, seed=4).to(gpu)
    other = lambda: ops.gemv_fp4(c4, s4, other_x)

    _replays_match(lambda: [ops.gemv_fp4(c4, s4, x), ops.gemv_fp8(c8, s8, x), ops.gemv_fp4(c4, s4, x4)], other)
    cs = [c4] * 16
    ss = [s4] * 16
    xs = [data.activation(1, k, seed=10 + j).to(gpu) for j in range(16)]
    _replays_match(lambda: ops.gemv_batch(cs, ss, xs, ops.FP4), other)

    dim, inter = 7168, 2048
    slot = ops.quant_expert(data.weight(inter, dim, 5).to(gpu), data.weight(inter, dim, 6).to(gpu),
                            data.weight(dim, inter, 7).to(gpu), ops.FP4)
    _replays_match(lambda: [ops.expert_ffn(slot, x, ops.FP4, dim, inter)], other)

    shared = ops.quant_expert(data.weight(inter, dim, 8).to(gpu), data.weight(inter, dim, 9).to(gpu),
                              data.weight(dim, inter, 10).to(gpu), ops.FP8_E8M0)
    slots = [slot, slot.clone(), slot.clone(), shared]
    xt = data.activation(2, dim, seed=11).to(gpu)
    work = torch.empty(ops.moe_work_bytes(2, 3, dim, inter), dtype=torch.uint8, device=gpu)
    _replays_match(lambda: [ops.moe_experts(xt, slots, [[0, 1, 2], [2, 0, 1]], [[0.5, 0.3, 0.2], [0.6, 0.3, 0.1]],
                                            ops.FP4, dim, inter, shared=3, limit=10.0, official=True, work=work,
                                            shared_fmt=ops.FP8_E8M0)], other)

    xg = data.activation(64, k, seed=12).to(gpu)
    aq, a_s = ops.act_quant_e4m3(xg, 128)
    _replays_match(lambda: [ops.gemm_q(c4, s4, aq, a_s, ops.FP4), ops.gemm(c8, s8, xg, ops.FP8)], other)
