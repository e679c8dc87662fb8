"""stbl_amd_moe_experts_noalloc, the routed-MoE step that allocates nothing (the library's static
device scratch takes the place of the caller's workspace), against stbl_amd_moe_experts on the same
inputs: bit-identical outputs on two calls in a row, the second on fewer tokens (the scratch keeps
the first call's contents); no change in the device's free memory over repeated calls; the same
result from a call captured in a HIP graph on every replay; and a clear refusal of a step larger
than the scratch."""

import ctypes

import pytest
import torch

from stblarge_amd import _lib, data, ops

pytestmark = pytest.mark.gpu

P = ctypes.c_void_p


def _expert(fmt, dim, inter, seed, gpu):
    return ops.quant_expert(data.weight(inter, dim, seed, gpu), data.weight(inter, dim, seed + 1, gpu),
                            data.weight(dim, inter, seed + 2, gpu), fmt)


def _noalloc(x, slots, pick, weights, dim, inter, shared, shared_fmt, limit, official, y=None):
    t, topk = x.shape[0], len(pick[0])
    if y is None:
        y = torch.full((t, dim), float("nan"), dtype=torch.bfloat16, device=x.device)
    arr = (P * len(slots))(*[s.data_ptr() for s in slots])
    pk = (ctypes.c_int * (t * topk))(*[int(v) for row in pick for v in row])
    wt = (ctypes.c_float * (t * topk))(*[float(v) for row in weights for v in row])
    st = _lib.load().stbl_amd_moe_experts_noalloc(ops.FP4, P(y.data_ptr()), P(x.data_ptr()), t, dim, inter, arr,
                                                  len(slots), pk, wt, topk, shared, shared_fmt, float(limit),
                                                  int(official), 0, ops._stream())
    _lib.check(st, "moe_experts_noalloc")
    return y


def test_noalloc_matches_moe_experts_on_two_calls(gpu):
    # the C4 shapes: 10 routed FP4 experts + an FP4 shared one; 4 tokens x top-8, then 1 token
    dim, inter, topk, n = 7168, 2048, 8, 10
    slots = [_expert(ops.FP4, dim, inter, 3000 + 3 * i, gpu) for i in range(n)] + [_expert(ops.FP4, dim, inter, 3099, gpu)]
    g = torch.Generator().manual_seed(5)
    for t, official in ((4, False), (1, True)):
        pick = [torch.randperm(n, generator=g)[:topk].tolist() for _ in range(t)]
        w = (torch.rand((t, topk), generator=g) / topk).tolist()
        x = data.activation(t, dim, seed=3100 + t).to(gpu)
        print(f"noalloc call: t={t} topk={topk} official={official}", flush=True)
        got = _noalloc(x, slots, pick, w, dim, inter, n, -1, 10.0, official)
        want = ops.moe_experts(x, slots, pick, w, ops.FP4, dim, inter, shared=n, limit=10.0, official=official)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"t={t}: noalloc differs from moe_experts"


def test_noalloc_allocates_nothing_and_replays_in_a_graph(gpu):
    # after a first call (which looks up the scratch's address), further calls leave the device's
    # free memory unchanged; a call captured in a HIP graph and replayed (with eager work and
    # synchronizations between the replays) gives moe_experts' result on every replay
    dim, inter, topk, n, t = 7168, 2048, 8, 9, 2
    slots = [_expert(ops.FP4, dim, inter, 4000 + 3 * i, gpu) for i in range(n)]
    g = torch.Generator().manual_seed(9)
    pick = [torch.randperm(n, generator=g)[:topk].tolist() for _ in range(t)]
    w = (torch.rand((t, topk), generator=g) / topk).tolist()
    x = data.activation(t, dim, seed=4100).to(gpu)
    want = ops.moe_experts(x, slots, pick, w, ops.FP4, dim, inter, limit=10.0)
    y = torch.full((t, dim), float("nan"), dtype=torch.bfloat16, device=gpu)
    _noalloc(x, slots, pick, w, dim, inter, -1, -1, 10.0, False, y=y)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(5):
        _noalloc(x, slots, pick, w, dim, inter, -1, -1, 10.0, False, y=y)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    assert torch.equal(y, want)
    yg = torch.full((t, dim), float("nan"), dtype=torch.bfloat16, device=gpu)
    graph = torch.cuda.CUDAGraph()
    print("noalloc graph capture", flush=True)
    with torch.cuda.graph(graph):
        _noalloc(x, slots, pick, w, dim, inter, -1, -1, 10.0, False, y=yg)
    for rep in range(3):
        yg.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, want), f"replay {rep} differs from moe_experts"
    del graph


def test_noalloc_refuses_a_step_beyond_its_scratch(gpu):
    # 16 tokens x top-16 at dim = inter = 16384 needs 17.8 MB of scratch, more than its 8 MiB: refused
    # before anything is launched
    t, topk, dim, inter = 16, 16, 16384, 16384
    x = torch.zeros((t, dim), dtype=torch.bfloat16, device=gpu)
    slot = torch.zeros(256, dtype=torch.uint8, device=gpu)
    with pytest.raises(_lib.StblError, match="bytes of scratch"):
        _noalloc(x, [slot], [[0] * topk] * t, [[0.0] * topk] * t, dim, inter, -1, -1, 0.0, False)
