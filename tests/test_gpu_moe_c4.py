"""Configuration C4 at its own shape: a routed MoE layer decoding 1 and 4 tokens over 256 FP4 experts
of gate/up [2048 x 7168] and down [7168 x 2048] plus one shared FP4 expert, a sigmoid top-8 router on
Zipf(1.1) Gumbel-top-k logits, and a 64-slot HBM LRU cache refilled from a pinned host pool.

Oracle: oracle.route (stbl/model.cu:444-451 with sigmoid scores), oracle.moe_fp4 (the expert
composition and top-k-order sum, stbl/model.cu:505-592) and oracle.lru_simulate (the cache's
bookkeeping, stbl/model.cu:347-422, 497-507).
Bar: router ids exact; every output within one bf16 step of each expert's output plus one of its
own (util.assert_moe_sum: a sum of nine bf16 expert outputs can cancel to a small result, where one
step of a term is several of the result), flips rare; the hit/miss sequence identical to the
replay; and every step bit-identical to one
stbl_amd_moe_experts call over the same slots, so the layer's split around the refill wait (the
resident experts queued before the wait, the refilled ones after) changes no bit.

The pool's 256 entries are 16 quantized experts repeated, each entry then made distinct by its own id
written into its first code byte, so a slot mapped to the wrong expert changes the output.
"""

import numpy as np
import pytest
import torch

import oracle
from stblarge_amd import data, ops
from stblarge_amd.moe import MoELayer
from util import assert_moe_sum, np_

pytestmark = pytest.mark.gpu

DIM, INTER, N_EXP, TOPK, SLOTS, N_BASE = data.DIM, data.INTER, data.N_EXPERTS, data.TOPK, data.CACHE_SLOTS, 16


@pytest.fixture(scope="module")
def c4_pool(gpu):
    sb, _ = ops.expert_layout(ops.FP4, DIM, INTER)
    base = [ops.quant_expert(data.weight(INTER, DIM, 5000 + 3 * i, gpu), data.weight(INTER, DIM, 5001 + 3 * i, gpu),
                             data.weight(DIM, INTER, 5002 + 3 * i, gpu), ops.FP4) for i in range(N_BASE)]
    pool = torch.empty(N_EXP * sb, dtype=torch.uint8, pin_memory=True)
    view = pool.view(N_EXP, sb)
    for e in range(N_EXP):
        view[e].copy_(base[e % N_BASE])
        view[e, 0] = e  # gate row 0, elements 0 and 1: this entry's own id
    del base
    shared = ops.quant_expert(data.weight(INTER, DIM, 4990, gpu), data.weight(INTER, DIM, 4991, gpu),
                              data.weight(DIM, INTER, 4992, gpu), ops.FP4)
    torch.cuda.synchronize()
    yield view, shared, sb
    del pool


@pytest.mark.parametrize("t,warm,checked", [(1, 60, 6), (4, 24, 3)])
def test_c4_moe_layer(gpu, c4_pool, t, warm, checked):
    view, shared, sb = c4_pool
    layer = MoELayer(ops.FP4, DIM, INTER, view.view(-1), N_EXP, TOPK, SLOTS, shared_slot=shared, max_tokens=4)
    spacked = shared.cpu().numpy()
    side = torch.cuda.Stream()
    looked, checked_hits, checked_misses = [], 0, 0
    for step in range(warm + checked):
        logits = data.zipf_logits(t, N_EXP, seed=1000 * t + step)
        x = data.activation(t, DIM, seed=2000 * t + step)
        xd, ld = x.to(gpu), logits.to(gpu)
        on_side = step >= warm and step % 2 == 1  # half the checked steps run on a side stream
        if on_side:
            side.wait_stream(torch.cuda.current_stream())
            y = layer.forward(xd, ld, stream=side)
            torch.cuda.current_stream().wait_stream(side)
        else:
            y = layer.forward(xd, ld)
        uniq, hits = layer.last_lookup
        looked.append((list(uniq), list(hits)))
        if step < warm:
            continue
        checked_hits += sum(hits)
        checked_misses += len(hits) - sum(hits)
        _, oids, ow = oracle.route(logits.numpy(), TOPK)
        assert [list(r) for r in layer.last_route[0]] == oids.tolist(), f"step {step}: routes differ"
        # one call over the same slots, all resident now: the same bits as the split step
        slots = [layer.cache.peek(e) for e in uniq] + [shared.data_ptr()]
        slot_of = {e: i for i, e in enumerate(uniq)}
        y1 = ops.moe_experts(xd, slots, [[slot_of[e] for e in row] for row in layer.last_route[0]],
                             layer.last_route[1], ops.FP4, DIM, INTER, shared=len(uniq))
        assert torch.equal(y, y1), f"step {step}: split step differs from one call (side stream: {on_side})"
        xf = x.float().numpy()
        want = oracle.moe_fp4([[view[e].numpy() for e in row] for row in oids], ow, spacked, DIM, INTER, xf)
        terms = np.zeros((t, DIM))
        for i, row in enumerate(oids):
            for p, e in enumerate(row):
                terms[i] += np.abs(oracle.expert_ffn_fp4(view[e].numpy(), DIM, INTER, xf[i], ow[i, p]))
            terms[i] += np.abs(oracle.expert_ffn_fp4(spacked, DIM, INTER, xf[i], 1.0))
        assert_moe_sum(np_(y), want, terms)
    replay = oracle.lru_simulate([u for u, _ in looked], SLOTS)
    assert [h for _, h in looked] == [r[0] for r in replay]
    assert checked_hits > 0 and checked_misses > 0, "the checked steps should both hit and miss"
    st = layer.cache.stats()
    assert st["refill_bytes"] == st["misses"] * sb and st["in_use"] == SLOTS
    layer.close()
