"""The file tier of the expert cache: routed experts read from a GGUF file on misses
(stbl_amd_cache_create_gguf; the reference's demand read, stbl/model.cu:283-308, :383-422).

Parity bar: bit-exact. A slot refilled from the file holds exactly the bytes of the slot built
directly from the same OCP codes and scales (ops.pack_slot), whose GGUF blocks the writer produced
with the conversion pinned on the oracle (test_gguf_cpu.py); the MoE layer over the file tier gives
bit-identical outputs to the same layer over the pinned host pool, and stays within the MoE bar of
the oracle. LRU bookkeeping is checked against oracle.lru_simulate. Files are written both where
O_DIRECT is refused (the test's temporary directory on tmpfs) and, where the box's disk allows it,
under the repository, so the aligned-read path runs too.
"""

import os
import pathlib
import shutil
from collections import OrderedDict

import numpy as np
import pytest
import torch

import oracle
from stblarge_amd import data, gguf, ops
from stblarge_amd.moe import ExpertCache, MoELayer, MoEStack
from util import bf16_ulps, np_, read_device

pytestmark = pytest.mark.gpu

REPO = pathlib.Path(__file__).resolve().parent.parent


def _accepts_direct(d):
    probe = d / "direct.probe"
    probe.write_bytes(bytes(4096))
    try:
        os.close(os.open(probe, os.O_RDONLY | os.O_DIRECT))
        return True
    except OSError:
        return False
    finally:
        probe.unlink()


@pytest.fixture(params=["buffered", "direct"])
def file_dir(request, tmp_path):
    """(directory, whether reads there use O_DIRECT)."""
    if request.param == "buffered":
        yield tmp_path, False
        return
    for d in (tmp_path, REPO / "_direct_io_tmp"):
        d.mkdir(exist_ok=True)
        if _accepts_direct(d):
            yield d, True
            if d != tmp_path:
                shutil.rmtree(d, ignore_errors=True)
            return
    shutil.rmtree(REPO / "_direct_io_tmp", ignore_errors=True)
    pytest.skip("no file system here accepts O_DIRECT")


def random_parts(dim, inter, seed):
    """OCP FP4 parts of one expert: random codes, scale bytes 118..125 (stbl/test_kernels.py:101-117)."""
    rng = np.random.default_rng(seed)
    out = []
    for rows, k in ((inter, dim), (inter, dim), (dim, inter)):
        out += [rng.integers(0, 256, (rows, k // 2), dtype=np.uint8), rng.integers(118, 126, (rows, k // 32), dtype=np.uint8)]
    return out


def quantized_parts(dim, inter, seed):
    """OCP FP4 parts of seeded N(0, 0.02) weights quantized by the oracle (the MoE tests' weights)."""
    out = []
    for i, (rows, k) in enumerate(((inter, dim), (inter, dim), (dim, inter))):
        out += list(oracle.quant_fp4(data.weight(rows, k, seed + i).numpy()))
    return out


def expert_file(path, dim, inter, n_layers, n_experts, seed=0, first_layer=0, make=random_parts):
    parts = {(first_layer + l, e): make(dim, inter, seed + 100 * l + 3 * e)
             for l in range(n_layers) for e in range(n_experts)}
    gguf.write_experts(path, lambda l, e: parts[l, e], n_layers, n_experts, dim, inter, first_layer=first_layer)
    return parts


def direct_slot(parts, dim, inter, gpu):
    return ops.pack_slot([torch.from_numpy(p).to(gpu) for p in parts], ops.FP4, dim, inter).cpu()


@pytest.mark.parametrize("dim,inter,n_layers,n_experts,readers", [(256, 128, 2, 6, 3), (7168, 2048, 1, 3, 8)])
def test_file_slots_equal_directly_built_slots(gpu, file_dir, dim, inter, n_layers, n_experts, readers):
    d, direct = file_dir
    path = d / f"experts_{dim}.gguf"
    parts = expert_file(path, dim, inter, n_layers, n_experts, seed=dim, first_layer=2)
    want = {k: direct_slot(v, dim, inter, gpu) for k, v in parts.items()}
    slots = min(4, n_experts - 1)
    cache = ExpertCache.from_gguf(slots, path, first_layer=2, n_layers=n_layers, readers=readers, direct=direct)
    info = cache.file_info()
    assert (info["dim"], info["inter"], info["experts"]) == (dim, inter, n_experts)
    assert info["direct"] == int(direct)
    assert cache.slot_bytes == ops.expert_layout(ops.FP4, dim, inter)[0]
    rng = np.random.default_rng(1)
    steps = [(int(rng.integers(n_layers)), [int(e) for e in rng.choice(n_experts, size=min(3, slots), replace=False)])
             for _ in range(12 if dim < 1024 else 5)]
    sim = oracle.lru_simulate([[l * 1000 + e for e in ids] for l, ids in steps], slots)
    for (l, ids), (hits, _, _) in zip(steps, sim):
        ptrs, got_hits, nmiss = cache.lookup(ids, layer=l)
        assert got_hits == hits and nmiss == hits.count(False)
        cache.mark_used()
        torch.cuda.synchronize()
        for e, p in zip(ids, ptrs):
            got = read_device(p, cache.slot_bytes)
            assert torch.equal(got, want[2 + l, e]), f"layer {l} expert {e}"
    st, info = cache.stats(), cache.file_info()
    part = inter * dim // 32 * 17
    assert info["experts_read"] == st["misses"] and info["bytes_read"] == st["misses"] * 3 * part
    cache.close()


def test_file_read_failures_leave_slots_unmapped(gpu, tmp_path):
    dim, inter, n = 256, 128, 5
    path = tmp_path / "e.gguf"
    parts = expert_file(path, dim, inter, 1, n, seed=7)
    cache = ExpertCache.from_gguf(4, path, readers=2)
    cache.fail_refill_after(1)  # the second miss of the next lookup fails before anything is read
    with pytest.raises(RuntimeError, match="injected"):
        cache.lookup([0, 1, 2])
    assert all(cache.peek(e) is None for e in (0, 1, 2))
    assert cache.stats()["misses"] == 0
    ptrs, hits, nmiss = cache.lookup([0, 1, 2])
    assert nmiss == 3
    torch.cuda.synchronize()
    for e, p in zip((0, 1, 2), ptrs):
        assert torch.equal(read_device(p, cache.slot_bytes), direct_slot(parts[0, e], dim, inter, gpu))
    # the file loses half of its last expert's down blocks: that read ends early, the slot stays unmapped
    with gguf.GgufFile(path) as g:
        down = g.tensor(gguf.expert_tensor(0, "down"))
    part = inter * dim // 32 * 17
    os.truncate(path, down["offset"] + (n - 1) * part + part // 2)
    with pytest.raises(RuntimeError, match="file offset"):
        cache.lookup([n - 1])
    assert cache.peek(n - 1) is None
    ptrs, hits, _ = cache.lookup([1, 3])  # the cache still serves hits and readable experts
    assert hits == [True, False]
    torch.cuda.synchronize()
    assert torch.equal(read_device(ptrs[1], cache.slot_bytes), direct_slot(parts[0, 3], dim, inter, gpu))
    cache.close()


def test_moe_layer_over_file_equals_host_pool(gpu, file_dir):
    d, _ = file_dir
    dim, inter, n, topk, slots = 256, 128, 16, 3, 12
    path = d / "moe.gguf"
    parts = expert_file(path, dim, inter, 1, n, seed=31, make=quantized_parts)
    slot_bytes, _ = ops.expert_layout(ops.FP4, dim, inter)
    pool = torch.empty(n * slot_bytes, dtype=torch.uint8, pin_memory=True)
    packed = []
    for e in range(n):
        s = direct_slot(parts[0, e], dim, inter, gpu)
        pool[e * slot_bytes:(e + 1) * slot_bytes].copy_(s)
        packed.append(np.concatenate([p.ravel() for p in parts[0, e]]))
    sparts = quantized_parts(dim, inter, 999)
    shared = direct_slot(sparts, dim, inter, gpu).to(gpu)
    spacked = np.concatenate([p.ravel() for p in sparts])
    over_pool = MoELayer(ops.FP4, dim, inter, pool, n, topk, slots, shared_slot=shared)
    over_file = MoELayer(ops.FP4, dim, inter, None, n, topk, slots, shared_slot=shared,
                         cache=ExpertCache.from_gguf(slots, path, readers=4))
    for step in range(10):
        t = 1 + step % 4
        logits = data.zipf_logits(t, n, seed=step).to(gpu)
        x = data.activation(t, dim, seed=70 + step).to(gpu)
        y_pool, y_file = over_pool.forward(x, logits), over_file.forward(x, logits)
        assert torch.equal(y_pool, y_file)
        _, oids, ow = oracle.route(logits.cpu().numpy(), topk)
        want = oracle.moe_fp4([[packed[i] for i in row] for row in oids], ow, spacked, dim, inter, x.float().cpu().numpy())
        assert bf16_ulps(np_(y_file), want).max() <= 1
    assert over_file.cache.stats() == over_pool.cache.stats()
    over_pool.close()
    over_file.close()


# ---- prefetch (stbl/model.cu:310-345, :478-496, :550-586) -----------------------------------------------

def _wait_for(cond, seconds=60.0):
    import time
    end = time.monotonic() + seconds
    while not cond():
        assert time.monotonic() < end, "prefetch readers did not finish"
        time.sleep(0.005)


def test_prefetch_cancel_take_over_and_land(gpu, tmp_path):
    dim, inter, n = 256, 128, 10
    path = tmp_path / "pf.gguf"
    parts = expert_file(path, dim, inter, 2, n, seed=11)
    want = {k: direct_slot(v, dim, inter, gpu) for k, v in parts.items()}
    expert_bytes = 3 * (inter * dim // 32 * 17)
    cache = ExpertCache.from_gguf(8, path, n_layers=2, readers=2)
    cache.enable_prefetch(3)
    cache.prefetch_pause(True)  # every job stays queued
    assert cache.prefetch([0, 1, 2, 3], layer=1) == 4
    assert cache.prefetch([0, 3], layer=1) == 0  # already mapped
    ptrs, hits, nmiss = cache.lookup([0, 5], layer=1)
    # 0 was queued and not started: the lookup took it over (a miss into the job's slot);
    # 1, 2 and 3 were not routed and not started: cancelled, their slots free again
    assert hits == [False, False] and nmiss == 2
    st = cache.prefetch_stats()
    assert (st["issued"], st["taken_over"], st["cancelled"], st["routed_landed"], st["bytes_read"]) == (4, 1, 3, 0, 0)
    assert all(cache.peek(e, layer=1) is None for e in (1, 2, 3))
    torch.cuda.synchronize()
    for e, p in zip((0, 5), ptrs):
        assert torch.equal(read_device(p, cache.slot_bytes), want[1, e])
    cache.mark_used()
    cache.prefetch_pause(False)
    assert cache.prefetch([6, 7], layer=0) == 2
    _wait_for(lambda: cache.prefetch_stats()["bytes_read"] == 2 * expert_bytes)
    ptrs, hits, nmiss = cache.lookup([6, 7, 8], layer=0)
    assert hits == [True, True, False] and nmiss == 1
    st = cache.prefetch_stats()
    assert st["routed_landed"] + st["routed_reading"] == 2 and st["issued"] == 6
    torch.cuda.synchronize()
    for e, p in zip((6, 7, 8), ptrs):
        assert torch.equal(read_device(p, cache.slot_bytes), want[0, e])
    cache.mark_used()
    # a guess queued for the next layer lands before that layer is looked up: a hit
    assert cache.prefetch([9], layer=1) == 1
    _wait_for(lambda: cache.prefetch_stats()["bytes_read"] == 3 * expert_bytes)
    ptrs, hits, _ = cache.lookup([9], layer=1)
    assert hits == [True]
    torch.cuda.synchronize()
    assert torch.equal(read_device(ptrs[0], cache.slot_bytes), want[1, 9])
    cache.close()


def test_moe_stack_with_prefetch_equals_without(gpu, file_dir):
    # three layers over one file: decode tokens layer by layer, with and without stale-router guesses
    # for the next layer queued after each layer; the outputs must be bit-identical
    d, _ = file_dir
    dim, inter, n, topk, slots, n_layers = 256, 128, 16, 3, 12, 3
    path = d / "stack.gguf"
    expert_file(path, dim, inter, n_layers, n, seed=41, make=quantized_parts)
    sparts = quantized_parts(dim, inter, 77)
    shared = direct_slot(sparts, dim, inter, gpu).to(gpu)
    plain = ExpertCache.from_gguf(slots, path, n_layers=n_layers, readers=2)
    ahead = ExpertCache.from_gguf(slots, path, n_layers=n_layers, readers=2)
    ahead.enable_prefetch(3)
    mk = lambda cache, l: MoELayer(ops.FP4, dim, inter, None, n, topk, slots, shared_slot=shared, cache=cache, layer=l)
    stack_plain = [mk(plain, l) for l in range(n_layers)]
    stack_ahead = [mk(ahead, l) for l in range(n_layers)]
    rng = np.random.default_rng(3)
    for token in range(10):
        x = data.activation(1, dim, seed=500 + token).to(gpu)
        for l in range(n_layers):
            logits = data.zipf_logits(1, n, seed=1000 * token + l).to(gpu)
            y_plain = stack_plain[l].forward(x, logits)
            y_ahead = stack_ahead[l].forward(x, logits)
            assert torch.equal(y_plain, y_ahead), f"token {token} layer {l}"
            if l + 1 < n_layers:  # a guess: the next layer's true top-k mixed with random experts
                nxt = data.zipf_logits(1, n, seed=1000 * token + l + 1)
                true = [int(e) for e in torch.topk(nxt[0], topk).indices]
                guess = true[:2] + [int(e) for e in rng.choice(n, 3, replace=False)]
                ahead.prefetch(list(dict.fromkeys(guess)), l + 1)
            x = y_plain
    st = ahead.prefetch_stats()
    assert st["issued"] > 0 and st["routed_landed"] + st["routed_reading"] + st["taken_over"] > 0
    assert plain.stats()["hits"] + plain.stats()["misses"] == ahead.stats()["hits"] + ahead.stats()["misses"]
    plain.close()
    ahead.close()


def test_moe_stack_stale_router_prefetch(gpu, tmp_path):
    # the engine's own guesses: layer l+1's router run on layer l's input (stbl/model.cu:432-475),
    # its top 6 queued after each layer; outputs bit-identical to the same stack without prefetch
    dim, inter, n, topk, slots, n_layers = 256, 128, 16, 3, 12, 3
    path = tmp_path / "stale.gguf"
    expert_file(path, dim, inter, n_layers, n, seed=51, make=quantized_parts)
    routers = [data.normal((n, dim), 0.05, seed=60 + l).to(gpu) for l in range(n_layers)]
    shared = direct_slot(quantized_parts(dim, inter, 88), dim, inter, gpu).to(gpu)
    mk = lambda pf: MoEStack(ExpertCache.from_gguf(slots, path, n_layers=n_layers, readers=2), ops.FP4, dim, inter, n,
                             topk, routers, shared_slots=[shared] * n_layers, prefetch=pf)
    plain, ahead = mk(0), mk(6)
    for token in range(8):
        h = data.activation(1 + token % 2, dim, seed=700 + token).to(gpu)
        a, b = plain.step(h), ahead.step(h)
        assert torch.equal(a, b), f"token {token}"
        assert torch.isfinite(a.float()).all()
    st = ahead.cache.prefetch_stats()
    # small residual updates keep the next layer's routing close to the stale guess
    assert st["issued"] > 0 and st["routed_landed"] + st["routed_reading"] > 0
    assert plain.cache.stats()["hits"] + plain.cache.stats()["misses"] == ahead.cache.stats()["hits"] + ahead.cache.stats()["misses"]
    plain.close()
    ahead.close()


def _replay_lookahead(trace, slots):
    """Host replay of the lookahead counters (stbl/model.cu:452-460) over a stack's trace, on the
    plain LRU of a cache without prefetch: keys (layer, expert); a guess's cold flags are taken when
    it is noted; the next lookup of its layer counts it, before its own misses are mapped."""
    lru, la, noted = OrderedDict(), [0, 0, 0, 0], {}
    for kind, layer, ids in trace:
        if kind == "guess":
            noted[layer] = (ids, [(layer, e) not in lru for e in ids])
            continue
        if layer in noted:
            guess, cold = noted.pop(layer)
            la[0] += sum(cold)
            la[1] += sum(1 for e, c in zip(guess, cold) if c and e in ids)
            miss = [e for e in ids if (layer, e) not in lru]
            la[2] += len(miss)
            la[3] += sum(1 for e in miss if e in guess)
        for e in ids:
            if (layer, e) in lru:
                lru.move_to_end((layer, e))
        for e in ids:
            k = (layer, e)
            if k in lru:
                lru.move_to_end(k)
            else:
                if len(lru) >= slots:
                    lru.popitem(last=False)
                lru[k] = True
    return la


def test_moe_stack_prefetch2_and_lookahead(gpu, tmp_path):
    # four layers: guesses for the next layer are noted for the lookahead counters (STBL_LOOKAHEAD)
    # and, with prefetch, read in the background, with prefetch2 also the layer after next's
    # (STBL_PREFETCH2, stbl/model.cu:437-442, 573-583). Outputs are bit-identical to the stack that
    # only counts; its counters equal a host replay of its guesses and lookups.
    dim, inter, n, topk, slots, n_layers = 256, 128, 16, 3, 12, 4
    path = tmp_path / "ahead2.gguf"
    expert_file(path, dim, inter, n_layers, n, seed=61, make=quantized_parts)
    routers = [data.normal((n, dim), 0.05, seed=80 + l).to(gpu) for l in range(n_layers)]
    shared = direct_slot(quantized_parts(dim, inter, 89), dim, inter, gpu).to(gpu)
    mk = lambda **kw: MoEStack(ExpertCache.from_gguf(slots, path, n_layers=n_layers, readers=2), ops.FP4, dim, inter, n,
                               topk, routers, shared_slots=[shared] * n_layers, **kw)
    counting = mk(lookahead=5, trace=True)
    ahead2 = mk(prefetch=5, prefetch2=3)
    for token in range(8):
        h = data.activation(1 + token % 2, dim, seed=900 + token).to(gpu)
        a, b = counting.step(h), ahead2.step(h)
        assert torch.equal(a, b), f"token {token}"
    la = counting.cache.lookahead()
    assert list(la.values()) == _replay_lookahead(counting.trace, slots)
    assert la["cold_guesses"] > 0 and la["misses"] > 0 and la["misses_guessed"] > 0
    la2 = ahead2.cache.lookahead()
    assert la2["cold_guesses"] >= la2["cold_guesses_routed"] and la2["misses"] >= la2["misses_guessed"]
    st = ahead2.cache.prefetch_stats()
    assert st["issued"] > 0 and st["routed_landed"] + st["routed_reading"] > 0
    assert counting.cache.stats()["lookups"] == ahead2.cache.stats()["lookups"] == 8 * n_layers
    counting.close()
    ahead2.close()
