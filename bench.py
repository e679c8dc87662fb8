"""Benchmark of the quantized expert-GEMV path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only fp4|all]

A step is one launch of the hot path over one batch of synthetic input. The headline workload is
one FP4 (e2m1, E8M0 per 32) GEMV, W [2048 x 7168], x bf16 [1 x 7168],
y bf16 [1 x 2048]. Weights are seeded N(0, 0.02) quantized on the GPU; the timed launches cycle
through enough distinct weight copies (>= 512 MB) that the 256 MB Infinity Cache cannot serve
repeats, so every step reads its weights from HBM. Launches are replayed from a HIP graph so that
the GPU runs them back to back. Each timed sample is exactly K steps between two clock-stamp
launches in the same graph (the GPU's wall clock as each stamp starts), net of the stamps' own cost;
with small K, several samples are taken and the median reported (`timing` in the line).

`value` = algorithmic bytes per step (codes + scales + x + y, each once) / measured time per step.
One JSON line is printed; other configurations appear under "extra".
"""

import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
ROTATE_BYTES = 512 << 20
METRIC = "HBM GB/s (% of peak) for FP8/FP4 expert GEMV; MoE-layer decode tokens/s"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", default="all",
                    help="fp4 (headline and its floors) | gemv | batch | ffn | gemm | moe | moeallhit | refabi | "
                         "file | filestack | floor | all")
    ap.add_argument("--moe-steps", type=int, default=200)
    ap.add_argument("--moe-warmup", type=int, default=1000)
    ap.add_argument("--eager", action="store_true", help="also time launches issued one by one from Python")
    ap.add_argument("--no-graph", action="store_true", help="launch every step from Python (for counter runs)")
    ap.add_argument("--rows-out", default=None, help="write every row's full figures to this JSON file")
    ap.add_argument("--trace-summary", default=None, metavar="CSV",
                    help="print the per-dispatch summary of a rocprofv3 kernel-trace CSV and exit (no GPU)")
    ap.add_argument("--trace-kernel", default=r"k_gemv<\(stbl::WFmt\)0, false, 1,",
                    help="kernel-name regex for --trace-summary (default: the headline FP4 GEMV kernel)")
    ap.add_argument("--counter-summary", default=None, metavar="CSV",
                    help="print per (kernel, grid, counter) medians of a rocprofv3 --pmc counter_collection CSV and exit")
    ap.add_argument("--counter-last", type=int, default=0, metavar="N",
                    help="with --counter-summary: instead of medians, the values of the last N matching dispatches "
                         "(by dispatch id), e.g. the calibration copies --copy-calib issues at the end of a run")
    ap.add_argument("--trace-by-grid", action="store_true",
                    help="with --trace-summary: one line per (kernel, grid) with calls and median / mean duration")
    ap.add_argument("--sweep", default=None, choices=["gemv", "gemv-tokens"],
                    help="gemv: FP4 and FP8 single GEMVs (one token) over a grid of shapes, each against the "
                         "bare read of its bytes; gemv-tokens: the same with 2, 3 and 4 tokens; one JSON line "
                         "per shape on stdout, and exit")
    ap.add_argument("--copy-calib", action="store_true",
                    help="after the workloads, copy 64 MiB device to device 5 times (the reference transfer for "
                         "scaling HBM byte counters)")
    return ap.parse_args()


LAST_TIMING = {}  # the last graph-timed row's samples, for the headline line


def timed_steps(torch, launch, copies, steps, warmup, use_graph=True, isolated=0):
    """Times exactly `steps` steps (launch(i) issues step i on the current stream) after `warmup`
    untimed ones, and returns (ms per step, steps).

    Graph path: one captured graph holds the warmup steps, then R samples of exactly `steps` steps,
    each between two clock-stamp launches (stbl_amd_clock_stamp: the GPU wall clock as the stamp
    starts), then 8 back-to-back stamp pairs; step i uses weight copy i % copies all the way through,
    so no copy is read again within a pass over the >= 512 MB rotation. The graph is replayed once
    untimed and once timed, with the stream synchronized on both sides. A sample's time is its stamp
    interval minus the median interval of the back-to-back pairs (one stamp launch and its launch
    gap, the instrument's own cost), and ms per step is the median sample over `steps`; R =
    max(1, ceil(10 copies / steps)) so that at least ten passes over the rotation are sampled. HIP
    events around the timed replay give a cross-check over all of its steps.

    isolated > 0 adds that many single launches after the pairs, each alone between two stamps with
    a stamp pair before it (no step of its own kind running before or after it, the condition a
    profiler's serialized dispatches run in); their median, net of the stamps' cost, is reported as
    isolated_launch_us next to the steady-state samples."""
    if not use_graph:
        stream = torch.cuda.Stream()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            for i in range(warmup):
                launch(i % copies)
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for i in range(steps):
                launch(i % copies)
            b.record(stream)
            torch.cuda.synchronize()
        return a.elapsed_time(b) / steps, steps
    from stblarge_amd import _lib

    lib = _lib.load()
    khz = ctypes.c_int(0)
    _lib.check(lib.stbl_amd_clock_rate_khz(ctypes.byref(khz)), "clock_rate_khz")
    if khz.value <= 0:
        raise RuntimeError(f"the GPU reports a wall clock of {khz.value} kHz")
    reps, pairs = max(1, math.ceil(10 * copies / steps)), 8
    iso0 = reps + 1 + 2 * pairs
    stamps = torch.zeros(iso0 + 3 * isolated, dtype=torch.int64, device="cuda:0")
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):

        def stamp(i):
            _lib.check(lib.stbl_amd_clock_stamp(ctypes.c_void_p(stamps.data_ptr()), i, stream.cuda_stream),
                       "clock_stamp")

        for i in range(copies):  # warm the code path before capture
            launch(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            n = 0
            for _ in range(warmup):
                launch(n % copies)
                n += 1
            stamp(0)
            for r in range(reps):
                for _ in range(steps):
                    launch(n % copies)
                    n += 1
                stamp(r + 1)
            for p in range(pairs):
                stamp(reps + 1 + 2 * p)
                stamp(reps + 2 + 2 * p)
            for j in range(isolated):
                stamp(iso0 + 3 * j)
                stamp(iso0 + 3 * j + 1)
                launch(n % copies)
                n += 1
                stamp(iso0 + 3 * j + 2)
        graph.replay()
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        graph.replay()
        ev1.record(stream)
        torch.cuda.synchronize()
    t = stamps.cpu().tolist()
    ms = lambda ticks: ticks / khz.value
    calib = sorted(ms(t[reps + 2 + 2 * p] - t[reps + 1 + 2 * p]) for p in range(pairs))[pairs // 2]
    samples = sorted(ms(t[r + 1] - t[r]) - calib for r in range(reps))
    del graph
    LAST_TIMING.clear()
    LAST_TIMING.update({"samples": reps, "steps_per_sample": steps, "sample_ms_min": samples[0],
                        "sample_ms_median": samples[reps // 2], "sample_ms_max": samples[-1],
                        "stamp_pair_us": calib * 1e3, "clock_khz": khz.value,
                        # cross-check: HIP events around the whole timed replay, over all its steps
                        # (warmup included; the stamps and the graph's start add a little)
                        "events_ms_per_step_whole_replay": ev0.elapsed_time(ev1) / (warmup + reps * steps + isolated)})
    if isolated:
        iso = sorted(ms(t[iso0 + 3 * j + 2] - t[iso0 + 3 * j + 1]) - calib for j in range(isolated))
        LAST_TIMING.update({"isolated_launches": isolated, "isolated_launch_us": iso[isolated // 2] * 1e3})
    return samples[reps // 2] / steps, steps


def gemv_workload(torch, fmt, rows, k, m, steps, warmup, use_graph=True, isolated=0):
    from stblarge_amd import data, ops

    dev = torch.device("cuda:0")
    w = data.weight(rows, k, seed=1, device=dev)
    if fmt == "fp4":
        codes, scales = ops.quant_fp4(w)
        alg = data.algorithmic_bytes_fp4(rows, k, m)
        wbytes = codes.numel() + scales.numel()
    else:
        codes, scales = ops.quant_fp8_b128(w)
        alg = data.algorithmic_bytes_fp8(rows, k, m)
        wbytes = codes.numel() + scales.numel() * 4
    del w
    copies = max(2, math.ceil(ROTATE_BYTES / wbytes))
    cs = [codes.clone() for _ in range(copies)]
    ss = [scales.clone() for _ in range(copies)]
    x = data.activation(m, k, seed=2, device=dev)
    y = torch.empty((m, rows), dtype=torch.bfloat16, device=dev)
    fn = ops.gemv_fp4 if fmt == "fp4" else ops.gemv_fp8

    def launch(i):
        fn(cs[i], ss[i], x, out=y)

    ms, n = timed_steps(torch, launch, copies, steps, warmup, use_graph, isolated=isolated if use_graph else 0)
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": f"{fmt}_gemv_{rows}x{k}_m{m}", "rows": rows, "k": k, "m": m, "ms_per_step": ms,
            "steps": n, "alg_bytes": alg, "GB_s": gbs, "frac_hbm_peak": gbs / PEAK_HBM_GBS, "weight_copies": copies,
            "graph": use_graph}


def gemv_batch_workload(torch, fmt, rows, k, steps, warmup, nb=16, use_graph=True):
    """Sustained GEMV bandwidth: nb same-shape GEMVs per launch (the reference's kMxBatch batching,
    stbl/kernels.h:18-20, is 16; the v2 batches take up to 64, about what the MoE step's gate/up
    launch holds at 4 tokens), every launch on nb different weight matrices from a >= 512 MB
    rotation."""
    from stblarge_amd import data, ops

    dev = torch.device("cuda:0")
    w = data.weight(rows, k, seed=1, device=dev)
    codes, scales = ops.quant_fp4(w) if fmt == "fp4" else ops.quant_fp8_b128(w)
    del w
    wbytes = codes.numel() + scales.numel() * scales.element_size()
    groups = max(2, math.ceil(ROTATE_BYTES / (nb * wbytes)))
    cs = [[codes.clone() for _ in range(nb)] for _ in range(groups)]
    ss = [[scales.clone() for _ in range(nb)] for _ in range(groups)]
    xs = [data.activation(1, k, seed=2, device=dev) for _ in range(nb)]
    ys = [torch.empty((1, rows), dtype=torch.bfloat16, device=dev) for _ in range(nb)]
    f = ops.FP4 if fmt == "fp4" else ops.FP8

    def launch(i):
        ops.gemv_batch(cs[i], ss[i], xs, f, outs=ys)

    ms, n = timed_steps(torch, launch, groups, steps, warmup, use_graph)
    per = data.algorithmic_bytes_fp4(rows, k, 1) if fmt == "fp4" else data.algorithmic_bytes_fp8(rows, k, 1)
    alg = nb * per
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": f"{fmt}_gemv_batch{nb}_{rows}x{k}_m1", "ms_per_step": ms, "gemv_per_launch": nb,
            "steps": n, "alg_bytes": alg, "GB_s": gbs, "frac_hbm_peak": gbs / PEAK_HBM_GBS}


def ffn_workload(torch, fmt, steps, warmup, use_graph=True):
    """C3: one expert FFN (gate/up + SwiGLU, down) at dim 7168, inter 2048, one token."""
    from stblarge_amd import data, ops

    dev = torch.device("cuda:0")
    dim, inter = 7168, 2048
    slot = ops.quant_expert(data.weight(inter, dim, 11, dev), data.weight(inter, dim, 12, dev),
                            data.weight(dim, inter, 13, dev), fmt)
    copies = max(2, math.ceil(ROTATE_BYTES / slot.numel()))
    slots = [slot.clone() for _ in range(copies)]
    x = data.activation(1, dim, seed=14, device=dev)
    y = torch.empty((1, dim), dtype=torch.bfloat16, device=dev)
    work = torch.empty(inter, dtype=torch.bfloat16, device=dev)
    from stblarge_amd import _lib

    lib = _lib.load()

    def launch(i):
        st = ops._stream()
        _lib.check(lib.stbl_amd_expert_ffn(fmt, ops._ptr(y), ops._ptr(slots[i]), ops._ptr(x), 1, dim, inter, 1.0, 0.0,
                                           0, 0, ops._ptr(work), st), "expert_ffn")

    ms, n = timed_steps(torch, launch, copies, steps, warmup, use_graph)
    nbytes, offs = ops.expert_layout(fmt, dim, inter)
    wbytes = sum(ops._mat_bytes(fmt, r, k) for r, k in ((inter, dim), (inter, dim), (dim, inter)))
    alg = wbytes + 2 * dim + 2 * dim
    gbs = alg / (ms * 1e-3) / 1e9
    name = "fp4" if fmt == ops.FP4 else "fp8"
    # the weight bytes of its two launches (gate + up, then down): the bare reads of those byte counts,
    # one launch each, are the floor of a plan whose second launch needs the first's output
    launch_bytes = [2 * ops._mat_bytes(fmt, inter, dim), ops._mat_bytes(fmt, dim, inter)]
    return {"workload": f"{name}_expert_ffn_7168x2048_m1", "ms_per_step": ms, "steps": n, "alg_bytes": alg,
            "GB_s": gbs, "frac_hbm_peak": gbs / PEAK_HBM_GBS, "slot_copies": copies, "launch_bytes": launch_bytes}


def moe_workload(torch, tokens, steps, warmup_steps):
    """C4: routed MoE layer decode, 256 FP4 experts (pinned host pool) + 1 shared, top-8, sigmoid
    router on Zipf(1.1) Gumbel-top-k logits, 64-slot HBM LRU refilled over PCIe."""
    import time as _t

    from stblarge_amd import data, ops
    from stblarge_amd.moe import MoELayer

    dev = torch.device("cuda:0")
    dim, inter, n_exp, topk, slots = data.DIM, data.INTER, data.N_EXPERTS, data.TOPK, data.CACHE_SLOTS
    fmt = ops.FP4
    sb, _ = ops.expert_layout(fmt, dim, inter)
    pool = torch.empty(n_exp * sb, dtype=torch.uint8, pin_memory=True)
    for e in range(n_exp):
        s = ops.quant_expert(data.weight(inter, dim, 1000 + 3 * e, dev), data.weight(inter, dim, 1001 + 3 * e, dev),
                             data.weight(dim, inter, 1002 + 3 * e, dev), fmt)
        pool[e * sb:(e + 1) * sb].copy_(s, non_blocking=False)
    shared = ops.quant_expert(data.weight(inter, dim, 7, dev), data.weight(inter, dim, 8, dev),
                              data.weight(dim, inter, 9, dev), fmt)
    layer = MoELayer(fmt, dim, inter, pool, n_exp, topk, slots, shared_slot=shared, max_tokens=tokens)
    total = warmup_steps + steps
    logits = data.zipf_logits(total * tokens, n_exp, seed=77).view(total, tokens, n_exp).to(dev)
    x = data.activation(tokens, dim, seed=78, device=dev)
    for i in range(warmup_steps):
        layer.forward(x, logits[i])
    torch.cuda.synchronize()
    st0 = layer.cache.stats()
    t0 = _t.perf_counter()
    for i in range(warmup_steps, total):
        layer.forward(x, logits[i])
    torch.cuda.synchronize()
    el = _t.perf_counter() - t0
    st1 = layer.cache.stats()
    hits, misses = st1["hits"] - st0["hits"], st1["misses"] - st0["misses"]
    layer.close()
    del pool
    return {"workload": f"moe_layer_t{tokens}_fp4_256x_top8_lru64", "tokens": tokens, "steps": steps,
            "ms_per_step": el * 1e3 / steps, "tokens_per_s": tokens * steps / el,
            "hit_rate": hits / max(1, hits + misses), "misses_per_token": misses / (tokens * steps),
            "refill_GB_s": (st1["refill_bytes"] - st0["refill_bytes"]) / el / 1e9}


def moe_allhit_workload(torch, tokens, steps, warmup, v41=False, use_graph=True, fp8_shared=False):
    """C4's expert kernels alone with every expert resident (the kernel bound of the layer): per
    step, each token's 8 routed experts are drawn from 64 resident slots (1.5 GB, so weights come
    from HBM) plus the shared expert; algorithmic bytes = every distinct expert's weights once.
    v41: the reference engine's own MoE instead (stbl/model.cu:426-594 at stbl/bench_gemv.py:15's
    shapes): dim 5120, inter 2304, top-6 FP4 experts + an FP8 E8M0 shared expert, official numerics
    (act_quant of the input and of the SwiGLU output), SwiGLU limit 10. fp8_shared: C4's shapes with
    the shared expert in the engine's FP8 E8M0 32x32 format (stbl/model.cu:544-547) instead of FP4."""
    import numpy as np

    from stblarge_amd import data, ops

    dev = torch.device("cuda:0")
    dim, inter, topk, nres = data.DIM, data.INTER, data.TOPK, data.CACHE_SLOTS
    if v41:
        dim, inter, topk = 5120, 2304, 6
    fmt = ops.FP4
    sfmt = ops.FP8_E8M0 if v41 or fp8_shared else fmt
    base = ops.quant_expert(data.weight(inter, dim, 21, dev), data.weight(inter, dim, 22, dev),
                            data.weight(dim, inter, 23, dev), fmt)
    res = [base.clone() for _ in range(nres)]
    shared = ops.quant_expert(data.weight(inter, dim, 24, dev), data.weight(inter, dim, 25, dev),
                              data.weight(dim, inter, 26, dev), sfmt)
    # one shared-expert copy per plan: an engine reads each layer's shared expert once per token with
    # the rest of the model in between, so it must not stay in the 256 MB memory-side cache here either
    shared = [shared] + [shared.clone() for _ in range(15)]
    shapes = ((inter, dim), (inter, dim), (dim, inter))
    wbytes = sum(ops._mat_bytes(fmt, r, k) for r, k in shapes)
    sbytes = sum(ops._mat_bytes(sfmt, r, k) for r, k in shapes)
    rng = np.random.default_rng(5)
    plans = []
    for i in range(16):
        pick = [list(rng.choice(nres, size=topk, replace=False)) for _ in range(tokens)]
        uniq = sorted({e for row in pick for e in row})
        slot_of = {e: i for i, e in enumerate(uniq)}
        plans.append(([res[e] for e in uniq] + [shared[i]], [[slot_of[e] for e in row] for row in pick], len(uniq)))
    w = [[1.0 / topk] * topk for _ in range(tokens)]
    x = data.activation(tokens, dim, seed=24, device=dev)
    y = torch.empty((tokens, dim), dtype=torch.bfloat16, device=dev)
    work = torch.empty(ops.moe_work_bytes(tokens, topk, dim, inter), dtype=torch.uint8, device=dev)

    def launch(i):
        sl, pick, _ = plans[i]
        ops.moe_experts(x, sl, pick, w, fmt, dim, inter, shared=len(sl) - 1, work=work, out=y, shared_fmt=sfmt,
                        official=v41, limit=10.0 if v41 else 0.0)

    ms, n = timed_steps(torch, launch, len(plans), steps, warmup, use_graph)
    alg = np.mean([p[2] for p in plans]) * wbytes + sbytes + 4 * dim * tokens
    gbs = alg / (ms * 1e-3) / 1e9
    name = (f"moe_v41_allhit_t{tokens}_fp4_top6_fp8e8m0_shared" if v41 else
            f"moe_experts_allhit_t{tokens}_fp4" + ("_fp8e8m0_shared" if fp8_shared else ""))
    return {"workload": name, "ms_per_step": ms, "steps": n, "tokens_per_s":
            tokens / (ms * 1e-3), "alg_bytes": alg, "GB_s": gbs, "frac_hbm_peak": gbs / PEAK_HBM_GBS}


def compat_gemv_workload(torch, kind, rows, k, steps, warmup, group_rows=0):
    """The reference ABI's GEMVs at the reference's own benchmark shapes (stbl/bench_gemv.py:15,
    :35-62, :80-85, :93-107): stbl_gemv_mxfp4 on GGUF rows (scale bytes 120, random codes),
    stbl_gemv_fp8 on E8M0 32x32 FP8 (codes < 120, scale bytes 120), stbl_gemv_bf16 (optionally
    grouped x), fp32 x and y, round_out; stbl_gemv_f32 for the router. Unlike the reference's loop,
    every launch reads a different weight copy (>= 512 MB)."""
    from stblarge_amd import _lib, ops

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(rows + k)
    if kind == "mxfp4":
        w = torch.randint(0, 256, (rows, k // 32 * 17), dtype=torch.uint8, device=dev, generator=g)
        w[:, ::17] = 120
        s = None
        wb = w.numel()
    elif kind == "fp8":
        w = torch.randint(0, 120, (rows, k), dtype=torch.uint8, device=dev, generator=g)
        s = torch.full(((rows + 31) // 32, k // 32), 120, dtype=torch.uint8, device=dev)
        wb = w.numel() + s.numel()
    elif kind == "bf16":
        w = (torch.randn((rows, k), device=dev, generator=g) * 0.02).to(torch.bfloat16)
        s = None
        wb = w.numel() * 2
    else:
        w = torch.randn((rows, k), device=dev, generator=g) * 0.02
        s = None
        wb = w.numel() * 4
    copies = max(2, math.ceil(ROTATE_BYTES / wb))
    ws = [w.clone() for _ in range(copies)]
    xrows = (rows + group_rows - 1) // group_rows if group_rows else 1
    x = torch.randn(xrows * k, device=dev, generator=g)
    y = torch.empty(rows, device=dev)
    lib = _lib.load()
    st = ops._stream

    def launch(i):
        if kind == "mxfp4":
            lib.stbl_gemv_mxfp4(ops._ptr(y), ops._ptr(ws[i]), ops._ptr(x), rows, k, st())
        elif kind == "fp8":
            lib.stbl_gemv_fp8(ops._ptr(y), ops._ptr(ws[i]), ops._ptr(s), ops._ptr(x), rows, k, 1, st())
        elif kind == "bf16":
            lib.stbl_gemv_bf16(ops._ptr(y), ops._ptr(ws[i]), ops._ptr(x), rows, k, 1, group_rows, st())
        else:
            lib.stbl_gemv_f32(ops._ptr(y), ops._ptr(ws[i]), ops._ptr(x), rows, k, 0, st())

    launch(0)
    _lib.check(None, f"stbl_gemv_{kind}")
    ms, n = timed_steps(torch, launch, copies, steps, warmup)
    alg = wb + 4 * k * xrows + 4 * rows
    gbs = alg / (ms * 1e-3) / 1e9
    name = f"ref_abi_gemv_{kind}_{rows}x{k}" + (f"_group{group_rows}" if group_rows else "")
    return {"workload": name, "ms_per_step": ms, "steps": n, "alg_bytes": alg,
            "GB_s": gbs, "frac_hbm_peak": gbs / PEAK_HBM_GBS, "weight_copies": copies}


def compat_batch_workload(torch, rows, k, n, steps, warmup):
    """stbl_gemv_mxfp4_batch as the reference engine issues it for one layer's experts
    (stbl/model.cu:536-539: gate and up of every selected expert in one call, then their down
    projections in another): n GGUF matrices per launch, fp32 x quantized by stbl_act_quant_fp8 as
    the engine's is (:516-540), every launch on n different matrices from a >= 512 MB rotation."""
    from stblarge_amd import _lib, ops

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(rows * n + k)
    wb = rows * (k // 32) * 17
    sets = max(2, math.ceil(ROTATE_BYTES / (wb * n)))
    mats = []
    for _ in range(sets * n):
        w = torch.randint(0, 256, (rows, k // 32 * 17), dtype=torch.uint8, device=dev, generator=g)
        w[:, ::17] = 120
        mats.append(w)
    xs = [torch.randn(k, device=dev, generator=g) for _ in range(n)]
    ys = [torch.empty(rows, device=dev) for _ in range(n)]
    P = ctypes.c_void_p
    y_arr = (P * n)(*[y.data_ptr() for y in ys])
    x_arr = (P * n)(*[x.data_ptr() for x in xs])
    w_arrs = [(P * n)(*[mats[i * n + j].data_ptr() for j in range(n)]) for i in range(sets)]
    lib = _lib.load()
    st = ops._stream
    for x in xs:
        lib.stbl_act_quant_fp8(P(x.data_ptr()), k, st())

    def launch(i):
        lib.stbl_gemv_mxfp4_batch(y_arr, w_arrs[i], x_arr, n, rows, k, st())

    launch(0)
    _lib.check(None, "stbl_gemv_mxfp4_batch")
    ms, steps_run = timed_steps(torch, launch, sets, steps, warmup)
    alg = n * (wb + 4 * k + 4 * rows)
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": f"ref_abi_gemv_mxfp4_batch{n}_{rows}x{k}", "ms_per_step": ms, "steps": steps_run,
            "alg_bytes": alg, "GB_s": gbs, "frac_hbm_peak": gbs / PEAK_HBM_GBS, "weight_sets": sets}


def engine_abi_moe_workload(torch, steps, warmup):
    """One token of the reference engine's MoE step issued through the drop-in ABI as
    stbl/model.cu:508-592 issues it, at its V4.1 shapes (dim 5120, inter 2304, top-6 GGUF FP4 experts
    from a >= 512 MB rotation, FP8 E8M0 shared expert, official numerics): act_quant of x, the gate/up
    batch of 12, swiglu_batch, act_quant, the down batch of 6, the shared expert's three stbl_gemv_fp8
    with its SwiGLU and act_quant, a zeroed accumulator, 7 axpys and round_bf16. The same step as
    stbl_amd_moe_experts (moe_v41_allhit_t1) computes it in 3 fused launches."""
    from stblarge_amd import _lib, ops

    dev = torch.device("cuda:0")
    dim, inter, topk, limit = 5120, 2304, 6, 10.0
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    part = lambda rows, k: rows * (k // 32) * 17
    ebytes = 2 * part(inter, dim) + part(dim, inter)
    n_exp = max(topk + 1, math.ceil(ROTATE_BYTES / ebytes))
    experts = []
    for _ in range(n_exp):
        gate, up = (torch.randint(0, 256, (part(inter, dim),), dtype=torch.uint8, device=dev, generator=g)
                    for _ in range(2))
        down = torch.randint(0, 256, (part(dim, inter),), dtype=torch.uint8, device=dev, generator=g)
        for t in (gate, up, down):
            t[::17] = 120
        experts.append((gate, up, down))
    # the shared expert rotates with the routed ones (one copy per plan, below): an engine reads each
    # layer's shared expert once per token, so it must not stay in the 256 MB memory-side cache here
    shared = []
    for _ in range(max(1, n_exp // topk)):
        sh = [torch.randint(0, 120, (r * k,), dtype=torch.uint8, device=dev, generator=g)
              for r, k in ((inter, dim), (inter, dim), (dim, inter))]
        shs = [torch.full((((r + 31) // 32) * (k // 32),), 120, dtype=torch.uint8, device=dev)
               for r, k in ((inter, dim), (inter, dim), (dim, inter))]
        shared.append((sh, shs))
    x = torch.randn(dim, device=dev, generator=g).to(torch.bfloat16).float()
    f32 = lambda n: torch.zeros(n, dtype=torch.float32, device=dev)
    xq, gb, ub, mid, eo = f32(dim), f32(topk * inter), f32(topk * inter), f32(topk * inter), f32(topk * dim)
    sg, su, smid, sout, y = f32(inter), f32(inter), f32(inter), f32(dim), f32(dim)
    P = ctypes.c_void_p
    arr = lambda ts: (P * len(ts))(*[t if isinstance(t, int) else t.data_ptr() for t in ts])
    gu_y = arr([gb.data_ptr() + 4 * j * inter for j in range(topk)] + [ub.data_ptr() + 4 * j * inter for j in range(topk)])
    gu_x = arr([xq] * (2 * topk))
    d_y = arr([eo.data_ptr() + 4 * j * dim for j in range(topk)])
    d_x = arr([mid.data_ptr() + 4 * j * inter for j in range(topk)])
    ws = (ctypes.c_float * topk)(*[0.3, 0.2, 0.15, 0.15, 0.1, 0.1])
    plans = []
    for i in range(max(1, n_exp // topk)):
        sel = [experts[(i * topk + j) % n_exp] for j in range(topk)]
        plans.append((arr([e[0] for e in sel] + [e[1] for e in sel]), arr([e[2] for e in sel]), shared[i]))
    lib = _lib.load()
    st = ops._stream

    def launch(i):
        gu_w, d_w, (sh, shs) = plans[i]
        s = st()
        xq.copy_(x)
        lib.stbl_act_quant_fp8(P(xq.data_ptr()), dim, s)
        lib.stbl_gemv_mxfp4_batch(gu_y, gu_w, gu_x, 2 * topk, inter, dim, s)
        lib.stbl_swiglu_batch(P(mid.data_ptr()), P(gb.data_ptr()), P(ub.data_ptr()), ws, topk, limit, inter, s)
        lib.stbl_act_quant_fp8(P(mid.data_ptr()), topk * inter, s)
        lib.stbl_gemv_mxfp4_batch(d_y, d_w, d_x, topk, dim, inter, s)
        lib.stbl_gemv_fp8(P(sg.data_ptr()), P(sh[0].data_ptr()), P(shs[0].data_ptr()), P(xq.data_ptr()), inter, dim, 1, s)
        lib.stbl_gemv_fp8(P(su.data_ptr()), P(sh[1].data_ptr()), P(shs[1].data_ptr()), P(xq.data_ptr()), inter, dim, 1, s)
        lib.stbl_swiglu_batch(P(smid.data_ptr()), P(sg.data_ptr()), P(su.data_ptr()), (ctypes.c_float * 1)(1.0), 1,
                              limit, inter, s)
        lib.stbl_act_quant_fp8(P(smid.data_ptr()), inter, s)
        lib.stbl_gemv_fp8(P(sout.data_ptr()), P(sh[2].data_ptr()), P(shs[2].data_ptr()), P(smid.data_ptr()), dim,
                          inter, 1, s)
        y.zero_()
        for j in range(topk):
            lib.stbl_axpy(P(y.data_ptr()), P(eo.data_ptr() + 4 * j * dim), 1.0, dim, s)
        lib.stbl_axpy(P(y.data_ptr()), P(sout.data_ptr()), 1.0, dim, s)
        lib.stbl_round_bf16(P(y.data_ptr()), dim, s)

    launch(0)
    _lib.check(None, "engine MoE step through the reference ABI")
    ms, n = timed_steps(torch, launch, len(plans), steps, warmup)
    sh, shs = shared[0]
    alg = topk * ebytes + sum(t.numel() for t in sh + shs) + 4 * dim * 2
    gbs = alg / (ms * 1e-3) / 1e9
    return {"workload": "ref_abi_moe_step_v41_t1", "ms_per_step": ms, "steps": n, "tokens_per_s": 1 / (ms * 1e-3),
            "launches_per_step": 20, "alg_bytes": alg, "GB_s": gbs, "frac_hbm_peak": gbs / PEAK_HBM_GBS}


def ref_method_workload(torch, kind, rows, k, group_rows=0, reps=200):
    """The reference ABI's GEMVs timed the way stbl/bench_gemv.py:18-28 times them, for a
    like-for-like comparison with that script's output: the same weight tensor every launch (so it
    stays in the 256 MB Infinity Cache), launches issued one by one, events around 200 of them after
    10 warmups, and GB/s = weight-tensor bytes / time (stbl/bench_gemv.py:40,48,55,83: the GGUF rows
    with their scale bytes, the FP8 codes without their scales, the bf16 weights). kind "copy" is
    the script's 64 MiB device copy (read + write bytes, 50 launches, :58-61)."""
    from stblarge_amd import _lib, ops

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(rows + k)
    lib = _lib.load()
    st = ops._stream
    y = torch.empty(max(rows, 1), device=dev)
    if kind == "copy":
        a = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        fn, nbytes, reps = (lambda: b.copy_(a)), 2 * a.numel(), 50
    elif kind == "mxfp4":
        w = torch.randint(0, 256, (rows, k // 32 * 17), dtype=torch.uint8, device=dev, generator=g)
        w[:, ::17] = 120
        x = torch.randn(k, device=dev, generator=g)
        fn, nbytes = (lambda: lib.stbl_gemv_mxfp4(ops._ptr(y), ops._ptr(w), ops._ptr(x), rows, k, st())), w.numel()
    elif kind == "fp8":
        w = torch.randint(0, 120, (rows, k), dtype=torch.uint8, device=dev, generator=g)
        sc = torch.full((rows // 32 + 1, k // 32), 120, dtype=torch.uint8, device=dev)
        x = torch.randn(k, device=dev, generator=g)
        fn = lambda: lib.stbl_gemv_fp8(ops._ptr(y), ops._ptr(w), ops._ptr(sc), ops._ptr(x), rows, k, 1, st())
        nbytes = w.numel()
    else:  # bf16, optionally grouped
        w = torch.randn((rows, k), device=dev, generator=g).to(torch.bfloat16)
        xrows = rows // group_rows if group_rows else 1
        x = torch.randn(xrows * k, device=dev, generator=g)
        fn = lambda: lib.stbl_gemv_bf16(ops._ptr(y), ops._ptr(w), ops._ptr(x), rows, k, 1, group_rows, st())
        nbytes = w.numel() * 2
    for _ in range(10):
        fn()
    _lib.check(None, f"ref_method {kind}")
    a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a0.record()
    for _ in range(reps):
        fn()
    a1.record()
    torch.cuda.synchronize()
    us = a0.elapsed_time(a1) / reps * 1000
    name = "ref_method_" + ("device_copy_64MiB" if kind == "copy" else f"gemv_{kind}_{rows}x{k}" +
                            (f"_group{group_rows}" if group_rows else ""))
    return {"workload": name, "us": us, "GB_s": nbytes / us / 1e3, "bytes": nbytes, "reps": reps}


def gemm_workload(torch, fmt, steps, warmup, m=64, n=2048, k=7168, prequant=False, use_graph=True, packed=False):
    """C5: multi-token expert GEMM, M = 64 tokens, W [2048 x 7168] FP4 or FP8 (scaled f8f6f4 MFMA).
    prequant: the activations are quantized outside the timed region and the GEMM proper is timed
    (stbl_amd_gemm_q, fp8_gemm(a, a_s, b, b_s)'s form); otherwise act_quant + GEMM (stbl_amd_gemm).
    packed: the weight codes packed once beforehand into operand order (stbl_amd_gemm_pack), the
    calls stbl_amd_gemm_q_packed / stbl_amd_gemm_packed."""
    from stblarge_amd import _lib, data, ops

    dev = torch.device("cuda:0")
    w = data.weight(n, k, seed=31, device=dev)
    codes, scales = ops.quant_fp4(w) if fmt == ops.FP4 else ops.quant_fp8_b128(w)
    del w
    wbytes = ops._mat_bytes(fmt, n, k)
    copies = max(2, math.ceil(ROTATE_BYTES / wbytes))
    cs = [ops.gemm_pack(codes, fmt) if packed else codes.clone() for _ in range(copies)]
    ss = [scales.clone() for _ in range(copies)]
    x = data.activation(m, k, seed=32, device=dev)
    aq, a_s = ops.act_quant_e4m3(x, 128)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    work = ops.gemm_work(m, n, k, dev)
    lib = _lib.load()

    def launch(i):
        if prequant:
            fn = lib.stbl_amd_gemm_q_packed if packed else lib.stbl_amd_gemm_q
            _lib.check(fn(fmt, ops._ptr(y), ops._ptr(cs[i]), ops._ptr(ss[i]), ops._ptr(aq), ops._ptr(a_s), m, n, k, 128, 0,
                          ops._ptr(work), ops._stream()), "gemm_q")
        else:
            fn = lib.stbl_amd_gemm_packed if packed else lib.stbl_amd_gemm
            _lib.check(fn(fmt, ops._ptr(y), ops._ptr(cs[i]), ops._ptr(ss[i]), ops._ptr(x), m, n, k, 128, 0,
                          ops._ptr(work), ops._stream()), "gemm")

    ms, nsteps = timed_steps(torch, launch, copies, steps, warmup, use_graph)
    alg = wbytes + (m * k + m * k // 128 if prequant else 2 * m * k) + 2 * m * n
    flops = 2.0 * m * n * k
    name = "fp4" if fmt == ops.FP4 else "fp8"
    peak_tf = 5000.0  # e4m3 activations: the MFMA runs at the fp8 rate for both weight formats
    return {"workload": f"{name}_gemm{'_q' if prequant else ''}{'_packed' if packed else ''}_m{m}_{n}x{k}",
            "ms_per_step": ms, "steps": nsteps,
            "alg_bytes": alg, "GB_s": alg / (ms * 1e-3) / 1e9, "frac_hbm_peak": alg / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
            "TFLOP_s": flops / (ms * 1e-3) / 1e12, "frac_mfma_peak": flops / (ms * 1e-3) / 1e12 / peak_tf}


def file_tier_workload(torch, mode, readers=8, n_experts=40, per_lookup=1, lookups=30):
    """The expert cache's file tier: misses read from a GGUF file of V4.1 routed experts (dim 5120,
    inter 2304, MXFP4: 18,800,640 bytes per expert, the size the reference's SSD bench reads,
    scripts/ssd_expert_bench.py:10) in 2 MiB pieces by `readers` threads, copied to the device and
    repacked into FP4 slots. Each lookup asks for per_lookup experts that are not cached; the time
    is host wall clock from the lookup to the end of the repack. mode: "direct" (O_DIRECT reads from
    the disk), "cold" (buffered reads after the file's pages were dropped from the page cache) or
    "warm" (buffered reads of a file the page cache holds: the pipeline without the disk)."""
    import shutil
    import time as _t

    import numpy as np

    from stblarge_amd import gguf
    from stblarge_amd.moe import ExpertCache

    dim, inter = 5120, 2304
    d = os.path.join(ROOT, "_direct_io_tmp")
    os.makedirs(d, exist_ok=True)
    path = os.path.join(d, "bench_experts.gguf")
    part = dim * inter // 32 * 17
    rng = np.random.default_rng(5)
    tensors = [(gguf.expert_tensor(0, p), gguf.QT_MXFP4, [dim, inter, n_experts] if p != "down" else [inter, dim, n_experts],
                lambda: (np.frombuffer(rng.bytes(part), np.uint8) for _ in range(n_experts))) for p in ("gate", "up", "down")]
    gguf.write(path, tensors, alignment=16384)
    if mode == "cold":
        fd = os.open(path, os.O_RDONLY)
        os.fsync(fd)
        os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
        os.close(fd)
    try:
        cache = ExpertCache.from_gguf(2 * per_lookup, path, readers=readers, direct=mode == "direct")
        info0 = cache.file_info()
        order = list(np.random.default_rng(6).permutation(n_experts))
        lat = []
        for i in range(lookups):
            ids = [int(order[(i * per_lookup + j) % n_experts]) for j in range(per_lookup)]
            t0 = _t.perf_counter()
            cache.lookup(ids)
            torch.cuda.synchronize()
            lat.append(_t.perf_counter() - t0)
            cache.mark_used()
        info = cache.file_info()
        cache.close()
    finally:
        shutil.rmtree(d, ignore_errors=True)
    lat.sort()
    med = lat[len(lat) // 2]
    return {"workload": f"expert_file_{mode}_v41_{per_lookup}x_r{readers}",
            "mode": mode, "direct": bool(info["direct"]), "readers": readers, "experts_per_lookup": per_lookup,
            "expert_bytes": 3 * part, "lookups": lookups, "ms_per_lookup_median": med * 1e3,
            "ms_per_lookup_p90": lat[int(0.9 * len(lat))] * 1e3, "ms_per_expert": med * 1e3 / per_lookup,
            "GB_s": 3 * part * per_lookup / med / 1e9,
            "read_share": (info["read_ns"] - info0["read_ns"]) / 1e9 / sum(lat)}


def file_stack_workload(torch, guess_quality, n_layers=4, n_experts=24, topk=6, slots=16, tokens=6, readers=4,
                        pf_readers=8, pf_m=8):
    """Decode through n_layers routed MoE layers whose experts (V4.1 shape, 18.8 MB each) live in one
    GGUF file behind a 16-slot file-backed cache, reading misses with O_DIRECT. guess_quality None:
    no prefetch; q in [0, 1]: after each layer, pf_m guesses for the next layer are queued, each of
    its true top-k experts included with probability q, the rest drawn at random (the reference's
    stale-router prefetch, stbl/model.cu:555-586, with a controlled guess accuracy). Time per token
    = all layers' lookups and kernels, host wall clock."""
    import shutil
    import time as _t

    import numpy as np

    from stblarge_amd import data, gguf, ops
    from stblarge_amd.moe import ExpertCache, MoELayer

    dim, inter = 5120, 2304
    dev = torch.device("cuda:0")
    d = os.path.join(ROOT, "_direct_io_tmp")
    os.makedirs(d, exist_ok=True)
    path = os.path.join(d, "bench_stack.gguf")
    nb = dim * inter // 32
    rng = np.random.default_rng(7)

    def blocks():  # valid MXFP4 blocks: random codes, scale bytes 118..125
        for _ in range(n_experts):
            b = np.frombuffer(rng.bytes(nb * 17), np.uint8).reshape(nb, 17).copy()
            b[:, 0] = 118 + (b[:, 0] & 7)
            yield b
    tensors = []
    for l in range(n_layers):
        for p in ("gate", "up", "down"):
            tensors.append((gguf.expert_tensor(l, p), gguf.QT_MXFP4,
                            [dim, inter, n_experts] if p != "down" else [inter, dim, n_experts], blocks))
    gguf.write(path, tensors, alignment=16384)
    try:
        cache = ExpertCache.from_gguf(slots, path, n_layers=n_layers, readers=readers, direct=True)
        if guess_quality is not None:
            cache.enable_prefetch(pf_readers)
        stack = [MoELayer(ops.FP4, dim, inter, None, n_experts, topk, slots, cache=cache, layer=l) for l in range(n_layers)]
        grng = np.random.default_rng(8)
        logits = [[data.zipf_logits(1, n_experts, seed=100 * t + l).to(dev) for l in range(n_layers)] for t in range(tokens + 1)]
        true = [[[int(e) for e in torch.topk(logits[t][l][0], topk).indices] for l in range(n_layers)] for t in range(tokens + 1)]
        x = data.activation(1, dim, seed=9, device=dev)
        times = []
        for t in range(tokens + 1):  # token 0 warms the caches and readers
            torch.cuda.synchronize()
            t0 = _t.perf_counter()
            for l in range(n_layers):
                stack[l].forward(x, logits[t][l])
                nt, nl = (t, l + 1) if l + 1 < n_layers else (t + 1, 0)
                if guess_quality is not None and nt <= tokens:
                    keep = [e for e in true[nt][nl] if grng.random() < guess_quality]
                    rest = [int(e) for e in grng.permutation(n_experts) if e not in keep]
                    cache.prefetch((keep + rest)[:pf_m], nl)
            torch.cuda.synchronize()
            times.append(_t.perf_counter() - t0)
        st = cache.stats()
        pst = cache.prefetch_stats() if guess_quality is not None else None
        info = cache.file_info()
        cache.close()
    finally:
        shutil.rmtree(d, ignore_errors=True)
    ms = 1e3 * sum(times[1:]) / tokens
    name = "off" if guess_quality is None else f"q{guess_quality:g}"
    return {"workload": f"expert_file_stack_{n_layers}l_v41_top{topk}_prefetch_{name}", "ms_per_token": ms,
            "tokens_per_s": 1e3 / ms, "hit_rate": st["hits"] / max(1, st["hits"] + st["misses"]),
            "demand_GB_read": info["bytes_read"] / 1e9, "prefetch": pst, "direct": bool(info["direct"])}


def read_floor_workload(torch, nbytes, steps, warmup):
    """The bare streaming read of nbytes in one launch (stbl_amd_read_floor), timed exactly as the
    GEMV rows are: graph replays of launches that each read a different slice of a >= 512 MB buffer
    (so the 256 MB Infinity Cache cannot serve repeats), exact-K samples as timed_steps takes them."""
    from stblarge_amd import _lib, ops

    dev = torch.device("cuda:0")
    span = (nbytes + 4095) // 4096 * 4096
    copies = max(2, math.ceil(ROTATE_BYTES / span))
    buf = torch.randint(0, 256, (copies * span,), dtype=torch.uint8, device=dev)
    sink = torch.empty(int(_lib.load().stbl_amd_read_floor_sink_words(nbytes)), dtype=torch.int32, device=dev)
    lib = _lib.load()

    def launch(i):
        _lib.check(lib.stbl_amd_read_floor(ctypes.c_void_p(buf.data_ptr() + i * span), nbytes, ops._ptr(sink),
                                           ops._stream()), "read_floor")

    ms, n = timed_steps(torch, launch, copies, steps, warmup)
    gbs = nbytes / (ms * 1e-3) / 1e9
    del buf
    return {"workload": f"read_floor_{nbytes}B", "bytes": nbytes, "ms_per_step": ms, "steps": n, "GB_s": gbs,
            "frac_hbm_peak": gbs / PEAK_HBM_GBS}


def attach_floor(row, floors):
    """Adds the row's fraction of the bare-read floor for its byte count (the same bytes in one
    launch, timed the same way) next to its fraction of peak; for a row of several dependent launches
    (launch_bytes), also the sum of the bare reads of each launch's bytes and the row's time against
    it."""
    f = floors.get(int(row["alg_bytes"]))
    if f:
        row["read_floor_GB_s"] = f["GB_s"]
        row["frac_of_read_floor"] = row["GB_s"] / f["GB_s"]
    parts = [floors.get(int(b)) for b in row.get("launch_bytes", ())]
    if parts and all(parts):
        t = sum(p["ms_per_step"] for p in parts)
        row["launch_floors_us"] = 1e3 * t
        row["frac_of_launch_floors"] = t / row["ms_per_step"]
    return row


def measured_traffic():
    """HBM bytes per launch of the headline kernel from the committed rocprofv3 counter summary
    (profiles/gemv_fp4_2048x7168_traffic.md, line `traffic_bytes_per_launch: N`), or None."""
    path = os.path.join(ROOT, "profiles", "gemv_fp4_2048x7168_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def cpu_baseline(seconds):
    """ref/kernel.py's own CPU method for the headline workload (fp4_gemm, ref/kernel.py:94-102,
    restated in oracle.fp4_gemm_torch): per call the FP4 codes and E8M0 scales are dequantized into
    an fp32 [2048 x 7168] matrix and x @ W^T runs in fp32 on every core this process may use, with a
    bf16 result. Repeated for about `seconds`; algorithmic bytes per call as for the GPU row."""
    import torch

    import oracle
    from stblarge_amd import data

    rows, k = 2048, 7168
    cores = len(os.sched_getaffinity(0))
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    w = data.weight(rows, k, seed=1)
    codes, scales = oracle.quant_fp4(w.numpy())
    codes, scales = torch.from_numpy(codes), torch.from_numpy(scales)
    x = data.activation(1, k, seed=2)
    alg = data.algorithmic_bytes_fp4(rows, k, 1)
    for _ in range(3):  # warm
        oracle.fp4_gemm_torch(x, codes, scales)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.fp4_gemm_torch(x, codes, scales)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    torch.set_num_threads(prev)
    return {"value": alg * reps / el / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{reps} x fp4 GEMV 2048x7168 m=1 in {el:.1f} s by ref/kernel.py's method (torch CPU: dequant to "
                      f"fp32, x @ W^T, bf16 out; oracle.fp4_gemm_torch) on {cores} threads of {_cpu_model()} "
                      f"(os.cpu_count() {os.cpu_count()}); {el / reps * 1e3:.2f} ms per GEMV"}


def cpu_scalar_oracle(seconds):
    """The oracle's scalar C GEMV (oracle/stbl_oracle.c orc_gemv_fp4, one thread, fp64 accumulation)
    on the headline shape, repeated for about `seconds`: a second CPU row."""
    import oracle
    from stblarge_amd import data

    rows, k = 2048, 7168
    w = data.weight(rows, k, seed=1)
    codes, scales = oracle.quant_fp4(w.numpy())
    x = data.activation(1, k, seed=2).float().numpy()
    alg = data.algorithmic_bytes_fp4(rows, k, 1)
    oracle.gemv_fp4(codes, scales, x)  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.gemv_fp4(codes, scales, x)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"workload": "cpu_scalar_oracle_fp4_gemv_2048x7168", "GB_s": alg * reps / el / 1e9, "cores": 1,
            "ms_per_gemv": el / reps * 1e3,
            "sample": f"{reps} x orc_gemv_fp4 (scalar C, fp64 accumulate) in {el:.1f} s on one core of {_cpu_model()}"}


# rows whose figures the stdout line carries (every row goes to stderr and to --rows-out)
LINE_ROWS = (
    "fp4_gemv_7168x2048_m1", "fp8_gemv_2048x7168_m1", "fp8_gemv_7168x2048_m1", "fp4_gemv_2048x7168_m4",
    "fp8_gemv_2048x7168_m4", "fp4_gemv_batch16_7168x2048_m1", "fp8_gemv_batch16_7168x2048_m1",
    "fp4_gemv_batch64_7168x2048_m1", "fp8_gemv_batch64_7168x2048_m1", "fp4_expert_ffn_7168x2048_m1",
    "fp8_expert_ffn_7168x2048_m1", "fp4_gemm_q_m64_2048x7168", "fp8_gemm_q_m64_2048x7168", "fp4_gemm_m64_2048x7168",
    "fp8_gemm_m64_2048x7168", "fp4_gemm_q_m64_7168x2048", "fp4_gemm_q_packed_m64_2048x7168",
    "fp8_gemm_q_packed_m64_2048x7168", "fp4_gemm_packed_m64_2048x7168", "fp8_gemm_packed_m64_2048x7168",
    "ref_abi_gemv_mxfp4_2304x5120",
    "ref_abi_gemv_mxfp4_5120x2304", "ref_abi_gemv_fp8_2304x5120", "ref_abi_gemv_mxfp4_batch12_2304x5120",
    "ref_abi_gemv_mxfp4_batch6_5120x2304", "ref_abi_moe_step_v41_t1", "moe_experts_allhit_t1_fp4",
    "moe_experts_allhit_t4_fp4", "moe_experts_allhit_t1_fp4_fp8e8m0_shared", "moe_v41_allhit_t1_fp4_top6_fp8e8m0_shared",
    "moe_v41_allhit_t4_fp4_top6_fp8e8m0_shared", "moe_layer_t1_fp4_256x_top8_lru64", "moe_layer_t4_fp4_256x_top8_lru64",
    "expert_file_direct_v41_1x_r8", "expert_file_stack_4l_v41_top6_prefetch_q1", "read_floor_7817216B",
)
LINE_MAX_BYTES = 4096


def _r(v, nd=3):
    """v rounded to nd significant digits (None stays None)."""
    if v is None or v == 0:
        return v
    return round(v, max(0, nd - 1 - int(math.floor(math.log10(abs(v))))))


def compact_row(r):
    """A row's figures for the stdout line: [us per step, GB/s, fraction of 8 TB/s] for GEMV-like rows
    (with TFLOP/s for GEMMs, tokens/s for MoE steps); a short dict for the LRU, file-tier and CPU rows."""
    if "hit_rate" in r and "refill_GB_s" in r:
        return {"ms": _r(r["ms_per_step"]), "tok_s": _r(r["tokens_per_s"]), "hit": _r(r["hit_rate"]),
                "refill_GB_s": _r(r["refill_GB_s"])}
    if "ms_per_lookup_median" in r:
        return {"ms_per_expert": _r(r["ms_per_expert"]), "GB_s": _r(r["GB_s"]), "direct": r["direct"]}
    if "ms_per_token" in r:
        return {"ms_per_token": _r(r["ms_per_token"]), "hit": _r(r["hit_rate"])}
    if "ms_per_gemv" in r:
        return {"GB_s": _r(r["GB_s"]), "cores": r["cores"]}
    out = [_r(r["ms_per_step"] * 1e3), _r(r["GB_s"]), _r(r["frac_hbm_peak"])]
    if "TFLOP_s" in r:
        out.append(_r(r["TFLOP_s"]))
    elif "tokens_per_s" in r:
        out.append(_r(r["tokens_per_s"]))
    return out


def stderr_text(r):
    """One short human-readable line per row."""
    w = r["workload"]
    if "hit_rate" in r and "refill_GB_s" in r:
        return (f"# {w}: {r['ms_per_step']:.3f} ms/step, {r['tokens_per_s']:.0f} tok/s, hit {r['hit_rate']:.3f}, "
                f"refill {r['refill_GB_s']:.1f} GB/s")
    if "ms_per_lookup_median" in r:
        return f"# {w}: {r['ms_per_expert']:.2f} ms/expert, {r['GB_s']:.2f} GB/s"
    if "ms_per_token" in r:
        return f"# {w}: {r['ms_per_token']:.1f} ms/token, hit {r['hit_rate']:.2f}"
    if "us" in r:  # stbl/bench_gemv.py's own method
        return f"# {w}: {r['us']:.2f} us, {r['GB_s']:.0f} GB/s"
    if "ms_per_gemv" in r:
        return f"# {w}: {r['GB_s']:.2f} GB/s"
    t = f"# {w}: {r['ms_per_step'] * 1e3:.2f} us, {r['GB_s']:.0f} GB/s ({100 * r['frac_hbm_peak']:.1f}%)"
    if "TFLOP_s" in r:
        t += f", {r['TFLOP_s']:.0f} TFLOP/s"
    elif "tokens_per_s" in r:
        t += f", {r['tokens_per_s']:.0f} tok/s"
    if "frac_of_read_floor" in r:
        t += f", {100 * r['frac_of_read_floor']:.0f}% of bare read"
    return t


def make_line(head, extra, cpu, timing, warmup, traffic=None, profiled=None):
    """The one JSON line bench.py prints on stdout (at most LINE_MAX_BYTES): the headline row's
    figures with its roofline, the target shape's rows, the CPU baseline, the timing samples and the
    LINE_ROWS figures of the other rows that ran."""
    gbs = head["GB_s"]
    target = {}
    for key, name in (("fp4", "fp4_gemv_7168x2048_m1"), ("fp8", "fp8_gemv_7168x2048_m1"),
                      ("fp4_batch16", "fp4_gemv_batch16_7168x2048_m1"), ("fp8_batch16", "fp8_gemv_batch16_7168x2048_m1"),
                      ("fp4_batch64", "fp4_gemv_batch64_7168x2048_m1"), ("fp8_batch64", "fp8_gemv_batch64_7168x2048_m1")):
        if name in extra:
            target[key] = {"us": _r(extra[name]["ms_per_step"] * 1e3), "GB_s": _r(extra[name]["GB_s"]),
                           "frac": _r(extra[name]["frac_hbm_peak"])}
    roof = {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic,
            "frac_of_read_floor": _r(head.get("frac_of_read_floor"))}
    if "isolated_launch_us" in timing:
        iso = timing["isolated_launch_us"]
        roof["isolated_launch_us"] = _r(iso, 4)
        roof["isolated_frac"] = round(head["alg_bytes"] / (iso * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)
    if profiled:
        roof["profiled"] = profiled
    tm = {k: (_r(v, 4) if isinstance(v, float) else v) for k, v in timing.items()}
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e2m1 weights x bf16 activations, f32 accumulate",
        "data": "synthetic (seeded N(0,0.02) weights quantized on the GPU, N(0,1) bf16 x)",
        "config": {"workload": head["workload"], "rows": head["rows"], "k": head["k"], "m": head["m"],
                   "weight_copies": head["weight_copies"],
                   "rotation_MB": round(head["weight_copies"] * head["alg_bytes"] / 1e6, 1)},
        "roofline": roof,
        "target_7168x2048": target,
        "cpu_baseline": cpu,
        "timing": tm,
        "extra_cols": "[us/step, GB/s, frac of 8 TB/s, TFLOP/s | tok/s]",
        "extra": {n: compact_row(extra[n]) for n in LINE_ROWS if n in extra},
    }
    return line


def profiled_headline():
    """The headline kernel's figures from the committed rocprofv3 kernel-trace summary
    (profiles/gemv_fp4_2048x7168_kernel_trace.md, `profiled_*:` lines), or None."""
    path = os.path.join(ROOT, "profiles", "gemv_fp4_2048x7168_kernel_trace.md")
    out = {}
    try:
        for line in open(path):
            if line.startswith("profiled_") and ":" in line:
                k, v = line.split(":", 1)
                out[k.strip()[len("profiled_"):]] = float(v.split()[0])
    except (OSError, ValueError):
        return None
    return out or None


def trace_summary(path, kernel_regex):
    """Per-dispatch figures of a rocprofv3 --kernel-trace CSV (…_kernel_trace.csv) for the kernels
    whose name matches kernel_regex: calls, median and mean duration, and the median and mean
    start-to-start spacing and idle gap between consecutive dispatches of those kernels with no other
    dispatch between them (the step time the profiled run itself saw). Returns a dict (ns)."""
    import csv
    import re
    import statistics

    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Start_Timestamp"]))
    pat = re.compile(kernel_regex)
    hit = [i for i, r in enumerate(rows) if pat.search(r["Kernel_Name"])]
    st = [int(r["Start_Timestamp"]) for r in rows]
    en = [int(r["End_Timestamp"]) for r in rows]
    dur = [en[i] - st[i] for i in hit]
    nxt = [(i, j) for i, j in zip(hit, hit[1:]) if j == i + 1]
    sp = [st[j] - st[i] for i, j in nxt]
    gap = [st[j] - en[i] for i, j in nxt]
    med = lambda v: statistics.median(v) if v else None
    avg = lambda v: statistics.mean(v) if v else None
    return {"calls": len(hit), "dur_median_ns": med(dur), "dur_mean_ns": avg(dur), "spacing_median_ns": med(sp),
            "spacing_mean_ns": avg(sp), "gap_median_ns": med(gap), "pairs": len(nxt)}


def trace_table(path, kernel_regex):
    """Per (kernel, grid) rows of a rocprofv3 --kernel-trace CSV for the kernels matching kernel_regex:
    calls and median / mean duration (ns), so that rows of one run that share a kernel (by shape)
    are told apart. Returns a list of dicts."""
    import csv
    import re
    import statistics

    pat = re.compile(kernel_regex)
    groups = {}
    for r in csv.DictReader(open(path)):
        if not pat.search(r["Kernel_Name"]):
            continue
        key = (r["Kernel_Name"], r["Grid_Size_X"], r["Grid_Size_Y"], r["Workgroup_Size_X"])
        groups.setdefault(key, []).append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    return [{"kernel": k[0], "grid": f"{k[1]}x{k[2]}", "workgroup": int(k[3]), "calls": len(v),
             "median_ns": statistics.median(v), "mean_ns": round(statistics.mean(v))} for k, v in groups.items()]


def counter_table(path, kernel_regex):
    """Per (kernel, grid, counter) medians of a rocprofv3 --pmc counter_collection CSV for the kernels
    matching kernel_regex. Returns a list of dicts."""
    import csv
    import re
    import statistics

    pat = re.compile(kernel_regex)
    groups = {}
    for r in csv.DictReader(open(path)):
        if not pat.search(r["Kernel_Name"]):
            continue
        key = (r["Kernel_Name"], r["Grid_Size"], r["Counter_Name"])
        groups.setdefault(key, []).append(float(r["Counter_Value"]))
    return [{"kernel": k[0], "grid": k[1], "counter": k[2], "dispatches": len(v), "median": statistics.median(v)}
            for k, v in sorted(groups.items())]


def counter_last(path, kernel_regex, n):
    """The last n dispatches (by dispatch id) of the kernels matching kernel_regex in a rocprofv3 --pmc
    counter_collection CSV, one dict per (dispatch, counter)."""
    import csv
    import re

    pat = re.compile(kernel_regex)
    rows = [r for r in csv.DictReader(open(path)) if pat.search(r["Kernel_Name"])]
    ids = sorted({int(r["Dispatch_Id"]) for r in rows})[-n:]
    keep = set(ids)
    return [{"dispatch": int(r["Dispatch_Id"]), "kernel": r["Kernel_Name"], "grid": r["Grid_Size"],
             "counter": r["Counter_Name"], "value": float(r["Counter_Value"])}
            for r in sorted(rows, key=lambda r: int(r["Dispatch_Id"])) if int(r["Dispatch_Id"]) in keep]


SWEEP_ROWS = (512, 1024, 2048, 4096, 7168, 16384)
SWEEP_K = (1024, 2048, 4096, 7168)


def gemv_sweep(torch, steps, warmup, tokens=(1,)):
    """The single-GEMV tile plans over a grid of shapes (rows x K, each token count): per shape the
    GEMV's time and its bare-read floor (the same bytes in one launch), both graph-timed as the rows
    are."""
    for m in tokens:
        for fmt in ("fp4", "fp8"):
            for rows in SWEEP_ROWS:
                for k in SWEEP_K:
                    r = gemv_workload(torch, fmt, rows, k, m, steps, warmup)
                    f = read_floor_workload(torch, int(r["alg_bytes"]) // 16 * 16, steps, warmup)
                    print(json.dumps({"fmt": fmt, "m": m, "rows": rows, "k": k, "us": _r(r["ms_per_step"] * 1e3, 4),
                                      "GB_s": _r(r["GB_s"]), "frac_hbm_peak": _r(r["frac_hbm_peak"]),
                                      "floor_us": _r(f["ms_per_step"] * 1e3, 4),
                                      "frac_of_read_floor": _r(f["ms_per_step"] / r["ms_per_step"])}), flush=True)
                    torch.cuda.empty_cache()


def main():
    args = parse()
    if args.counter_summary:
        rows = (counter_last(args.counter_summary, args.trace_kernel, args.counter_last) if args.counter_last > 0
                else counter_table(args.counter_summary, args.trace_kernel))
        for row in rows:
            print(json.dumps(row))
        return
    if args.trace_summary:
        if args.trace_by_grid:
            for row in trace_table(args.trace_summary, args.trace_kernel):
                print(json.dumps(row))
        else:
            print(json.dumps(trace_summary(args.trace_summary, args.trace_kernel)))
        return
    if args.steps < 1 or args.warmup < 0:
        print(f"bench.py needs --steps >= 1 and --warmup >= 0 (got {args.steps}, {args.warmup})", file=sys.stderr)
        sys.exit(2)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the path is single-GPU; see the sharding notes): --gpus {args.gpus} "
              "is not supported", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    from stblarge_amd import _lib

    _lib.load()  # fails loudly when the library was not built
    K, W, graph = args.steps, args.warmup, not args.no_graph
    if args.sweep:
        gemv_sweep(torch, K, W, (1,) if args.sweep == "gemv" else (2, 3, 4))
        return
    extra = {}

    def report(r):
        extra[r["workload"]] = r
        print(stderr_text(r), file=sys.stderr, flush=True)

    head = gemv_workload(torch, "fp4", 2048, 7168, 1, K, W, use_graph=graph, isolated=64)
    head_timing = dict(LAST_TIMING) if graph else {"samples": 1, "events": True}
    print(stderr_text(head), file=sys.stderr, flush=True)
    if args.only in ("all", "gemv"):
        for fmt, rows, k, m in (("fp4", 7168, 2048, 1), ("fp8", 2048, 7168, 1), ("fp8", 7168, 2048, 1),
                                ("fp4", 2048, 7168, 4), ("fp8", 2048, 7168, 4)):
            report(gemv_workload(torch, fmt, rows, k, m, K, W, use_graph=graph))
    if args.only in ("all", "gemv", "batch"):
        for fmt, rows, k, nb in (("fp4", 7168, 2048, 16), ("fp4", 2048, 7168, 16), ("fp8", 7168, 2048, 16),
                                 ("fp8", 2048, 7168, 16), ("fp4", 7168, 2048, 64), ("fp4", 2048, 7168, 64),
                                 ("fp8", 7168, 2048, 64)):
            report(gemv_batch_workload(torch, fmt, rows, k, K, W, nb=nb, use_graph=graph))
    if args.only in ("all", "ffn"):
        from stblarge_amd import ops

        for fmt in (ops.FP4, ops.FP8):
            report(ffn_workload(torch, fmt, K, W, use_graph=graph))
    if args.only in ("all", "gemm"):
        from stblarge_amd import ops

        for fmt, pq, n, k in [(ops.FP4, True, 2048, 7168), (ops.FP8, True, 2048, 7168), (ops.FP4, False, 2048, 7168),
                              (ops.FP8, False, 2048, 7168), (ops.FP4, True, 7168, 2048)]:
            report(gemm_workload(torch, fmt, K, W, n=n, k=k, prequant=pq, use_graph=graph))
        # the same GEMMs on weights packed once into operand order (stbl_amd_gemm_pack)
        for fmt, pq, n, k in [(ops.FP4, True, 2048, 7168), (ops.FP8, True, 2048, 7168), (ops.FP4, False, 2048, 7168),
                              (ops.FP8, False, 2048, 7168), (ops.FP4, True, 7168, 2048)]:
            report(gemm_workload(torch, fmt, K, W, n=n, k=k, prequant=pq, use_graph=graph, packed=True))
    if args.only in ("all", "refabi"):
        for kind, rows, k, grp in (("mxfp4", 2304, 5120, 0), ("mxfp4", 5120, 2304, 0), ("fp8", 2304, 5120, 0),
                                   ("fp8", 5120, 2304, 0), ("bf16", 4096, 5120, 0), ("fp8", 32768, 1280, 0),
                                   ("fp8", 5120, 8192, 0), ("fp8", 1280, 5120, 0), ("fp8", 512, 5120, 0),
                                   ("bf16", 8192, 4096, 1024), ("f32", 256, 5120, 0)):
            report(compat_gemv_workload(torch, kind, rows, k, K, W, grp))
        # the engine's expert batches at V4.1 shapes, top-6: 12 gate/up matrices, then 6 down
        for rows, k, n in ((2304, 5120, 12), (5120, 2304, 6)):
            report(compat_batch_workload(torch, rows, k, n, K, W))
        report(engine_abi_moe_workload(torch, K, W))
        # stbl/bench_gemv.py's own method and rows (:95-107): cache-resident weights, eager launches
        for kind, rows, k, grp in (("mxfp4", 2304, 5120, 0), ("mxfp4", 5120, 2304, 0), ("fp8", 2304, 5120, 0),
                                   ("fp8", 5120, 2304, 0), ("bf16", 4096, 5120, 0), ("bf16", 8192, 4096, 1024),
                                   ("fp8", 32768, 1280, 0), ("fp8", 5120, 8192, 0), ("fp8", 1280, 5120, 0),
                                   ("fp8", 512, 5120, 0), ("copy", 0, 0, 0)):
            report(ref_method_workload(torch, kind, rows, k, grp))
    if args.only in ("all", "moe", "moeallhit"):
        for t, v41, f8s in ((1, False, False), (4, False, False), (1, False, True), (4, False, True), (1, True, False),
                            (4, True, False)):
            report(moe_allhit_workload(torch, t, K, W, v41=v41, use_graph=graph, fp8_shared=f8s))
        for t in ((1, 4) if args.only != "moeallhit" else ()):
            report(moe_workload(torch, t, args.moe_steps, args.moe_warmup))
    if args.only in ("all", "file"):
        for mode, per, readers in (("direct", 1, 8), ("direct", 6, 8), ("direct", 1, 4), ("direct", 1, 16),
                                   ("cold", 1, 8), ("cold", 6, 8), ("warm", 1, 8), ("warm", 6, 8)):
            report(file_tier_workload(torch, mode, readers, per_lookup=per, lookups=30 if per == 1 else 6))
    if args.only in ("all", "filestack"):
        for q in (None, 0.0, 0.5, 1.0):
            report(file_stack_workload(torch, q))
    if args.eager:
        r = gemv_workload(torch, "fp4", 2048, 7168, 1, K, W, use_graph=False)
        r["workload"] += "_eager"
        report(r)
    if args.only in ("all", "fp4", "gemv", "batch", "ffn", "floor"):
        # bare-read floors at the single-launch rows' byte counts: FP4 / FP8 GEMV, FP4 / FP8 expert
        # FFN, 16 FP4 / FP8 GEMVs per launch, 64 FP4 / FP8 GEMVs per launch; then the FFN launches'
        # own (FP4 gate + up, down; FP8 gate + up, down)
        floors = {}
        for nbytes in (7817216, 14702080, 23425024, 44079616, 125075456, 235233280, 500301824, 940933120,
                       15597568, 7798784, 29367296, 14683648):
            r = read_floor_workload(torch, nbytes, K, W)
            floors[nbytes] = r
            report(r)
        for row in [head] + list(extra.values()):
            if "alg_bytes" in row and not row["workload"].startswith("read_floor"):
                attach_floor(row, floors)
                if "frac_of_launch_floors" in row:
                    print(f"# {row['workload']}: {100 * row['frac_of_launch_floors']:.0f}% of its launches' bare reads "
                          f"({row['launch_floors_us']:.2f} us)", file=sys.stderr, flush=True)
        if "frac_of_read_floor" in head:
            print(f"# headline: {100 * head['frac_of_read_floor']:.1f}% of the bare read of its bytes",
                  file=sys.stderr, flush=True)
    if "isolated_launch_us" in head_timing:
        print(f"# headline launch alone between stamps: {head_timing['isolated_launch_us']:.2f} us (median of "
              f"{head_timing['isolated_launches']})", file=sys.stderr, flush=True)
    if args.copy_calib:
        a = torch.empty(64 << 20, dtype=torch.uint8, device="cuda:0")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_seconds)
        extra["cpu_scalar_oracle"] = cpu_scalar_oracle(min(args.cpu_seconds, 5.0))
        print(f"# cpu baseline: {cpu['value']:.2f} GB/s on {cpu['cores']} threads; scalar oracle "
              f"{extra['cpu_scalar_oracle']['GB_s']:.2f} GB/s on 1", file=sys.stderr, flush=True)
    if args.rows_out:
        with open(args.rows_out, "w") as f:
            json.dump({"head": head, "timing": head_timing, "cpu_baseline": cpu, "rows": extra}, f, indent=1)
    line = make_line(head, extra, cpu, head_timing, W, traffic=measured_traffic(), profiled=profiled_headline())
    text = json.dumps(line, separators=(",", ":"))
    if len(text) > LINE_MAX_BYTES:  # keep the line whole for readers that keep only a tail of the output
        line["extra"] = {}
        text = json.dumps(line, separators=(",", ":"))
    print(text, flush=True)


if __name__ == "__main__":
    main()
