"""Host side of the routed MoE layer: the expert cache and the per-step orchestration.

Mirrors the reference engine's moe() (stbl/model.cu:426-594) for one layer:
  router (device) -> route ids to the host (the reference's to_host sync, :441) -> expert-cache
  lookups with LRU bookkeeping and refills of misses (:497-507, :383-422) -> the expert kernels
  (gate/up + SwiGLU, down, ordered combine) -> mark the slots used.
All device work is in libstbl_amd.so; this module only sequences it and keeps the host-side state.
"""

import contextlib
import ctypes

import torch

from . import _lib, ops


class ExpertCache:
    """HBM LRU cache of expert slots over a pinned host pool (stbl_amd_cache_*), or over a GGUF file
    (from_gguf)."""

    def __init__(self, slots, slot_bytes, host_pool, n_experts, n_layers=1, host_stride=None):
        if not isinstance(host_pool, torch.Tensor) or host_pool.is_cuda or not host_pool.is_pinned():
            raise ValueError("host_pool must be a pinned host tensor")
        stride = host_stride if host_stride is not None else slot_bytes
        if host_pool.numel() * host_pool.element_size() < stride * n_experts * n_layers:
            raise ValueError("host_pool is smaller than n_layers * n_experts * host_stride bytes")
        self.pool = host_pool  # keeps the pinned memory alive as long as the cache
        self.slots, self.slot_bytes, self.n_experts, self.n_layers = slots, slot_bytes, n_experts, n_layers
        self.handle = _lib.load().stbl_amd_cache_create(slots, slot_bytes, ctypes.c_void_p(host_pool.data_ptr()),
                                                        stride, n_experts, n_layers)
        if not self.handle:
            _lib.check(-1, "cache_create")

    @classmethod
    def from_gguf(cls, slots, path, first_layer=0, n_layers=1, readers=8, direct=True):
        """A cache whose misses are read from the routed-expert tensors of a GGUF file (layers
        first_layer .. first_layer + n_layers - 1) into FP4 (OCP) slots."""
        self = cls.__new__(cls)
        self.pool = None
        self.handle = _lib.load().stbl_amd_cache_create_gguf(slots, str(path).encode(), first_layer, n_layers, readers,
                                                             1 if direct else 0)
        if not self.handle:
            _lib.check(-1, "cache_create_gguf")
        info = self.file_info()
        self.slots, self.slot_bytes, self.n_experts, self.n_layers = slots, info["slot_bytes"], info["experts"], n_layers
        self.dim, self.inter = info["dim"], info["inter"]
        return self

    def file_info(self):
        out = (ctypes.c_uint64 * 8)()
        _lib.check(_lib.load().stbl_amd_cache_file_info(self.handle, out), "cache_file_info")
        keys = ("dim", "inter", "experts", "slot_bytes", "direct", "bytes_read", "read_ns", "experts_read")
        return dict(zip(keys, [int(v) for v in out]))

    def enable_prefetch(self, readers=8):
        """Background prefetch readers for a file-backed cache (stbl_amd_cache_enable_prefetch)."""
        _lib.check(_lib.load().stbl_amd_cache_enable_prefetch(self.handle, readers), "cache_enable_prefetch")

    def prefetch(self, ids, layer):
        """Queues background reads of guessed experts of `layer`, best first; returns how many."""
        n = len(ids)
        arr = (ctypes.c_int * max(n, 1))(*[int(i) for i in ids])
        r = _lib.load().stbl_amd_cache_prefetch(self.handle, arr, n, layer)
        if r < 0:
            _lib.check(r, "cache_prefetch")
        return r

    def prefetch_stats(self):
        out = (ctypes.c_uint64 * 6)()
        _lib.check(_lib.load().stbl_amd_cache_prefetch_stats(self.handle, out), "cache_prefetch_stats")
        keys = ("issued", "routed_landed", "routed_reading", "cancelled", "taken_over", "bytes_read")
        return dict(zip(keys, [int(v) for v in out]))

    def prefetch_pause(self, paused):
        _lib.check(_lib.load().stbl_amd_cache_prefetch_pause(self.handle, 1 if paused else 0), "cache_prefetch_pause")

    def lookup(self, ids, layer=0, stream=None):
        """Slots (device addresses) and hit flags of expert ids, in order; returns (ptrs, hits, misses)."""
        n = len(ids)
        arr = (ctypes.c_int * n)(*[int(i) for i in ids])
        ptrs = (ctypes.c_void_p * n)()
        hit = (ctypes.c_int * n)()
        s = ops._stream(stream)
        nmiss = _lib.load().stbl_amd_cache_lookup(self.handle, arr, n, layer, ptrs, hit, s)
        if nmiss < 0:
            _lib.check(nmiss, "cache_lookup")
        return [int(p) for p in ptrs], [bool(h) for h in hit], nmiss

    def lookup_begin(self, ids, layer=0, stream=None):
        """First half of lookup (stbl_amd_cache_lookup_begin): maps every id and queues pool refills;
        returns (ptrs, hits, ready, misses), ready[i] telling whether the slot may be read before
        lookup_end. lookup_end must follow before the next lookup or prefetch."""
        n = len(ids)
        arr = (ctypes.c_int * max(n, 1))(*[int(i) for i in ids])
        ptrs = (ctypes.c_void_p * max(n, 1))()
        hit = (ctypes.c_int * max(n, 1))()
        rdy = (ctypes.c_int * max(n, 1))()
        nmiss = _lib.load().stbl_amd_cache_lookup_begin(self.handle, arr, n, layer, ptrs, hit, rdy, ops._stream(stream))
        if nmiss < 0:
            _lib.check(nmiss, "cache_lookup_begin")
        return [int(p) for p in ptrs[:n]], [bool(h) for h in hit[:n]], [bool(r) for r in rdy[:n]], nmiss

    def lookup_end(self, stream=None):
        """Second half of lookup: file reads, routed prefetches still being read, and the compute
        stream's wait for every refill (stbl_amd_cache_lookup_end)."""
        _lib.check(_lib.load().stbl_amd_cache_lookup_end(self.handle, ops._stream(stream)), "cache_lookup_end")

    def note_guesses(self, ids, layer):
        """Records guesses for `layer` before the lookups that could evict them (lookahead counters)."""
        n = len(ids)
        arr = (ctypes.c_int * max(n, 1))(*[int(i) for i in ids])
        _lib.check(_lib.load().stbl_amd_cache_note_guesses(self.handle, arr, n, layer), "cache_note_guesses")

    def lookahead(self):
        """The reference's stbl_lookahead counters (stbl/model.cu:452-460)."""
        out = (ctypes.c_uint64 * 4)()
        _lib.check(_lib.load().stbl_amd_cache_lookahead(self.handle, out), "cache_lookahead")
        keys = ("cold_guesses", "cold_guesses_routed", "misses", "misses_guessed")
        return dict(zip(keys, [int(v) for v in out]))

    def mark_used(self, stream=None):
        _lib.check(_lib.load().stbl_amd_cache_mark_used(self.handle, ops._stream(stream)), "cache_mark_used")

    def stats(self):
        out = (ctypes.c_uint64 * 6)()
        _lib.check(_lib.load().stbl_amd_cache_stats(self.handle, out), "cache_stats")
        keys = ("hits", "misses", "refill_bytes", "lookups", "in_use", "slots")
        return dict(zip(keys, [int(v) for v in out]))

    def peek(self, expert, layer=0):
        p = _lib.load().stbl_amd_cache_peek(self.handle, layer, expert)
        return int(p) if p else None

    def fail_refill_after(self, n):
        _lib.check(_lib.load().stbl_amd_cache_fail_refill_after(self.handle, n), "cache_fail_refill_after")

    def close(self):
        if self.handle:
            _lib.load().stbl_amd_cache_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MoELayer:
    """One routed MoE layer: n_experts routed experts in a pinned host pool (or a GGUF file: pass
    cache=ExpertCache.from_gguf(...) and the cache layer) behind an HBM LRU cache, plus an always-on
    shared expert resident in HBM.

    forward(x, logits): x bf16 [t, dim] and router logits fp32 [t, n_experts] on the device; returns
    y bf16 [t, dim]. Routing follows the reference: top-k of score + bias, ties to the lower id,
    weights renormalized then scaled, with score_fn sigmoid (the configuration's) or sqrt-softplus
    (the reference engine's). shared_fmt: the shared expert's format (the reference engine pairs FP4
    routed experts with an FP8 E8M0 shared one), default the routed experts' format."""

    def __init__(self, fmt, dim, inter, host_pool, n_experts, topk, cache_slots, shared_slot=None, bias=None,
                 route_scale=1.0, limit=0.0, official=False, max_tokens=4, score_fn=ops.SCORE_SIGMOID,
                 shared_fmt=None, cache=None, layer=0):
        self.fmt, self.dim, self.inter, self.topk = fmt, dim, inter, topk
        self.score_fn = score_fn
        self.shared_fmt = fmt if shared_fmt is None else shared_fmt
        self.slot_bytes, _ = ops.expert_layout(fmt, dim, inter)
        if cache is None:
            cache = ExpertCache(cache_slots, self.slot_bytes, host_pool, n_experts)
        elif cache.slot_bytes != self.slot_bytes:
            raise ValueError("the cache's slots do not hold experts of this format and shape")
        self.cache, self.layer = cache, layer
        self.shared = shared_slot
        self.bias, self.route_scale, self.limit, self.official = bias, route_scale, limit, official
        dev = torch.device("cuda", torch.cuda.current_device())
        self.work = torch.empty(ops.moe_work_bytes(max_tokens, topk, dim, inter), dtype=torch.uint8, device=dev)
        self.max_tokens = max_tokens
        self.last_route = None  # (ids, weights) of the last step, as lists (stbl_last_route)
        self.last_lookup = None  # (distinct expert ids in lookup order, hit flags) of the last step

    def route(self, logits):
        ids, w = ops.route(logits, self.topk, self.bias, self.route_scale, score_fn=self.score_fn)
        return ids.cpu().tolist(), w.cpu().tolist()  # host sync, as the reference's to_host

    def forward(self, x, logits, route=None, stream=None, after_reads=None):
        """y = the layer's output for x. Every device call goes on `stream` (default: the current
        stream). As in the reference (stbl/model.cu:541-549, 588), the experts already in HBM and
        the shared expert are queued first, then the cache's misses are waited for (file reads
        block the host meanwhile), then the missed experts and the ordered combine run; the result
        is the same bits as one call over all experts. after_reads() runs between the two (the
        reference issues its prefetches there, stbl/model.cu:555-586)."""
        ctx = torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()
        with ctx:
            return self._forward(x, logits, route, after_reads)

    def _forward(self, x, logits, route, after_reads):
        t = x.shape[0]
        if t > self.max_tokens:
            raise ValueError(f"at most {self.max_tokens} tokens per step")
        ids, w = route if route is not None else self.route(logits)
        self.last_route = (ids, w)
        uniq = []
        for row in ids:
            for e in row:
                if e not in uniq:
                    uniq.append(e)
        ptrs, hits, ready, _ = self.cache.lookup_begin(uniq, layer=self.layer)
        self.last_lookup = (uniq, hits)
        slot_of = {e: i for i, e in enumerate(uniq)}
        slots = list(ptrs)
        shared = -1
        if self.shared is not None:
            shared = len(slots)
            slots.append(self.shared.data_ptr())
            ready = ready + [True]
        pick = [[slot_of[e] for e in row] for row in ids]
        y = torch.empty((t, self.dim), dtype=torch.bfloat16, device=x.device)
        kw = dict(shared=shared, limit=self.limit, official=self.official, work=self.work, out=y,
                  shared_fmt=self.shared_fmt)
        try:
            if all(ready):
                self.cache.lookup_end()
                if after_reads:
                    after_reads()
                return ops.moe_experts(x, slots, pick, w, self.fmt, self.dim, self.inter, **kw)
            if any(ready):
                try:
                    ops.moe_experts(x, slots, pick, w, self.fmt, self.dim, self.inter, slot_ready=ready, phase=1,
                                    **kw)
                except BaseException:
                    # end the open lookup (its reads and waits) so the cache takes the next one; the
                    # phase-1 error is the one reported
                    try:
                        self.cache.lookup_end()
                    except Exception:
                        pass
                    raise
            self.cache.lookup_end()
            if after_reads:
                after_reads()
            return ops.moe_experts(x, slots, pick, w, self.fmt, self.dim, self.inter, slot_ready=ready, phase=2, **kw)
        finally:
            self.cache.mark_used()  # after every kernel queued on the slots, whatever failed

    def close(self):
        self.cache.close()


class MoEStack:
    """Decode through routed MoE layers whose experts share one cache, with the reference engine's
    stale-router guesses (stbl/model.cu:426-475, 555-586). Before layer l's lookup, layer l+1's
    router is scored on layer l's input: its top `lookahead` experts per token are noted with the
    cache for the lookahead counters (STBL_LOOKAHEAD), and with prefetch > 0 the top `prefetch` are
    queued for background reads once layer l's own reads are done (STBL_PREFETCH); layer l+1's
    lookup then finds them landed, waits for them, reads them itself or cancels the unrouted ones.
    prefetch2 > 0 (with prefetch) also queues the top `prefetch2` of layer l+2's router on the same
    input, behind layer l+1's (STBL_PREFETCH2). As in the reference, lookahead is at least prefetch.

    routers[l]: fp32 [n_experts, dim] router weights of layer l; the logits are stbl_gemv_f32 of the
    layer's input, as in the engine (stbl/model.cu:430). Between layers the hidden state takes the
    layer's output as a residual update (h = bf16(h + y)); the layers between MoE blocks (attention,
    norms) are outside this path. step(h) returns the final hidden state, bf16 [t, dim].
    trace (when trace=True): per layer, ("guess", layer, ids) when guesses are noted and ("lookup",
    layer, distinct routed ids in lookup order), in the order they reach the cache."""

    def __init__(self, cache, fmt, dim, inter, n_experts, topk, routers, biases=None, shared_slots=None, prefetch=0,
                 score_fn=ops.SCORE_SIGMOID, route_scale=1.0, limit=0.0, official=False, shared_fmt=None,
                 max_tokens=4, prefetch2=0, lookahead=0, trace=False):
        n_layers = len(routers)
        biases = biases or [None] * n_layers
        shared_slots = shared_slots or [None] * n_layers
        self.cache, self.routers, self.biases = cache, routers, biases
        self.dim, self.n_experts, self.topk, self.prefetch = dim, n_experts, topk, prefetch
        self.prefetch2 = prefetch2 if prefetch else 0
        self.ahead = max(lookahead, prefetch)
        self.score_fn, self.route_scale = score_fn, route_scale
        self.trace = [] if trace else None
        self.layers = [MoELayer(fmt, dim, inter, None, n_experts, topk, cache.slots, shared_slot=shared_slots[l],
                                bias=biases[l], route_scale=route_scale, limit=limit, official=official,
                                max_tokens=max_tokens, score_fn=score_fn, shared_fmt=shared_fmt, cache=cache, layer=l)
                       for l in range(n_layers)]
        if prefetch:
            cache.enable_prefetch()

    def _logits(self, layer, hf):
        t = hf.shape[0]
        out = torch.empty((t, self.n_experts), dtype=torch.float32, device=hf.device)
        for i in range(t):
            ops.stbl_gemv_f32(out[i], self.routers[layer], hf[i], self.n_experts, self.dim)
        return out

    def _guess(self, layer, hf, m):
        """Per token, the top m experts of `layer`'s router on hf (best first)."""
        ids, _ = ops.route(self._logits(layer, hf), min(m, self.n_experts), self.biases[layer], self.route_scale,
                           score_fn=self.score_fn)
        return ids.cpu().tolist()

    @staticmethod
    def _union(rows, m):
        return list(dict.fromkeys(e for row in rows for e in row[:m]))

    def step(self, h, stream=None):
        n_layers = len(self.layers)
        ctx = torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()
        with ctx:
            for l, layer in enumerate(self.layers):
                hf = h.float()
                rows1 = self._guess(l + 1, hf, self.ahead) if self.ahead and l + 1 < n_layers else None
                rows2 = self._guess(l + 2, hf, self.prefetch2) if self.prefetch2 and l + 2 < n_layers else None
                if rows1 is not None:
                    guesses = self._union(rows1, self.ahead)
                    self.cache.note_guesses(guesses, l + 1)
                    if self.trace is not None:
                        self.trace.append(("guess", l + 1, guesses))

                def issue(rows1=rows1, rows2=rows2, l=l):
                    if self.prefetch and rows1 is not None:
                        self.cache.prefetch(self._union(rows1, self.prefetch), l + 1)
                    if rows2 is not None:
                        self.cache.prefetch(self._union(rows2, self.prefetch2), l + 2)
                y = layer.forward(h, self._logits(l, hf), after_reads=issue)
                if self.trace is not None:
                    self.trace.append(("lookup", l, list(layer.last_lookup[0])))
                h = (hf + y.float()).to(torch.bfloat16)
        return h

    def close(self):
        self.cache.close()
