"""CPU oracle for the quantized expert-GEMV path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and
only as the checker. The product (stblarge_amd) never imports, loads or falls back to it.

The arithmetic lives in stbl_oracle.c (a plain-C restatement of ref/kernel.py:12-102, the engine
epilogues of stbl/kernels.cu and the MoE composition of stbl/model.cu:426-594); this module wraps it
with numpy. `lru_simulate` restates the expert LRU bookkeeping of stbl/model.cu:347-422 in Python
(small inputs only). Every function here is pinned by tests/test_oracle_cpu.py against the golden
fixtures in tests/golden/ and against brute-force / closed-form / library checks.
"""

import ctypes
import os
import subprocess
from collections import OrderedDict

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(HERE, "liboracle.so")
_lib = None

P = ctypes.c_void_p
I = ctypes.c_int
F = ctypes.c_float


def build():
    """Compile liboracle.so with the committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_pow2_ceil.restype = F
        L.orc_pow2_ceil.argtypes = [F]
        L.orc_e4m3_decode.restype = F
        L.orc_e4m3_decode.argtypes = [ctypes.c_uint8]
        L.orc_e4m3_encode.restype = ctypes.c_uint8
        L.orc_e4m3_encode.argtypes = [F]
        L.orc_e2m1_decode.restype = F
        L.orc_e2m1_decode.argtypes = [ctypes.c_uint8]
        L.orc_e8m0_decode.restype = F
        L.orc_e8m0_decode.argtypes = [ctypes.c_uint8]
        L.orc_e8m0_engine.restype = ctypes.c_double
        L.orc_e8m0_engine.argtypes = [ctypes.c_uint8]
        L.orc_round_fp4.restype = F
        L.orc_round_fp4.argtypes = [F]
        L.orc_fp4_code.restype = ctypes.c_uint8
        L.orc_fp4_code.argtypes = [F]
        L.orc_f2bf.restype = ctypes.c_uint16
        L.orc_f2bf.argtypes = [F]
        L.orc_swiglu1.restype = F
        L.orc_swiglu1.argtypes = [F, F, F, F]
        L.orc_route_score.restype = F
        L.orc_route_score.argtypes = [F, I]
        for name in ("orc_act_quant", "orc_quant_fp4", "orc_quant_fp8_b128", "orc_dequant_fp8_b128",
                     "orc_dequant_fp8_e8m0_b32", "orc_dequant_fp4", "orc_dequant_gguf17", "orc_ocp_to_gguf17",
                     "orc_gemm", "orc_gemv_fp4", "orc_gemv_fp8_b128", "orc_swiglu", "orc_round_bf16",
                     "orc_route", "orc_e4m3_encode_n", "orc_expert_ffn_fp4", "orc_expert_ffn_fp8", "orc_moe_fp4",
                     "orc_quant_fp8_e8m0_b32", "orc_expert_ffn_deq", "orc_moe_deq", "orc_gemv_gguf_engine",
                     "orc_gemv_fp8_e8m0_engine"):
            getattr(L, name).restype = None
        _lib = L
    return _lib


def _p(a):
    return P(a.ctypes.data) if a is not None else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


# ---- scalar codecs (vectorised through the C scalars) --------------------------------------------

def pow2_ceil(t):
    t = _f32(t)
    return np.array([lib().orc_pow2_ceil(float(v)) for v in t.ravel()], dtype=np.float32).reshape(t.shape)


def e4m3_decode(codes):
    codes = _u8(codes)
    table = np.array([lib().orc_e4m3_decode(c) for c in range(256)], dtype=np.float32)
    return table[codes]


def e4m3_encode(x):
    x = _f32(x)
    out = np.empty(x.shape, np.uint8)
    lib().orc_e4m3_encode_n(_p(x), I(x.size), _p(out))
    return out


def e2m1_table():
    return np.array([lib().orc_e2m1_decode(c) for c in range(16)], dtype=np.float32)


def e8m0_decode(s):
    s = _u8(s)
    table = np.array([lib().orc_e8m0_decode(c) for c in range(256)], dtype=np.float32)
    return table[s]


def round_fp4(v):
    v = _f32(v)
    return np.array([lib().orc_round_fp4(float(a)) for a in v.ravel()], dtype=np.float32).reshape(v.shape)


def fp4_code(q):
    q = _f32(q)
    return np.array([lib().orc_fp4_code(float(a)) for a in q.ravel()], dtype=np.uint8).reshape(q.shape)


def f2bf_bits(x):
    """fp32 -> bf16 bit patterns (uint16), round to nearest even."""
    x = _f32(x)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        r[nan] = ((x.view(np.uint32)[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_round(x):
    """fp32 -> nearest-even bf16 value, returned as fp32."""
    return (f2bf_bits(x).astype(np.uint32) << 16).view(np.float32)


# ---- array routines ------------------------------------------------------------------------------

def act_quant(x, block=32, pow2=True):
    """ref/kernel.py:35-45 on x [rows][n]: returns (codes u8, scales f32 [rows][n/block], deq f32)."""
    x = _f32(x)
    rows, n = x.reshape(-1, x.shape[-1]).shape
    codes = np.empty((rows, n), np.uint8)
    scales = np.empty((rows, n // block), np.float32)
    deq = np.empty((rows, n), np.float32)
    lib().orc_act_quant(_p(x), I(rows), I(n), I(block), I(int(pow2)), _p(codes), _p(scales), _p(deq))
    return codes, scales, deq


def quant_fp4(w):
    """Weight [rows][k] -> (codes u8 [rows][k/2], e8m0 scales u8 [rows][k/32])."""
    w = _f32(w)
    rows, k = w.shape
    codes = np.empty((rows, k // 2), np.uint8)
    scales = np.empty((rows, k // 32), np.uint8)
    lib().orc_quant_fp4(_p(w), I(rows), I(k), _p(codes), _p(scales))
    return codes, scales


def quant_fp8_b128(w):
    """Weight [rows][k] -> (e4m3 codes u8 [rows][k], fp32 scales [ceil(rows/128)][ceil(k/128)])."""
    w = _f32(w)
    rows, k = w.shape
    codes = np.empty((rows, k), np.uint8)
    scales = np.empty(((rows + 127) // 128, (k + 127) // 128), np.float32)
    lib().orc_quant_fp8_b128(_p(w), I(rows), I(k), _p(codes), _p(scales))
    return codes, scales


def quant_fp8_e8m0_b32(w):
    """Weight [rows][k] -> (e4m3 codes u8 [rows][k], E8M0 scale bytes u8 [ceil(rows/32)][k/32]): per
    32x32 block s = pow2_ceil(max(amax, 1e-4) / 448), the reference engine's FP8 layout."""
    w = _f32(w)
    rows, k = w.shape
    codes = np.empty((rows, k), np.uint8)
    scales = np.empty(((rows + 31) // 32, k // 32), np.uint8)
    lib().orc_quant_fp8_e8m0_b32(_p(w), I(rows), I(k), _p(codes), _p(scales))
    return codes, scales


def dequant_fp8_b128(codes, scales):
    codes, scales = _u8(codes), _f32(scales)
    rows, k = codes.shape
    out = np.empty((rows, k), np.float32)
    lib().orc_dequant_fp8_b128(_p(codes), _p(scales), I(rows), I(k), _p(out))
    return out


def dequant_fp8_e8m0_b32(codes, scales):
    codes, scales = _u8(codes), _u8(scales)
    rows, k = codes.shape
    out = np.empty((rows, k), np.float32)
    lib().orc_dequant_fp8_e8m0_b32(_p(codes), _p(scales), I(rows), I(k), _p(out))
    return out


def dequant_fp4(codes, scales):
    codes, scales = _u8(codes), _u8(scales)
    rows, k = codes.shape[0], codes.shape[1] * 2
    out = np.empty((rows, k), np.float32)
    lib().orc_dequant_fp4(_p(codes), _p(scales), I(rows), I(k), _p(out))
    return out


def dequant_gguf17(w, rows, k):
    w = _u8(w)
    out = np.empty((rows, k), np.float32)
    lib().orc_dequant_gguf17(_p(w), I(rows), I(k), _p(out))
    return out


def ocp_to_gguf17(codes, scales):
    codes, scales = _u8(codes), _u8(scales)
    rows, k = codes.shape[0], codes.shape[1] * 2
    out = np.empty((rows, k // 32 * 17), np.uint8)
    lib().orc_ocp_to_gguf17(_p(codes), _p(scales), I(rows), I(k), _p(out))
    return out


def gemm(a, w):
    """C[M,N] = A[M,K] @ W[N,K]^T in double (ref/kernel.py:91)."""
    a, w = _f32(a), _f32(w)
    a2 = a.reshape(-1, a.shape[-1])
    m, k = a2.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float64)
    lib().orc_gemm(_p(a2), _p(w), I(m), I(n), I(k), _p(out))
    return out


def gemv_fp4(codes, scales, x):
    """y [m][n] (double) = x [m][k] . dequant_fp4(codes, scales)^T, without a dequantized copy."""
    codes, scales, x = _u8(codes), _u8(scales), _f32(x)
    x2 = x.reshape(-1, x.shape[-1])
    m, k = x2.shape
    n = codes.shape[0]
    y = np.empty((m, n), np.float64)
    lib().orc_gemv_fp4(_p(codes), _p(scales), _p(x2), I(m), I(n), I(k), _p(y))
    return y


def e8m0_engine(s):
    """The reference engine's scale decode (stbl/kernels.cu:32): byte 0 -> 0.0, 255 -> +Inf."""
    s = _u8(s)
    table = np.array([lib().orc_e8m0_engine(c) for c in range(256)], dtype=np.float64)
    return table[s]


def gemv_gguf_engine(blocks, x, n, k):
    """stbl_gemv_mxfp4 as the reference engine computes it (stbl/kernels.cu:134-191): GGUF 17-byte
    blocks [n][k/32][17], one fp32 token x[k]; each block's sum times the engine's scale decode.
    y[n] in double."""
    blocks, x = _u8(blocks), _f32(x).reshape(-1)
    y = np.empty(n, np.float64)
    lib().orc_gemv_gguf_engine(_p(blocks), _p(x), I(n), I(k), _p(y))
    return y


def gemv_fp8_e8m0_engine(codes, scales, x):
    """stbl_gemv_fp8 as the reference engine computes it (stbl/kernels.cu:98-132): e4m3 codes [n][k],
    E8M0 bytes per 32x32 block [(n+31)/32][k/32], one fp32 token x[k]. y[n] in double."""
    codes, scales, x = _u8(codes), _u8(scales), _f32(x).reshape(-1)
    n, k = codes.shape
    y = np.empty(n, np.float64)
    lib().orc_gemv_fp8_e8m0_engine(_p(codes), _p(scales), _p(x), I(n), I(k), _p(y))
    return y


def gemv_fp8_b128(codes, scales, x):
    codes, scales, x = _u8(codes), _f32(scales), _f32(x)
    x2 = x.reshape(-1, x.shape[-1])
    m, k = x2.shape
    n = codes.shape[0]
    y = np.empty((m, n), np.float64)
    lib().orc_gemv_fp8_b128(_p(codes), _p(scales), _p(x2), I(m), I(n), I(k), _p(y))
    return y


def swiglu(g, u, w=1.0, limit=0.0):
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    lib().orc_swiglu(_p(g), _p(u), F(w), F(limit), I(g.size), _p(out))
    return out


SCORE_SIGMOID, SCORE_SQRT_SOFTPLUS = 0, 1


def route_score(l, score_fn=SCORE_SIGMOID):
    """One router score: sigmoid (0) or sqrt(softplus) with threshold 20 (1, stbl/kernels.cu:436-442)."""
    return lib().orc_route_score(F(l), I(score_fn))


def route(logits, topk=8, bias=None, route_scale=1.0, score_fn=SCORE_SIGMOID):
    """Router scores (sigmoid, or sqrt(softplus) as the reference engine), top-k by score + bias
    (ties to the lower id), renormalised weights. Returns (scores, ids, weights)."""
    logits = _f32(logits)
    t, e = logits.shape
    scores = np.empty((t, e), np.float32)
    ids = np.empty((t, topk), np.int32)
    weights = np.empty((t, topk), np.float32)
    b = _f32(bias) if bias is not None else None
    lib().orc_route(_p(logits), _p(b), I(t), I(e), I(topk), F(route_scale), I(score_fn), _p(scores), _p(ids),
                    _p(weights))
    return scores, ids, weights


def expert_ffn_fp4(slot, dim, inter, x, w=1.0, limit=0.0, official=False, raw=False):
    """One FP4 expert on one token (stbl/model.cu:516-547). slot = the six parts packed back to back.
    Returns o = bf16(down product); with raw=True also the down product before rounding (double)."""
    slot, x = _u8(slot), _f32(x)
    o = np.empty(dim, np.float32)
    r = np.empty(dim, np.float64) if raw else None
    lib().orc_expert_ffn_fp4(_p(slot), I(dim), I(inter), _p(x), F(w), F(limit), I(int(official)), _p(o), _p(r))
    return (o, r) if raw else o


def expert_ffn_fp8(g, u, d, dim, inter, x, w=1.0, limit=0.0, official=False, raw=False):
    """g, u, d = (codes, fp32 scales) of gate [inter][dim], up [inter][dim], down [dim][inter]."""
    (gc, gs), (uc, us), (dc, ds) = [(_u8(c), _f32(s)) for c, s in (g, u, d)]
    x = _f32(x)
    o = np.empty(dim, np.float32)
    r = np.empty(dim, np.float64) if raw else None
    lib().orc_expert_ffn_fp8(_p(gc), _p(gs), _p(uc), _p(us), _p(dc), _p(ds), I(dim), I(inter), _p(x), F(w), F(limit),
                             I(int(official)), _p(o), _p(r))
    return (o, r) if raw else o


def moe_fp4(slots, weights, shared, dim, inter, x, limit=0.0, official=False):
    """slots: list (per token) of lists (top-k order) of uint8 slot arrays; weights [t][topk]."""
    x = _f32(x).reshape(-1, dim)
    t = x.shape[0]
    topk = len(slots[0])
    keep = [_u8(s) for row in slots for s in row]
    arr = (ctypes.c_void_p * len(keep))(*[k.ctypes.data for k in keep])
    w = _f32(weights)
    sh = _u8(shared) if shared is not None else None
    y = np.empty((t, dim), np.float32)
    lib().orc_moe_fp4(arr, _p(w), _p(sh), I(t), I(topk), I(dim), I(inter), _p(x), F(limit), I(int(official)), _p(y))
    return y


def expert_ffn_deq(gw, uw, dw, x, w=1.0, limit=0.0, official=False, raw=False):
    """One expert from dequantized fp32 matrices gate/up [inter][dim], down [dim][inter] (any weight
    format dequantizes exactly); the composition of expert_ffn_fp4."""
    gw, uw, dw, x = _f32(gw), _f32(uw), _f32(dw), _f32(x)
    inter, dim = gw.shape
    o = np.empty(dim, np.float32)
    r = np.empty(dim, np.float64) if raw else None
    lib().orc_expert_ffn_deq(_p(gw), _p(uw), _p(dw), I(dim), I(inter), _p(x), F(w), F(limit), I(int(official)),
                             _p(o), _p(r))
    return (o, r) if raw else o


def moe_deq(experts, weights, shared, x, limit=0.0, official=False):
    """experts: per token, a list (top-k order) of (gate, up, down) dequantized fp32 matrices;
    shared: (gate, up, down) or None; weights [t][topk]. The composition of moe_fp4."""
    x = _f32(x)
    dim = x.shape[-1]
    x = x.reshape(-1, dim)
    t, topk = x.shape[0], len(experts[0])
    keep = [_f32(m) for row in experts for e in row for m in e]
    inter = keep[0].shape[0]
    arr = (ctypes.c_void_p * len(keep))(*[k.ctypes.data for k in keep])
    sh_keep = [_f32(m) for m in shared] if shared is not None else None
    sh = (ctypes.c_void_p * 3)(*[k.ctypes.data for k in sh_keep]) if sh_keep else None
    w = _f32(weights)
    y = np.empty((t, dim), np.float32)
    lib().orc_moe_deq(arr, _p(w), sh, I(t), I(topk), I(dim), I(inter), _p(x), F(limit), I(int(official)), _p(y))
    return y


# ---- ref/kernel.py's own CPU method (torch), the CPU baseline of the measurements -------------------

_FP4_LUT = None


def fp4_gemm_torch(x, codes, scales):
    """fp4_gemm of ref/kernel.py:94-102 as the reference runs it on the CPU: every call dequantizes
    the whole weight into one fp32 matrix (each code's e2m1 value, low nibble first, times
    2^(scale - 127) per 32 along K) and multiplies x [m][k] (bf16 values) by its transpose in fp32
    with torch's CPU matmul on torch's thread pool; the result is rounded to bf16. codes uint8
    [n][k/2], scales uint8 [n][k/32] (torch tensors). Used as the timed CPU baseline; its bits
    depend on torch's summation order, so parity checks use the C restatement instead."""
    import torch

    global _FP4_LUT
    if _FP4_LUT is None:
        mags = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
        _FP4_LUT = torch.tensor(mags + [-v for v in mags], dtype=torch.float32)
    n, k = codes.shape[0], codes.shape[1] * 2
    w = torch.empty((n, k // 2, 2), dtype=torch.float32)
    w[..., 0] = _FP4_LUT[(codes & 15).long()]
    w[..., 1] = _FP4_LUT[(codes >> 4).long()]
    scale = torch.ldexp(torch.ones(1), scales.to(torch.int32) - 127)
    w = (w.view(n, k // 32, 32) * scale.view(n, k // 32, 1)).view(n, k)
    return (x.float().view(-1, k) @ w.t()).to(torch.bfloat16)


# ---- expert LRU bookkeeping (stbl/model.cu:347-422, 497-507) ---------------------------------------

def lru_simulate(steps, slots):
    """Replays the engine's expert-cache bookkeeping over `steps` (each a list of expert ids in the
    order they are looked up). Per step: cached experts of the step are first moved to the
    most-recently-used end (so a miss cannot evict them); then each id in order is looked up: a hit
    moves it to MRU; a miss takes a never-used slot (lowest first) or else evicts the least recently
    used entry, and inserts at MRU. Returns per step (hit flags, slot per id, evicted ids)."""
    lru = OrderedDict()  # id -> slot; last item = most recently used
    next_slot = 0
    out = []
    for ids in steps:
        for e in ids:
            if e in lru:
                lru.move_to_end(e)
        hits, where, evicted = [], [], []
        for e in ids:
            if e in lru:
                lru.move_to_end(e)
                hits.append(True)
            else:
                if next_slot < slots:
                    s = next_slot
                    next_slot += 1
                else:
                    victim, s = next(iter(lru.items()))
                    del lru[victim]
                    evicted.append(victim)
                lru[e] = s
                hits.append(False)
            where.append(lru[e])
        out.append((hits, where, evicted))
    return out
