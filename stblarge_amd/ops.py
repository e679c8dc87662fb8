"""Torch-facing wrappers over the C ABI: device tensors in, device tensors out.

PyTorch only allocates memory and supplies the current stream; every computation runs in
libstbl_amd.so. Shapes and dtypes are checked here so that a wrong call raises instead of launching a
kernel on a buffer of the wrong size.

Names follow the reference:
  * act_quant / gemv_fp8 / gemv_fp4 restate ref/kernel.py's act_quant, fp8_gemm and fp4_gemm for
    activation rows M <= 4 (the decode case), with bf16 activations;
  * stbl_* functions keep the reference engine's operator surface (stbl/kernels.h): fp32 activation
    buffers, results written into caller-provided tensors.
"""

import ctypes
import math

import torch

from . import _lib

P = ctypes.c_void_p


def _ptr(t):
    return P(t.data_ptr()) if t is not None else None


def _stream(stream=None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return P(s.cuda_stream)


def _need(t, dtype, name, dims=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dims is not None and t.dim() != dims:
        raise ValueError(f"{name} must have {dims} dims, got shape {tuple(t.shape)}")


def _rows2(x):
    return x if x.dim() == 2 else x.view(1, -1)


FP4, FP8, FP8_E8M0 = 0, 1, 2  # expert formats: OCP FP4; FP8 + fp32 128x128 scales; FP8 + E8M0 32x32


# ---- quantizers / dequantizers --------------------------------------------------------------------

def quant_fp4(w):
    """fp32 [N, K] -> (codes uint8 [N, K/2], E8M0 scales uint8 [N, K/32])."""
    _need(w, torch.float32, "w", 2)
    n, k = w.shape
    codes = torch.empty((n, k // 2), dtype=torch.uint8, device=w.device)
    scales = torch.empty((n, k // 32), dtype=torch.uint8, device=w.device)
    _lib.check(_lib.load().stbl_amd_quant_fp4(_ptr(codes), _ptr(scales), _ptr(w), n, k, _stream()), "quant_fp4")
    return codes, scales


def quant_fp8_b128(w):
    """fp32 [N, K] -> (e4m3 codes uint8 [N, K], fp32 scales [ceil(N/128), ceil(K/128)])."""
    _need(w, torch.float32, "w", 2)
    n, k = w.shape
    codes = torch.empty((n, k), dtype=torch.uint8, device=w.device)
    scales = torch.empty(((n + 127) // 128, (k + 127) // 128), dtype=torch.float32, device=w.device)
    _lib.check(_lib.load().stbl_amd_quant_fp8_b128(_ptr(codes), _ptr(scales), _ptr(w), n, k, _stream()),
               "quant_fp8_b128")
    return codes, scales


def quant_fp8_e8m0(w):
    """fp32 [N, K] -> (e4m3 codes uint8 [N, K], E8M0 scale bytes uint8 [ceil(N/32), K/32]), the
    reference engine's FP8 layout (per 32x32 block, power-of-two scales)."""
    _need(w, torch.float32, "w", 2)
    n, k = w.shape
    codes = torch.empty((n, k), dtype=torch.uint8, device=w.device)
    scales = torch.empty(((n + 31) // 32, k // 32), dtype=torch.uint8, device=w.device)
    _lib.check(_lib.load().stbl_amd_quant_fp8_e8m0(_ptr(codes), _ptr(scales), _ptr(w), n, k, _stream()),
               "quant_fp8_e8m0")
    return codes, scales


def dequant_fp4(codes, scales):
    _need(codes, torch.uint8, "codes", 2)
    _need(scales, torch.uint8, "scales", 2)
    n, k = codes.shape[0], codes.shape[1] * 2
    if scales.shape != (n, k // 32):
        raise ValueError(f"scales must be {(n, k // 32)}, got {tuple(scales.shape)}")
    out = torch.empty((n, k), dtype=torch.float32, device=codes.device)
    _lib.check(_lib.load().stbl_amd_dequant_fp4(_ptr(out), _ptr(codes), _ptr(scales), n, k, _stream()), "dequant_fp4")
    return out


def dequant_gguf17(w, rows, k):
    _need(w, torch.uint8, "w")
    if w.numel() != rows * (k // 32) * 17:
        raise ValueError("w must hold rows * k/32 17-byte blocks")
    out = torch.empty((rows, k), dtype=torch.float32, device=w.device)
    _lib.check(_lib.load().stbl_amd_dequant_gguf17(_ptr(out), _ptr(w), rows, k, _stream()), "dequant_gguf17")
    return out


def dequant_fp8(codes, scales, e8m0=False):
    _need(codes, torch.uint8, "codes", 2)
    n, k = codes.shape
    if e8m0:
        _need(scales, torch.uint8, "scales", 2)
        want = ((n + 31) // 32, k // 32)
    else:
        _need(scales, torch.float32, "scales", 2)
        want = ((n + 127) // 128, (k + 127) // 128)
    if tuple(scales.shape) != want:
        raise ValueError(f"scales must be {want}, got {tuple(scales.shape)}")
    out = torch.empty((n, k), dtype=torch.float32, device=codes.device)
    _lib.check(_lib.load().stbl_amd_dequant_fp8(_ptr(out), _ptr(codes), _ptr(scales), n, k, int(e8m0), _stream()),
               "dequant_fp8")
    return out


def act_quant(x, block_size=128, pow2=True, want_deq=False):
    """ref/kernel.py:35-45 on bf16 x [..., n]: (codes uint8 [..., n], fp32 scales [..., n/block]);
    with want_deq also the in-place form bf16(e4m3 * s)."""
    _need(x, torch.bfloat16, "x")
    n = x.shape[-1]
    rows = x.numel() // n
    codes = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    scales = torch.empty((*x.shape[:-1], n // block_size), dtype=torch.float32, device=x.device)
    deq = torch.empty_like(x) if want_deq else None
    _lib.check(_lib.load().stbl_amd_act_quant(_ptr(x), rows, n, block_size, int(pow2), _ptr(codes), _ptr(scales),
                                              _ptr(deq), _stream()), "act_quant")
    return (codes, scales, deq) if want_deq else (codes, scales)


# ---- GEMV ---------------------------------------------------------------------------------------------

def gemv_fp4(codes, scales, x, out_f32=False, out=None):
    """y [M, N] = x [M, K] . (e2m1(codes) * 2^(scales-127))^T, M <= 4; bf16 (or fp32) output."""
    _need(codes, torch.uint8, "codes", 2)
    _need(scales, torch.uint8, "scales", 2)
    _need(x, torch.bfloat16, "x")
    x2 = _rows2(x)
    n, k = codes.shape[0], codes.shape[1] * 2
    m = x2.shape[0]
    if x2.shape[1] != k or tuple(scales.shape) != (n, k // 32):
        raise ValueError(f"shape mismatch: codes {tuple(codes.shape)}, scales {tuple(scales.shape)}, x {tuple(x.shape)}")
    y = out if out is not None else torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16,
                                                device=codes.device)
    _lib.check(_lib.load().stbl_amd_gemv_fp4(_ptr(y), _ptr(codes), _ptr(scales), _ptr(x2), m, n, k, int(out_f32),
                                             _stream()), "gemv_fp4")
    return y


def gemv_fp8(codes, scales, x, out_f32=False, out=None):
    """y [M, N] = x [M, K] . (e4m3(codes) * scales[r/128][k/128])^T, M <= 4; bf16 (or fp32) output."""
    _need(codes, torch.uint8, "codes", 2)
    _need(scales, torch.float32, "scales", 2)
    _need(x, torch.bfloat16, "x")
    x2 = _rows2(x)
    n, k = codes.shape
    m = x2.shape[0]
    if x2.shape[1] != k or tuple(scales.shape) != ((n + 127) // 128, (k + 127) // 128):
        raise ValueError(f"shape mismatch: codes {tuple(codes.shape)}, scales {tuple(scales.shape)}, x {tuple(x.shape)}")
    y = out if out is not None else torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16,
                                                device=codes.device)
    _lib.check(_lib.load().stbl_amd_gemv_fp8(_ptr(y), _ptr(codes), _ptr(scales), _ptr(x2), m, n, k, int(out_f32),
                                             _stream()), "gemv_fp8")
    return y


def gemv_batch(codes, scales, xs, fmt, out_f32=False, outs=None):
    """len(codes) <= 64 same-shape GEMVs in one launch: ys[j] = gemv(codes[j], scales[j], xs[j])."""
    n = len(codes)
    if not (len(scales) == n == len(xs)) or n == 0 or n > 64:
        raise ValueError("gemv_batch: need 1..64 matching codes/scales/x")
    rows = codes[0].shape[0]
    k = codes[0].shape[1] * (2 if fmt == FP4 else 1)
    sdt = torch.uint8 if fmt == FP4 else torch.float32
    m = _rows2(xs[0]).shape[0]
    for c, s_, x in zip(codes, scales, xs):
        _need(c, torch.uint8, "codes", 2)
        _need(s_, sdt, "scales", 2)
        _need(x, torch.bfloat16, "x")
        if tuple(c.shape) != tuple(codes[0].shape) or tuple(_rows2(x).shape) != (m, k):
            raise ValueError("gemv_batch: all matrices and activations must have one shape")
    ys = outs if outs is not None else [torch.empty((m, rows), dtype=torch.float32 if out_f32 else torch.bfloat16,
                                                    device=codes[0].device) for _ in range(n)]
    arr = ctypes.c_void_p * n
    fn = _lib.load().stbl_amd_gemv_fp4_batch if fmt == FP4 else _lib.load().stbl_amd_gemv_fp8_batch
    _lib.check(fn(arr(*[y.data_ptr() for y in ys]), arr(*[c.data_ptr() for c in codes]),
                  arr(*[s_.data_ptr() for s_ in scales]), arr(*[x.data_ptr() for x in xs]), n, m, rows, k,
                  int(out_f32), _stream()), "gemv_batch")
    return ys


# ---- the reference engine's operator surface (stbl/kernels.h), fp32 activation buffers ---------------

def stbl_act_quant_fp8(x):
    _need(x, torch.float32, "x")
    _lib.load().stbl_act_quant_fp8(_ptr(x), x.numel(), _stream())
    _lib.check(None, "stbl_act_quant_fp8")
    return x


def stbl_round_bf16(x):
    _need(x, torch.float32, "x")
    _lib.load().stbl_round_bf16(_ptr(x), x.numel(), _stream())
    _lib.check(None, "stbl_round_bf16")
    return x


def stbl_gemv_fp8(y, w, scale, x, rows, k, round_out):
    _need(y, torch.float32, "y")
    _need(w, torch.uint8, "w")
    _need(scale, torch.uint8, "scale")
    _need(x, torch.float32, "x")
    if y.numel() < rows or w.numel() != rows * k or x.numel() < k or scale.numel() != ((rows + 31) // 32) * (k // 32):
        raise ValueError("stbl_gemv_fp8: buffer sizes do not match rows/k")
    _lib.load().stbl_gemv_fp8(_ptr(y), _ptr(w), _ptr(scale), _ptr(x), rows, k, int(round_out), _stream())
    _lib.check(None, "stbl_gemv_fp8")
    return y


def stbl_gemv_mxfp4(y, w, x, rows, k):
    return stbl_gemv_mxfp4_batch([y], [w], [x], rows, k)


def stbl_gemv_mxfp4_batch(ys, ws, xs, rows, k):
    n = len(ys)
    if not (len(ws) == n == len(xs)) or n == 0 or n > 16:
        raise ValueError("stbl_gemv_mxfp4_batch: need 1..16 matching y/w/x tensors")
    for y, w, x in zip(ys, ws, xs):
        _need(y, torch.float32, "y")
        _need(w, torch.uint8, "w")
        _need(x, torch.float32, "x")
        if y.numel() < rows or w.numel() != rows * (k // 32) * 17 or x.numel() < k:
            raise ValueError("stbl_gemv_mxfp4_batch: buffer sizes do not match rows/k")
    arr = ctypes.c_void_p * n
    _lib.load().stbl_gemv_mxfp4_batch(arr(*[y.data_ptr() for y in ys]), arr(*[w.data_ptr() for w in ws]),
                                      arr(*[x.data_ptr() for x in xs]), n, rows, k, _stream())
    _lib.check(None, "stbl_gemv_mxfp4_batch")
    return ys


def stbl_gemv_f32(y, w, x, rows, k, round_out=0):
    """fp32 GEMV of the reference ABI (the router's logits): y [rows] = w [rows, k] . x [k]."""
    _need(y, torch.float32, "y")
    _need(w, torch.float32, "w")
    _need(x, torch.float32, "x")
    if y.numel() < rows or w.numel() < rows * k or x.numel() < k:
        raise ValueError("stbl_gemv_f32: buffer sizes do not match rows/k")
    _lib.load().stbl_gemv_f32(_ptr(y), _ptr(w), _ptr(x), rows, k, int(round_out), _stream())
    _lib.check(None, "stbl_gemv_f32")
    return y


def stbl_sqrt_softplus(s, n=None):
    """The reference ABI's router scores in place: s = sqrt(softplus(s)) (fp32, device)."""
    _need(s, torch.float32, "s")
    n = s.numel() if n is None else n
    if n > s.numel():
        raise ValueError("stbl_sqrt_softplus: n exceeds the buffer")
    _lib.load().stbl_sqrt_softplus(_ptr(s), n, _stream())
    _lib.check(None, "stbl_sqrt_softplus")
    return s


def stbl_gemv_bf16(y, w, x, rows, k, round_out=0, group_rows=0):
    """bf16-weight GEMV of the reference ABI: y [rows] = w [rows, k] . x_r with x_r the (r /
    group_rows)-th k-long row of x when group_rows > 0."""
    _need(y, torch.float32, "y")
    _need(w, torch.bfloat16, "w")
    _need(x, torch.float32, "x")
    xrows = (rows + group_rows - 1) // group_rows if group_rows > 0 else 1
    if y.numel() < rows or w.numel() < rows * k or x.numel() < xrows * k:
        raise ValueError("stbl_gemv_bf16: buffer sizes do not match rows/k/group_rows")
    _lib.load().stbl_gemv_bf16(_ptr(y), _ptr(w), _ptr(x), rows, k, int(round_out), int(group_rows), _stream())
    _lib.check(None, "stbl_gemv_bf16")
    return y


def stbl_swiglu(out, g, u, weight, limit, n):
    return stbl_swiglu_batch(out, g, u, [weight], limit, n)


def stbl_swiglu_batch(out, g, u, weights, limit, n):
    count = len(weights)
    for t, nm in ((out, "out"), (g, "g"), (u, "u")):
        _need(t, torch.float32, nm)
        if t.numel() < count * n:
            raise ValueError(f"{nm} holds fewer than count * n values")
    w = (ctypes.c_float * count)(*weights)
    _lib.load().stbl_swiglu_batch(_ptr(out), _ptr(g), _ptr(u), w, count, float(limit), n, _stream())
    _lib.check(None, "stbl_swiglu_batch")
    return out


def stbl_axpy(y, x, a, n):
    _need(y, torch.float32, "y")
    _need(x, torch.float32, "x")
    if y.numel() < n or x.numel() < n:
        raise ValueError("stbl_axpy: buffers shorter than n")
    _lib.load().stbl_axpy(_ptr(y), _ptr(x), float(a), n, _stream())
    _lib.check(None, "stbl_axpy")
    return y


# ---- expert FFN / MoE / router (v2) ------------------------------------------------------------------


def expert_layout(fmt, dim, inter):
    """(slot bytes, [offsets of gate codes, gate scales, up codes, up scales, down codes, down scales])."""
    offs = (ctypes.c_uint64 * 6)()
    n = _lib.load().stbl_amd_expert_layout(fmt, dim, inter, offs)
    return int(n), [int(o) for o in offs]


def _mat_bytes(fmt, rows, k):
    """Codes + scales bytes of one quantized [rows x k] matrix."""
    if fmt == FP4:
        return rows * k // 2 + rows * k // 32
    if fmt == FP8_E8M0:
        return rows * k + ((rows + 31) // 32) * (k // 32)
    return rows * k + 4 * ((rows + 127) // 128) * ((k + 127) // 128)


def _mat_shapes(fmt, dim, inter):
    out = []
    for rows, k in ((inter, dim), (inter, dim), (dim, inter)):
        if fmt == FP4:
            out += [((rows, k // 2), torch.uint8), ((rows, k // 32), torch.uint8)]
        elif fmt == FP8_E8M0:
            out += [((rows, k), torch.uint8), (((rows + 31) // 32, k // 32), torch.uint8)]
        else:
            out += [((rows, k), torch.uint8), (((rows + 127) // 128, (k + 127) // 128), torch.float32)]
    return out


def slot_views(slot, fmt, dim, inter):
    """Views of the six parts (codes/scales of gate, up, down) of a uint8 slot tensor."""
    nbytes, offs = expert_layout(fmt, dim, inter)
    if slot.dtype != torch.uint8 or slot.numel() < nbytes:
        raise ValueError(f"slot must be >= {nbytes} uint8 bytes")
    views = []
    for off, (shape, dt) in zip(offs, _mat_shapes(fmt, dim, inter)):
        n = math.prod(shape) * (4 if dt == torch.float32 else 1)
        views.append(slot[off:off + n].view(dt).view(shape))
    return views


def pack_slot(parts, fmt, dim, inter, out=None):
    """Writes [gate codes, gate scales, up codes, up scales, down codes, down scales] into a slot."""
    nbytes, _ = expert_layout(fmt, dim, inter)
    dev = parts[0].device
    slot = out if out is not None else torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    for v, p in zip(slot_views(slot, fmt, dim, inter), parts):
        v.copy_(p)
    return slot


def quant_expert(w_gate, w_up, w_down, fmt, out=None):
    """Quantize fp32 gate/up [inter, dim] and down [dim, inter] on the device into one slot."""
    q = {FP4: quant_fp4, FP8: quant_fp8_b128, FP8_E8M0: quant_fp8_e8m0}[fmt]
    parts = []
    for w in (w_gate, w_up, w_down):
        parts += list(q(w))
    inter, dim = w_gate.shape
    return pack_slot(parts, fmt, dim, inter, out)


def expert_ffn(slot, x, fmt, dim, inter, weight=1.0, limit=0.0, official=False, out_f32=False):
    """y [m, dim] = down(swiglu(gate x, up x)) for one expert slot, m <= 4 tokens."""
    _need(slot, torch.uint8, "slot")
    _need(x, torch.bfloat16, "x")
    x2 = _rows2(x)
    m = x2.shape[0]
    if x2.shape[1] != dim:
        raise ValueError("x must be [m, dim]")
    if slot.numel() < expert_layout(fmt, dim, inter)[0]:
        raise ValueError("slot too small")
    y = torch.empty((m, dim), dtype=torch.float32 if out_f32 else torch.bfloat16, device=x.device)
    work = torch.empty(m * inter, dtype=torch.bfloat16, device=x.device)
    _lib.check(_lib.load().stbl_amd_expert_ffn(fmt, _ptr(y), _ptr(slot), _ptr(x2), m, dim, inter, float(weight),
                                               float(limit), int(official), int(out_f32), _ptr(work), _stream()),
               "expert_ffn")
    return y


def moe_work_bytes(t, topk, dim, inter):
    return int(_lib.load().stbl_amd_moe_work_bytes(t, topk, dim, inter))


def moe_experts(x, slots, pick, weights, fmt, dim, inter, shared=-1, limit=0.0, official=False, out_f32=False,
                work=None, out=None, shared_fmt=-1, stream=None, slot_ready=None, phase=0):
    """Expert part of a routed MoE layer. slots: list of device uint8 slot tensors (or raw device
    addresses); pick: [t][topk] indices into slots; weights: [t][topk] floats; shared: slot index of
    the always-on expert or -1; shared_fmt: its format when it differs from the routed experts'.
    phase 1 / 2 with slot_ready (one flag per slot): the experts of ready slots, then the others and
    the combine (stbl_amd_moe_experts_phase); both calls need the same out and work."""
    _need(x, torch.bfloat16, "x")
    x2 = _rows2(x)
    t = x2.shape[0]
    topk = len(pick[0])
    addrs = [s if isinstance(s, int) else s.data_ptr() for s in slots]
    arr = (ctypes.c_void_p * len(addrs))(*addrs)
    pk = (ctypes.c_int * (t * topk))(*[int(v) for row in pick for v in row])
    wt = (ctypes.c_float * (t * topk))(*[float(v) for row in weights for v in row])
    nbytes = moe_work_bytes(t, topk, dim, inter)
    if work is None or work.numel() < nbytes:
        work = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    y = out if out is not None else torch.empty((t, dim), dtype=torch.float32 if out_f32 else torch.bfloat16,
                                                device=x.device)
    if phase == 0:
        _lib.check(_lib.load().stbl_amd_moe_experts(fmt, _ptr(y), _ptr(x2), t, dim, inter, arr, len(addrs), pk, wt,
                                                    topk, shared, int(shared_fmt), float(limit), int(official),
                                                    int(out_f32), _ptr(work), _stream(stream)), "moe_experts")
        return y
    if slot_ready is None or len(slot_ready) != len(addrs):
        raise ValueError("moe_experts: phases 1 and 2 need one slot_ready flag per slot")
    rd = (ctypes.c_int * len(addrs))(*[1 if r else 0 for r in slot_ready])
    _lib.check(_lib.load().stbl_amd_moe_experts_phase(fmt, _ptr(y), _ptr(x2), t, dim, inter, arr, len(addrs), pk, wt,
                                                      topk, shared, int(shared_fmt), float(limit), int(official),
                                                      int(out_f32), rd, int(phase), _ptr(work), _stream(stream)),
               f"moe_experts phase {phase}")
    return y


SCORE_SIGMOID, SCORE_SQRT_SOFTPLUS = 0, 1


def route(logits, topk, bias=None, route_scale=1.0, want_scores=False, score_fn=SCORE_SIGMOID, stream=None):
    """Device router: (ids int32 [t, topk], weights fp32 [t, topk][, scores fp32 [t, E]]). score_fn:
    SCORE_SIGMOID (the configuration's) or SCORE_SQRT_SOFTPLUS (the reference engine's)."""
    _need(logits, torch.float32, "logits", 2)
    t, e = logits.shape
    ids = torch.empty((t, topk), dtype=torch.int32, device=logits.device)
    w = torch.empty((t, topk), dtype=torch.float32, device=logits.device)
    sc = torch.empty((t, e), dtype=torch.float32, device=logits.device) if want_scores else None
    if bias is not None:
        _need(bias, torch.float32, "bias", 1)
    _lib.check(_lib.load().stbl_amd_route(_ptr(logits), _ptr(bias), t, e, topk, float(route_scale), int(score_fn),
                                          _ptr(ids), _ptr(w), _ptr(sc), _stream(stream)), "route")
    return (ids, w, sc) if want_scores else (ids, w)


# ---- multi-token GEMM (scaled MFMA) ------------------------------------------------------------------

def _gemm_shapes(codes, scales, fmt, k):
    _need(codes, torch.uint8, "codes", 2)
    _need(scales, torch.uint8 if fmt == FP4 else torch.float32, "scales", 2)
    n = codes.shape[0]
    if fmt == FP4:
        ok = codes.shape[1] * 2 == k and tuple(scales.shape) == (n, k // 32)
    else:
        ok = codes.shape[1] == k and tuple(scales.shape) == ((n + 127) // 128, (k + 127) // 128)
    if not ok:
        raise ValueError(f"shape mismatch: codes {tuple(codes.shape)}, scales {tuple(scales.shape)}, k {k}")
    return n


def gemm_work(m, n, k, device):
    """Scratch for gemm / gemm_q (split-K partial tiles and the quantized activations)."""
    return torch.empty(int(_lib.load().stbl_amd_gemm_work_bytes(m, n, k)), dtype=torch.uint8, device=device)


def _work_for(work, m, n, k, device):
    if work is None or work.numel() < int(_lib.load().stbl_amd_gemm_work_bytes(m, n, k)):
        return gemm_work(m, n, k, device)
    return work


GEMM_MAX_M = 64  # rows per stbl_amd_gemm / stbl_amd_gemm_q launch


def gemm(codes, scales, x, fmt, act_block=128, out_f32=False, work=None):
    """Y [M, N] = act_quant(X, act_block) . Wdeq^T (fp4_gemm / fp8_gemm of ref/kernel.py), any M: one
    launch per 64 rows (each output row depends only on its own activation row). `work` (from
    gemm_work) may be passed to reuse the scratch across calls on one stream."""
    _need(x, torch.bfloat16, "x", 2)
    m, k = x.shape
    if m < 1:
        raise ValueError("gemm: x has no rows")
    n = _gemm_shapes(codes, scales, fmt, k)
    work = _work_for(work, min(m, GEMM_MAX_M), n, k, x.device)
    y = torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=x.device)
    for r0 in range(0, m, GEMM_MAX_M):
        mc = min(GEMM_MAX_M, m - r0)
        _lib.check(_lib.load().stbl_amd_gemm(fmt, _ptr(y[r0:r0 + mc]), _ptr(codes), _ptr(scales), _ptr(x[r0:r0 + mc]),
                                             mc, n, k, act_block, int(out_f32), _ptr(work), _stream()), "gemm")
    return y


def gemm_q(codes, scales, aq, a_s, fmt, act_block=128, out_f32=False, work=None):
    """Y [M, N] = (Aq * a_s) . Wdeq^T with the activations already quantized: aq e4m3 codes uint8 [M, K],
    a_s E8M0 scale bytes uint8 [M, K / act_block] (act_quant_e4m3's output), as ref/kernel.py's
    fp8_gemm(a, a_s, b, b_s) takes them; any M, one launch per 64 rows."""
    _need(aq, torch.uint8, "aq", 2)
    _need(a_s, torch.uint8, "a_s", 2)
    m, k = aq.shape
    if m < 1:
        raise ValueError("gemm_q: aq has no rows")
    if tuple(a_s.shape) != (m, k // act_block):
        raise ValueError(f"a_s {tuple(a_s.shape)} does not match aq {tuple(aq.shape)} at block {act_block}")
    n = _gemm_shapes(codes, scales, fmt, k)
    work = _work_for(work, min(m, GEMM_MAX_M), n, k, aq.device)
    y = torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=aq.device)
    for r0 in range(0, m, GEMM_MAX_M):
        mc = min(GEMM_MAX_M, m - r0)
        _lib.check(_lib.load().stbl_amd_gemm_q(fmt, _ptr(y[r0:r0 + mc]), _ptr(codes), _ptr(scales), _ptr(aq[r0:r0 + mc]),
                                               _ptr(a_s[r0:r0 + mc]), mc, n, k, act_block, int(out_f32), _ptr(work),
                                               _stream()), "gemm_q")
    return y


def gemm_pack(codes, fmt):
    """The weight codes in MFMA operand order (stbl_amd_gemm_pack), for gemm_packed / gemm_q_packed:
    a uint8 tensor of the codes' size; rows (n) a multiple of 16, K a multiple of 128."""
    _need(codes, torch.uint8, "codes", 2)
    n = codes.shape[0]
    k = codes.shape[1] * (2 if fmt == FP4 else 1)
    packed = torch.empty_like(codes)
    _lib.check(_lib.load().stbl_amd_gemm_pack(fmt, _ptr(packed), _ptr(codes), n, k, _stream()), "gemm_pack")
    return packed


def gemm_packed(packed, scales, x, fmt, act_block=128, out_f32=False, work=None):
    """gemm() with the weight codes from gemm_pack; the same result bit for bit."""
    _need(x, torch.bfloat16, "x", 2)
    m, k = x.shape
    if m < 1:
        raise ValueError("gemm_packed: x has no rows")
    n = _gemm_shapes(packed, scales, fmt, k)
    work = _work_for(work, min(m, GEMM_MAX_M), n, k, x.device)
    y = torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=x.device)
    for r0 in range(0, m, GEMM_MAX_M):
        mc = min(GEMM_MAX_M, m - r0)
        _lib.check(_lib.load().stbl_amd_gemm_packed(fmt, _ptr(y[r0:r0 + mc]), _ptr(packed), _ptr(scales),
                                                    _ptr(x[r0:r0 + mc]), mc, n, k, act_block, int(out_f32), _ptr(work),
                                                    _stream()), "gemm_packed")
    return y


def gemm_q_packed(packed, scales, aq, a_s, fmt, act_block=128, out_f32=False, work=None):
    """gemm_q() with the weight codes from gemm_pack; the same result bit for bit."""
    _need(aq, torch.uint8, "aq", 2)
    _need(a_s, torch.uint8, "a_s", 2)
    m, k = aq.shape
    if m < 1:
        raise ValueError("gemm_q_packed: aq has no rows")
    if tuple(a_s.shape) != (m, k // act_block):
        raise ValueError(f"a_s {tuple(a_s.shape)} does not match aq {tuple(aq.shape)} at block {act_block}")
    n = _gemm_shapes(packed, scales, fmt, k)
    work = _work_for(work, min(m, GEMM_MAX_M), n, k, aq.device)
    y = torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=aq.device)
    for r0 in range(0, m, GEMM_MAX_M):
        mc = min(GEMM_MAX_M, m - r0)
        _lib.check(_lib.load().stbl_amd_gemm_q_packed(fmt, _ptr(y[r0:r0 + mc]), _ptr(packed), _ptr(scales),
                                                      _ptr(aq[r0:r0 + mc]), _ptr(a_s[r0:r0 + mc]), mc, n, k, act_block,
                                                      int(out_f32), _ptr(work), _stream()), "gemm_q_packed")
    return y


def act_quant_e4m3(x, block=128):
    """(e4m3 codes uint8 [rows, k], E8M0 scale bytes uint8 [rows, k/block]) of bf16 x."""
    _need(x, torch.bfloat16, "x", 2)
    rows, k = x.shape
    codes = torch.empty((rows, k), dtype=torch.uint8, device=x.device)
    scales = torch.empty((rows, k // block), dtype=torch.uint8, device=x.device)
    _lib.check(_lib.load().stbl_amd_act_quant_e4m3(_ptr(x), rows, k, block, _ptr(codes), _ptr(scales), _stream()),
               "act_quant_e4m3")
    return codes, scales
