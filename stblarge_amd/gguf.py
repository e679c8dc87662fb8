"""GGUF files of routed experts: the reader (over stbl_amd_gguf_*) and a streaming writer.

The reference engine reads one GGUF file converted from the checkpoint (stbl/gguf.h:9-36,
stbl/gguf.cpp); its routed experts are the tensors blk.N.ffn_{gate,up,down}_exps.weight, MXFP4
blocks of 17 bytes with dims [k, rows, experts] (innermost first), and the data section is aligned
to general.alignment. The writer produces that layout from OCP codes and scales, so tests and
benchmarks can build expert files without the reference's converter.
"""

import ctypes
import struct

import numpy as np

from . import _lib

# GGUF metadata value types
GV_U8, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STR, GV_ARR, GV_U64, GV_I64, GV_F64 = range(13)
# tensor types (stbl/gguf.h:34-36)
QT_F32, QT_I8, QT_BF16, QT_MXFP4, QT_STBL_E4M3, QT_STBL_E8M0 = 0, 24, 30, 39, 200, 201

_SCALAR = {GV_U8: "<B", GV_I8: "<b", GV_U16: "<H", GV_I16: "<h", GV_U32: "<I", GV_I32: "<i", GV_F32: "<f",
           GV_BOOL: "<?", GV_U64: "<Q", GV_I64: "<q", GV_F64: "<d"}
_NOT_FOUND = -500  # -hipErrorNotFound


def expert_tensor(layer, part):
    """Name of a layer's routed-expert tensor; part is gate, up or down."""
    return f"blk.{layer}.ffn_{part}_exps.weight"


def tensor_bytes(qtype, n):
    if qtype == QT_MXFP4:
        return n // 32 * 17
    return n * {QT_F32: 4, 1: 2, QT_BF16: 2, QT_I8: 1, QT_STBL_E4M3: 1, QT_STBL_E8M0: 1}[qtype]


class GgufFile:
    """A parsed GGUF header: tensor infos with absolute offsets, and scalar metadata."""

    def __init__(self, path):
        self.path = str(path)
        self.handle = _lib.load().stbl_amd_gguf_open(self.path.encode())
        if not self.handle:
            _lib.check(-1, "gguf_open")

    def tensor(self, name):
        """{type, dims, offset, nbytes} of a tensor, or None when the file has no such tensor."""
        t = ctypes.c_uint32()
        dims = (ctypes.c_uint64 * 4)()
        nd = ctypes.c_int()
        off, nb = ctypes.c_uint64(), ctypes.c_uint64()
        rc = _lib.load().stbl_amd_gguf_tensor(self.handle, name.encode(), ctypes.byref(t), dims, ctypes.byref(nd),
                                              ctypes.byref(off), ctypes.byref(nb))
        if rc == _NOT_FOUND:
            return None
        _lib.check(rc, "gguf_tensor")
        return {"type": t.value, "dims": [int(d) for d in dims[:nd.value]], "offset": off.value, "nbytes": nb.value}

    def u32(self, key):
        v = ctypes.c_uint32()
        rc = _lib.load().stbl_amd_gguf_u32(self.handle, key.encode(), ctypes.byref(v))
        return None if rc == _NOT_FOUND else (_lib.check(rc, "gguf_u32"), v.value)[1]

    def f32(self, key):
        v = ctypes.c_float()
        rc = _lib.load().stbl_amd_gguf_f32(self.handle, key.encode(), ctypes.byref(v))
        return None if rc == _NOT_FOUND else (_lib.check(rc, "gguf_f32"), v.value)[1]

    def uints(self, key):
        lib = _lib.load()
        n = lib.stbl_amd_gguf_uints(self.handle, key.encode(), None, 0)
        if n == _NOT_FOUND:
            return None
        _lib.check(min(int(n), 0), "gguf_uints")
        out = (ctypes.c_uint64 * max(int(n), 1))()
        lib.stbl_amd_gguf_uints(self.handle, key.encode(), out, n)
        return [int(v) for v in out[:n]]

    def close(self):
        if self.handle:
            _lib.load().stbl_amd_gguf_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype == GV_STR:
        return _str(v)
    if vtype == GV_ARR:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, x) for x in items)
    return struct.pack(_SCALAR[vtype], v)


def ocp_to_gguf17(codes, scales):
    """OCP FP4 codes [rows, k/2] (element 2j in the low nibble of byte j) and E8M0 scales
    [rows, k/32] -> GGUF MXFP4 blocks [rows, k/32 * 17] (byte 0 the scale, byte 1+i element i in the
    low nibble and element 16+i in the high one)."""
    codes, scales = np.asarray(codes, np.uint8), np.asarray(scales, np.uint8)
    rows, nb = scales.shape
    c = codes.reshape(rows, nb, 16)
    v = np.empty((rows, nb, 32), np.uint8)
    v[..., 0::2] = c & 15
    v[..., 1::2] = c >> 4
    out = np.empty((rows, nb, 17), np.uint8)
    out[..., 0] = scales
    out[..., 1:] = v[..., :16] | (v[..., 16:] << 4)
    return out.reshape(rows, nb * 17)


def write(path, tensors, kv=None, alignment=32):
    """Writes a GGUF v3 file. tensors: list of (name, qtype, dims innermost first, data), where data
    is a uint8-viewable array of the tensor's bytes, or a callable returning such an array or an
    iterable of arrays that concatenate to it (called when the tensor is written, so large files
    need not be held in memory). kv: {key: (value type, value)}; general.alignment is written when
    alignment differs from GGUF's default 32. Returns [(name, absolute offset, bytes)]."""
    kv = dict(kv or {})
    if alignment != 32:
        kv["general.alignment"] = (GV_U32, alignment)
    infos, off = [], 0
    for name, qtype, dims, _ in tensors:
        n = int(np.prod(dims))
        nb = tensor_bytes(qtype, n)
        infos.append((name, qtype, dims, off, nb))
        off = (off + nb + alignment - 1) // alignment * alignment
    head = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kv))
    head += b"".join(_str(k) + struct.pack("<I", t) + _value(t, v) for k, (t, v) in kv.items())
    for name, qtype, dims, o, _ in infos:
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", qtype, o)
    with open(path, "wb") as f:
        f.write(head)
        base = (len(head) + alignment - 1) // alignment * alignment
        f.write(b"\0" * (base - len(head)))
        for (name, qtype, dims, data), (_, _, _, o, nb) in zip(tensors, infos):
            arr = data() if callable(data) else data
            chunks = [arr] if isinstance(arr, np.ndarray) else arr
            f.seek(base + o)
            done = 0
            for chunk in chunks:
                raw = np.ascontiguousarray(chunk).view(np.uint8).reshape(-1)
                done += raw.size
                if done > nb:
                    break
                f.write(raw.data)
            if done != nb:
                raise ValueError(f"{name}: {done} bytes given, {nb} expected")
        end = base + off
        if f.tell() < end:
            f.truncate(end)
    return [(name, base + o, nb) for name, _, _, o, nb in infos]


def write_experts(path, expert, n_layers, n_experts, dim, inter, alignment=16384, first_layer=0, kv=None):
    """A GGUF file of routed FP4 experts as the reference's converter lays them out: per layer
    blk.N.ffn_{gate,up,down}_exps.weight, MXFP4 [dim, inter, experts] for gate and up and
    [inter, dim, experts] for down, expert e's blocks after expert e-1's. expert(layer, e) returns
    the OCP parts [gate codes, gate scales, up codes, up scales, down codes, down scales] as numpy
    arrays. Experts are produced one at a time per tensor, so memory stays at one expert's part."""
    tensors = []
    for layer in range(first_layer, first_layer + n_layers):
        for p, part in enumerate(("gate", "up", "down")):
            dims = [dim, inter, n_experts] if p < 2 else [inter, dim, n_experts]

            def chunks(layer=layer, p=p):
                for e in range(n_experts):
                    parts = expert(layer, e)
                    yield ocp_to_gguf17(parts[2 * p], parts[2 * p + 1])
            tensors.append((expert_tensor(layer, part), QT_MXFP4, dims, chunks))
    return write(path, tensors, kv, alignment)
