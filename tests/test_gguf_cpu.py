"""The GGUF reader (stbl_amd_gguf_*, the reference's stbl/gguf.cpp) and the expert-file writer, on CPU.

The reader is pinned on a header assembled byte by byte in this file from the GGUF v3 layout
(magic, version, tensor and key counts, keys, tensor infos with offsets relative to the data
start, data aligned to general.alignment), not by the writer, so a shared misreading of the format
by writer and reader cannot pass. The OCP -> GGUF block conversion is pinned on the oracle's
(itself pinned on the golden vector of test_oracle_cpu.py).
"""

import struct

import numpy as np
import pytest

import oracle
from stblarge_amd import _lib, gguf

pytestmark = pytest.mark.filterwarnings("ignore")


def _s(text):
    b = text.encode()
    return struct.pack("<Q", len(b)) + b


def _hand_file(path, alignment=64):
    # keys: alignment (u32), a float, a string, a u64 array, a string array, a bool
    kv = [
        _s("general.alignment") + struct.pack("<II", 4, alignment),
        _s("test.scale") + struct.pack("<If", 6, 2.5),
        _s("general.name") + struct.pack("<I", 8) + _s("tiny"),
        _s("test.ids") + struct.pack("<IIQ", 9, 10, 3) + struct.pack("<3Q", 7, 1 << 40, 9),
        _s("test.words") + struct.pack("<IIQ", 9, 8, 2) + _s("ab") + _s("c"),
        _s("test.flag") + struct.pack("<IB", 7, 1),
        _s("test.u32s") + struct.pack("<IIQ", 9, 4, 2) + struct.pack("<2I", 5, 6),
    ]
    # tensors: F32 [3, 2] at relative 0 (24 bytes), MXFP4 [64, 2, 3] at relative 64 (12 blocks, 204 bytes)
    infos = [_s("a.f32") + struct.pack("<I2QIQ", 2, 3, 2, 0, 0),
             _s("blk.0.ffn_gate_exps.weight") + struct.pack("<I3QIQ", 3, 64, 2, 3, 39, 64)]
    head = struct.pack("<IIQQ", 0x46554747, 3, len(infos), len(kv)) + b"".join(kv) + b"".join(infos)
    base = (len(head) + alignment - 1) // alignment * alignment
    f32 = np.arange(6, dtype=np.float32)
    blocks = np.arange(204, dtype=np.uint8)
    body = bytearray(64 + 204)
    body[:24] = f32.tobytes()
    body[64:] = blocks.tobytes()
    path.write_bytes(head + bytes(base - len(head)) + bytes(body))
    return base, f32, blocks


def test_reader_on_hand_assembled_file(tmp_path):
    p = tmp_path / "hand.gguf"
    base, f32, blocks = _hand_file(p)
    with gguf.GgufFile(p) as g:
        a = g.tensor("a.f32")
        assert a == {"type": 0, "dims": [3, 2], "offset": base, "nbytes": 24}
        e = g.tensor("blk.0.ffn_gate_exps.weight")
        assert e == {"type": 39, "dims": [64, 2, 3], "offset": base + 64, "nbytes": 204}
        raw = p.read_bytes()
        assert raw[a["offset"]:a["offset"] + 24] == f32.tobytes()
        assert raw[e["offset"]:e["offset"] + 204] == blocks.tobytes()
        assert g.u32("general.alignment") == 64
        assert g.f32("test.scale") == 2.5
        assert g.uints("test.ids") == [7, 1 << 40, 9]
        assert g.uints("test.u32s") == [5, 6]
        assert g.tensor("missing") is None and g.u32("missing") is None
        assert g.u32("test.scale") is None  # wrong type reads as absent
        assert g.uints("test.words") is None  # a string array is not a uint array


def test_reader_default_alignment(tmp_path):
    # without general.alignment the data start is aligned to 32
    info = _s("t") + struct.pack("<I1QIQ", 1, 4, 0, 0)
    head = struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + info
    base = (len(head) + 31) // 32 * 32
    p = tmp_path / "a32.gguf"
    p.write_bytes(head + bytes(base - len(head)) + np.ones(4, np.float32).tobytes())
    with gguf.GgufFile(p) as g:
        assert g.tensor("t")["offset"] == base


@pytest.mark.parametrize("damage", ["magic", "truncated", "past_end", "empty"])
def test_reader_rejects_damaged_files(tmp_path, damage):
    p = tmp_path / "bad.gguf"
    _hand_file(p)
    raw = bytearray(p.read_bytes())
    if damage == "magic":
        raw[0] = ord("X")
    elif damage == "truncated":
        raw = raw[:40]
    elif damage == "past_end":
        raw = raw[:-10]  # the MXFP4 tensor now runs past the end
    else:
        raw = bytearray()
    p.write_bytes(bytes(raw))
    with pytest.raises(RuntimeError) as e:
        gguf.GgufFile(p)
    assert "gguf_open" in str(e.value)


@pytest.mark.parametrize("case", ["huge_dims", "huge_offset"])
def test_reader_rejects_overflowing_tensor_infos(tmp_path, case):
    # a shape whose element count overflows 64 bits, or an offset near 2^64, must not wrap around
    # into a small in-bounds range
    dims = (1 << 40, 1 << 40) if case == "huge_dims" else (4,)
    off = 0 if case == "huge_dims" else (1 << 64) - 16
    info = _s("t") + struct.pack("<I", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims) + struct.pack("<IQ", 0, off)
    head = struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + info
    base = (len(head) + 31) // 32 * 32
    p = tmp_path / "ovf.gguf"
    p.write_bytes(head + bytes(base - len(head)) + bytes(64))
    with pytest.raises(RuntimeError, match="implausible shape|past the end"):
        gguf.GgufFile(p)


def test_reader_missing_file(tmp_path):
    with pytest.raises(RuntimeError, match="cannot open"):
        gguf.GgufFile(tmp_path / "nope.gguf")


def test_writer_round_trip(tmp_path):
    p = tmp_path / "w.gguf"
    rng = np.random.default_rng(0)
    a = rng.standard_normal((5, 7)).astype(np.float32)
    b = rng.integers(0, 256, 3 * 17 * 4, dtype=np.uint8)
    placed = gguf.write(p, [("a", gguf.QT_F32, [7, 5], a), ("b", gguf.QT_MXFP4, [96, 4], lambda: iter([b[:51], b[51:]]))],
                        kv={"x.n": (gguf.GV_U32, 11), "x.l": (gguf.GV_ARR, (gguf.GV_U32, [1, 2]))}, alignment=16384)
    raw = p.read_bytes()
    with gguf.GgufFile(p) as g:
        for name, off, nb in placed:
            t = g.tensor(name)
            assert (t["offset"], t["nbytes"]) == (off, nb) and off % 16384 == 0
        assert raw[placed[0][1]:placed[0][1] + 140] == a.tobytes()
        assert raw[placed[1][1]:placed[1][1] + 204] == b.tobytes()
        assert g.u32("x.n") == 11 and g.uints("x.l") == [1, 2] and g.u32("general.alignment") == 16384


def test_ocp_to_gguf17_matches_oracle():
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 256, (9, 64), dtype=np.uint8)
    scales = rng.integers(100, 140, (9, 4), dtype=np.uint8)
    assert np.array_equal(gguf.ocp_to_gguf17(codes, scales), oracle.ocp_to_gguf17(codes, scales))


def test_write_experts_layout(tmp_path):
    # expert e's part p sits at the tensor's offset + e * (rows * k / 32 * 17)
    dim, inter, n = 64, 32, 3
    rng = np.random.default_rng(2)
    ex = {}

    def expert(layer, e):
        if (layer, e) not in ex:
            ex[layer, e] = [rng.integers(0, 256, s, dtype=np.uint8) for s in
                            ((inter, dim // 2), (inter, dim // 32), (inter, dim // 2), (inter, dim // 32),
                             (dim, inter // 2), (dim, inter // 32))]
        return ex[layer, e]
    p = tmp_path / "e.gguf"
    gguf.write_experts(p, expert, 2, n, dim, inter, first_layer=3)
    raw = np.fromfile(p, np.uint8)
    with gguf.GgufFile(p) as g:
        for layer in (3, 4):
            for pi, part in enumerate(("gate", "up", "down")):
                t = g.tensor(gguf.expert_tensor(layer, part))
                assert t["type"] == gguf.QT_MXFP4
                assert t["dims"] == ([dim, inter, n] if pi < 2 else [inter, dim, n])
                per = dim * inter // 32 * 17
                for e in range(n):
                    got = raw[t["offset"] + e * per:t["offset"] + (e + 1) * per]
                    want = oracle.ocp_to_gguf17(ex[layer, e][2 * pi], ex[layer, e][2 * pi + 1]).ravel()
                    assert np.array_equal(got, want)


def test_cache_create_gguf_rejects_bad_files(tmp_path):
    # the checks run before any device call, so they hold without a GPU
    lib = _lib.load()
    p = tmp_path / "x.gguf"
    _hand_file(p)  # its gate tensor has inter = 2
    assert not lib.stbl_amd_cache_create_gguf(4, str(p).encode(), 0, 1, 2, 1)
    assert "multiples of 32" in _lib.last_error()[1]
    dim, inter = 64, 32
    blocks = np.zeros(dim * inter * 2 // 32 * 17, np.uint8)
    gguf.write(p, [(gguf.expert_tensor(0, "gate"), gguf.QT_MXFP4, [dim, inter, 2], blocks)])  # no up / down
    assert not lib.stbl_amd_cache_create_gguf(4, str(p).encode(), 0, 1, 2, 1)
    assert "no tensor blk.0.ffn_up_exps.weight" in _lib.last_error()[1]
    assert not lib.stbl_amd_cache_create_gguf(4, str(p).encode(), 1, 1, 2, 1)  # no layer 1
    assert "no tensor blk.1.ffn_gate_exps.weight" in _lib.last_error()[1]
    assert not lib.stbl_amd_cache_create_gguf(4, str(p).encode(), 0, 1, 0, 1)  # no readers
    assert not lib.stbl_amd_cache_create_gguf(4, str(tmp_path / "none").encode(), 0, 1, 2, 1)
    # mismatched shapes across parts
    t = [(gguf.expert_tensor(0, "gate"), gguf.QT_MXFP4, [dim, inter, 2], np.zeros(dim * inter * 2 // 32 * 17, np.uint8)),
         (gguf.expert_tensor(0, "up"), gguf.QT_MXFP4, [dim, inter, 2], np.zeros(dim * inter * 2 // 32 * 17, np.uint8)),
         (gguf.expert_tensor(0, "down"), gguf.QT_MXFP4, [dim, inter, 2], np.zeros(dim * inter * 2 // 32 * 17, np.uint8))]
    gguf.write(p, t)
    assert not lib.stbl_amd_cache_create_gguf(4, str(p).encode(), 0, 1, 2, 1)
    assert "shape differs" in _lib.last_error()[1]


_MUTATE = r'''
import struct, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from stblarge_amd import gguf
raw = open(sys.argv[2], "rb").read()
head = int(sys.argv[3])
rng = np.random.default_rng(int(sys.argv[4]))
path = sys.argv[2] + ".m"
opened = refused = 0
for it in range(int(sys.argv[5])):
    b = bytearray(raw)
    kind = it % 4
    if kind == 0:  # random bytes in the header
        for _ in range(rng.integers(1, 8)):
            b[rng.integers(0, head)] = rng.integers(0, 256)
    elif kind == 1:  # a count, length, dim or offset field set to an extreme value
        at = int(rng.integers(0, head - 8)) & ~7
        b[at:at + 8] = struct.pack("<Q", [0, 1, 2**31, 2**32 - 1, 2**63, 2**64 - 1][int(rng.integers(0, 6))])
    elif kind == 2:  # truncated anywhere
        b = b[:rng.integers(0, len(b))]
    else:  # a header region repeated (lengths now point into the wrong fields)
        s = int(rng.integers(0, head)); e = int(rng.integers(s, head))
        b = b[:e] + b[s:e] + b[e:]
    open(path, "wb").write(bytes(b))
    try:
        with gguf.GgufFile(path) as g:
            g.tensor("a.f32"); g.tensor("blk.0.ffn_gate_exps.weight"); g.u32("general.alignment"); g.uints("test.ids")
        opened += 1
    except RuntimeError:
        refused += 1
print(opened, refused)
'''


def test_reader_survives_mutated_headers(tmp_path):
    # 400 corrupted copies of the hand-assembled file: each either opens or is refused with an error;
    # none may crash the process (run in a child, so a crash fails this test instead of the session)
    import os
    import subprocess
    import sys

    p = tmp_path / "hand.gguf"
    base, _, _ = _hand_file(p)
    script = tmp_path / "mutate.py"
    script.write_text(_MUTATE)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, str(script), root, str(p), str(base), "5", "400"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, f"reader crashed (exit {r.returncode}): {r.stderr[-2000:]}"
    opened, refused = map(int, r.stdout.split()[-2:])
    assert opened + refused == 400 and refused > 0
