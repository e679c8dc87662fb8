"""The C-ABI library without a GPU: it loads, exports every function include/stbl_amd.h declares,
the ctypes table covers exactly that list, and argument checks fail before any device call."""

import ctypes
import os
import re

import pytest

from stblarge_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    src = ""
    for name in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if name.endswith(".h"):
            src += open(os.path.join(ROOT, "include", name)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"^\s*(?:void|int|int64_t|void\s*\*|uint64_t|const\s+char\s*\*)\s*\**\s*(stbl_\w+)\s*\(", src, re.M))


def test_library_exists():
    assert os.path.exists(_lib.LIB_PATH), "build the library first: python -m stblarge_amd.build"


def test_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    declared = header_functions()
    assert len(declared) >= 15
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_table_matches_header():
    assert set(_lib.SIGNATURES) == header_functions()


def test_load_binds_all():
    lib = _lib.load()
    assert lib.stbl_amd_version() >= 1


def test_argument_checks_fail_without_touching_the_device():
    lib = _lib.load()
    _lib.last_error()  # clear
    P = ctypes.c_void_p
    # k not a multiple of 32
    st = lib.stbl_amd_gemv_fp4(P(16), P(16), P(16), P(16), 1, 8, 33, 0, None)
    assert st < 0
    code, msg = _lib.last_error()
    assert code != 0 and "k % 32" in msg
    # one chunk past the largest K a launch takes (8 waves x 64 chunks)
    assert lib.stbl_amd_gemv_fp4(P(16), P(16), P(16), P(16), 1, 8, 16384 + 32, 0, None) < 0
    assert "k <= 16384" in _lib.last_error()[1]
    assert lib.stbl_amd_gemv_fp8(P(16), P(16), P(16), P(16), 1, 8, 8192 + 16, 0, None) < 0
    assert "k <= 8192" in _lib.last_error()[1]
    # m out of range
    assert lib.stbl_amd_gemv_fp8(P(16), P(16), P(16), P(16), 5, 8, 64, 0, None) < 0
    assert "m must be" in _lib.last_error()[1]
    # misaligned codes
    assert lib.stbl_amd_gemv_fp4(P(16), P(17), P(16), P(16), 1, 8, 64, 0, None) < 0
    assert "aligned" in _lib.last_error()[1]
    # void reference entry point records its failure
    lib.stbl_gemv_mxfp4(P(16), P(16), P(16), 8, 100, None)
    code, msg = _lib.last_error()
    assert code != 0 and "stbl_gemv_mxfp4" in msg
    assert _lib.last_error() == (0, "")
    # batch sizes: the reference ABI's batch stops at its kMxBatch of 16, the v2 batches at 64
    arr = (P * 65)(*[P(256)] * 65)
    lib.stbl_gemv_mxfp4_batch(arr, arr, arr, 17, 8, 256, None)
    assert "stbl_gemv_mxfp4_batch" in _lib.last_error()[1]
    assert lib.stbl_amd_gemv_fp4_batch(arr, arr, arr, arr, 65, 1, 8, 64, 0, None) < 0
    assert "1..64 matrices" in _lib.last_error()[1]


def test_check_raises():
    lib = _lib.load()
    with pytest.raises(_lib.StblError):
        _lib.check(lib.stbl_amd_quant_fp4(None, None, None, 1, 32, None), "quant_fp4")


def _zero_args(argtypes):
    import ctypes as C
    out = []
    for t in argtypes:
        if t in (C.c_int, C.c_int64, C.c_uint64):
            out.append(0)
        elif t is C.c_float:
            out.append(0.0)
        else:
            out.append(None)  # any pointer, char*, stream
    return out


_NO_ERROR_ON_ZERO = {"stbl_amd_version", "stbl_amd_last_error", "stbl_amd_expert_layout", "stbl_amd_moe_work_bytes",
                     "stbl_amd_gemm_work_bytes", "stbl_amd_cache_destroy", "stbl_amd_gguf_close",
                     "stbl_amd_cache_peek", "stbl_amd_read_floor_sink_words"}


@pytest.mark.parametrize("name", sorted(n for n in _lib.SIGNATURES if n not in _NO_ERROR_ON_ZERO))
def test_every_entry_point_rejects_null_and_zero_arguments(name):
    # null pointers and zero sizes: each entry point refuses before touching the device, records why
    # (readable through stbl_amd_last_error) and returns a negative status or NULL; void entry points
    # of the reference ABI only record it
    lib = _lib.load()
    _lib.last_error()  # clear
    ret, argtypes = _lib.SIGNATURES[name]
    r = getattr(lib, name)(*_zero_args(argtypes))
    code, msg = _lib.last_error()
    if ret is not None and r is not None:
        assert (r < 0) if isinstance(r, int) else not r, f"{name} returned {r}"
    assert code != 0 and msg, f"{name} recorded no error"


def test_moe_experts_host_jobs_at_the_largest_step():
    # The host side of stbl_amd_moe_experts builds its job tables before any launch: 16 tokens x
    # top-16 whose every pick is the shared slot of another format (272 pairs, 68 shared-format
    # jobs) must fit them. Without a GPU the call then fails at the launch with "no device"; on a
    # machine with a GPU this would launch on fake pointers, so it is skipped there.
    import torch

    if torch.cuda.device_count() > 0:
        pytest.skip("needs a machine without a GPU (fake device pointers)")
    lib = _lib.load()
    _lib.last_error()
    P = ctypes.c_void_p
    t, topk = 16, 16
    slots = (P * 2)(0x10000, 0x20000)
    pk = (ctypes.c_int * (t * topk))(*([1] * (t * topk)))
    wt = (ctypes.c_float * (t * topk))(*([0.1] * (t * topk)))
    st = lib.stbl_amd_moe_experts(0, P(0x30000), P(0x40000), t, 256, 128, slots, 2, pk, wt, topk, 1, 2, 0.0, 0, 0,
                                  P(0x50000), None)
    code, msg = _lib.last_error()
    assert st < 0 and "moe_experts launch" in msg, (st, msg)
    # phases 1 and 2 need the ready flags; phase 3 does not exist
    for phase, ready in ((1, None), (3, (ctypes.c_int * 2)(1, 0))):
        st = lib.stbl_amd_moe_experts_phase(0, P(0x30000), P(0x40000), t, 256, 128, slots, 2, pk, wt, topk, 1, 2, 0.0,
                                            0, 0, ready, phase, P(0x50000), None)
        assert st < 0 and "phase" in _lib.last_error()[1]


def test_gemm_workspace_for_m_serves_every_smaller_m():
    # the GEMM's tile plan depends on m (row groups when m > 32), and a plan with split-K partial
    # tiles can need more workspace than one without: a workspace sized for m must still hold any
    # smaller m's partials, activation codes and scales (n = 6100, K = 2048 switches from one plan
    # without partials at m = 64 to a split-K plan at m <= 32)
    lib = _lib.load()
    for n, k in ((6100, 2048), (7168, 2048), (2048, 7168), (4096, 4096)):
        sizes = [lib.stbl_amd_gemm_work_bytes(m, n, k) for m in range(1, 65)]
        assert all(a <= b for a, b in zip(sizes, sizes[1:])), (n, k, sizes)
