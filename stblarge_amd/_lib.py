"""ctypes binding of libstbl_amd.so (the C ABI declared in include/stbl_amd.h).

The library is loaded from the package directory, where stblarge_amd.build puts it. There is no
fallback: if the library is missing, load() raises, and every op in stblarge_amd.ops fails loudly.
"""

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# STBL_AMD_LIB names another build of the library (for comparing builds); default the in-tree one
LIB_PATH = os.environ.get("STBL_AMD_LIB") or os.path.join(HERE, "libstbl_amd.so")

P = ctypes.c_void_p
I = ctypes.c_int
F = ctypes.c_float
PP = ctypes.POINTER(ctypes.c_void_p)
PF = ctypes.POINTER(ctypes.c_float)
PI = ctypes.POINTER(ctypes.c_int)
U64 = ctypes.c_uint64
PU64 = ctypes.POINTER(ctypes.c_uint64)

# name -> (restype, argtypes). Every function of include/stbl_amd.h appears here.
SIGNATURES = {
    # reference surface (stbl/kernels.h)
    "stbl_act_quant_fp8": (None, [P, I, P]),
    "stbl_round_bf16": (None, [P, I, P]),
    "stbl_gemv_fp8": (None, [P, P, P, P, I, I, I, P]),
    "stbl_gemv_mxfp4": (None, [P, P, P, I, I, P]),
    "stbl_gemv_mxfp4_batch": (None, [PP, PP, PP, I, I, I, P]),
    "stbl_gemv_f32": (None, [P, P, P, I, I, I, P]),
    "stbl_sqrt_softplus": (None, [P, I, P]),
    "stbl_gemv_bf16": (None, [P, P, P, I, I, I, I, P]),
    "stbl_swiglu": (None, [P, P, P, F, F, I, P]),
    "stbl_swiglu_batch": (None, [P, P, P, PF, I, F, I, P]),
    "stbl_axpy": (None, [P, P, F, I, P]),
    # v2
    "stbl_amd_gemv_fp4": (I, [P, P, P, P, I, I, I, I, P]),
    "stbl_amd_gemv_fp8": (I, [P, P, P, P, I, I, I, I, P]),
    "stbl_amd_gemv_fp4_batch": (I, [PP, PP, PP, PP, I, I, I, I, I, P]),
    "stbl_amd_gemv_fp8_batch": (I, [PP, PP, PP, PP, I, I, I, I, I, P]),
    "stbl_amd_act_quant": (I, [P, I, I, I, I, P, P, P, P]),
    "stbl_amd_quant_fp4": (I, [P, P, P, I, I, P]),
    "stbl_amd_quant_fp8_b128": (I, [P, P, P, I, I, P]),
    "stbl_amd_quant_fp8_e8m0": (I, [P, P, P, I, I, P]),
    "stbl_amd_dequant_fp4": (I, [P, P, P, I, I, P]),
    "stbl_amd_dequant_gguf17": (I, [P, P, I, I, P]),
    "stbl_amd_dequant_fp8": (I, [P, P, P, I, I, I, P]),
    "stbl_amd_expert_layout": (U64, [I, I, I, PU64]),
    "stbl_amd_expert_ffn": (I, [I, P, P, P, I, I, I, F, F, I, I, P, P]),
    "stbl_amd_moe_experts": (I, [I, P, P, I, I, I, PP, I, PI, PF, I, I, I, F, I, I, P, P]),
    "stbl_amd_moe_experts_phase": (I, [I, P, P, I, I, I, PP, I, PI, PF, I, I, I, F, I, I, PI, I, P, P]),
    "stbl_amd_moe_experts_noalloc": (I, [I, P, P, I, I, I, PP, I, PI, PF, I, I, I, F, I, I, P]),
    "stbl_amd_moe_work_bytes": (U64, [I, I, I, I]),
    "stbl_amd_route": (I, [P, P, I, I, I, F, I, P, P, P, P]),
    "stbl_amd_gemm": (I, [I, P, P, P, P, I, I, I, I, I, P, P]),
    "stbl_amd_gemm_q": (I, [I, P, P, P, P, P, I, I, I, I, I, P, P]),
    "stbl_amd_gemm_work_bytes": (U64, [I, I, I]),
    "stbl_amd_gemm_pack": (I, [I, P, P, I, I, P]),
    "stbl_amd_gemm_q_packed": (I, [I, P, P, P, P, P, I, I, I, I, I, P, P]),
    "stbl_amd_gemm_packed": (I, [I, P, P, P, P, I, I, I, I, I, P, P]),
    "stbl_amd_act_quant_e4m3": (I, [P, I, I, I, P, P, P]),
    "stbl_amd_cache_create": (P, [I, U64, P, U64, I, I]),
    "stbl_amd_cache_create_gguf": (P, [I, ctypes.c_char_p, I, I, I, I]),
    "stbl_amd_cache_file_info": (I, [P, PU64]),
    "stbl_amd_cache_enable_prefetch": (I, [P, I]),
    "stbl_amd_cache_prefetch": (I, [P, PI, I, I]),
    "stbl_amd_cache_prefetch_stats": (I, [P, PU64]),
    "stbl_amd_cache_prefetch_pause": (I, [P, I]),
    "stbl_amd_cache_destroy": (None, [P]),
    "stbl_amd_gguf_open": (P, [ctypes.c_char_p]),
    "stbl_amd_gguf_close": (None, [P]),
    "stbl_amd_gguf_tensor": (I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32), PU64, PI, PU64, PU64]),
    "stbl_amd_gguf_u32": (I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)]),
    "stbl_amd_gguf_f32": (I, [P, ctypes.c_char_p, PF]),
    "stbl_amd_gguf_uints": (ctypes.c_int64, [P, ctypes.c_char_p, PU64, ctypes.c_int64]),
    "stbl_amd_cache_lookup": (I, [P, PI, I, I, PP, PI, P]),
    "stbl_amd_cache_lookup_begin": (I, [P, PI, I, I, PP, PI, PI, P]),
    "stbl_amd_cache_lookup_end": (I, [P, P]),
    "stbl_amd_cache_note_guesses": (I, [P, PI, I, I]),
    "stbl_amd_cache_lookahead": (I, [P, PU64]),
    "stbl_amd_cache_mark_used": (I, [P, P]),
    "stbl_amd_cache_stats": (I, [P, PU64]),
    "stbl_amd_cache_peek": (P, [P, I, I]),
    "stbl_amd_cache_fail_refill_after": (I, [P, I]),
    "stbl_amd_read_floor": (I, [P, U64, P, P]),
    "stbl_amd_read_floor_sink_words": (U64, [U64]),
    "stbl_amd_clock_stamp": (I, [P, I, P]),
    "stbl_amd_clock_rate_khz": (I, [P]),
    "stbl_amd_last_error": (I, [ctypes.c_char_p, I]),
    "stbl_amd_version": (I, []),
}

_lib = None


class StblError(RuntimeError):
    pass


def load():
    """The bound library (loaded once). Raises if it was not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise StblError(f"{LIB_PATH} is missing: build it with `python -m stblarge_amd.build`")
        # torch first: its HIP runtime is then the one the library's HIP symbols bind to, so device
        # memory, streams and graphs are shared with torch's (one runtime per process)
        import torch  # noqa: F401

        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error():
    """(code, message) of the calling thread's last recorded failure; clears it."""
    buf = ctypes.create_string_buffer(256)
    code = load().stbl_amd_last_error(buf, 256)
    return code, buf.value.decode(errors="replace")


def check(status, what):
    """Raise StblError for a non-zero v2 status (or a recorded failure of a void entry point)."""
    code, msg = last_error()
    if status not in (0, None) or code:
        raise StblError(f"{what} failed: status {status}, hipError {code}: {msg}")
