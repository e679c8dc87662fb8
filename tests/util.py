"""Comparison helpers shared by the GPU parity tests."""

import numpy as np
import torch

import oracle


def np_(t):
    """Device/host tensor -> numpy (bf16 widened to fp32)."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.numpy()


def bits_equal(got, want):
    """Bit-identical fp32 arrays (NaNs compared by position only)."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    gn, wn = np.isnan(got), np.isnan(want)
    if not np.array_equal(gn, wn):
        return False
    return np.array_equal(got[~gn].view(np.uint32), want[~wn].view(np.uint32))


def rel_err(got, want):
    """max |got - want| / max |want| -- the reference's check() metric (stbl/test_kernels.py:47-52)."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / max(float(np.max(np.abs(want))), 1e-30))


def bf16_ulps(got_bf16, want_f64):
    """Per element, how many bf16 steps the bf16 result is from bf16(want) (0 = same rounding)."""
    want = oracle.f2bf_bits(np.asarray(want_f64, np.float32)).astype(np.int32)
    got = oracle.f2bf_bits(np.asarray(got_bf16, np.float32)).astype(np.int32)

    def ordered(b):  # sign-magnitude bf16 bits -> monotone integers
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)

    return np.abs(ordered(got) - ordered(want))


def assert_gemv(got_f32, got_bf16, want, tol=1e-3):
    """fp32 output within `tol` (max error over max output), bf16 output at most one bf16 step from
    bf16(want).

    The step check skips outputs below 2^-16 of the largest: those are sums that cancel to ~1e-5 of
    their terms, whose last bf16 digits fp32 accumulation in any order cannot resolve (a row of 5120
    random FP4 products summing to 5.9e-5 from an absolute sum of 608 came out 3.9e-7 from exact,
    two bf16 steps). The max-over-max bound above still covers them."""
    e = rel_err(got_f32, want)
    assert e <= tol, f"relative error {e:.3e} > {tol}"
    if got_bf16 is not None:
        u = bf16_ulps(got_bf16, want)
        w = np.abs(np.asarray(want, np.float64))
        resolved = w > 2.0 ** -16 * w.max()
        assert u[resolved].max(initial=0) <= 1, f"bf16 output {u[resolved].max()} steps away"
        assert np.mean(u[resolved]) < 0.05, f"{np.mean(u[resolved]):.3f} of bf16 outputs flipped"
    return e


def assert_moe_sum(got_bf16, want, term_abs_sum):
    """A routed MoE output y = bf16(sum_i o_i) against the oracle's, where each expert output o_i is
    a bf16-rounded FFN that may sit one bf16 step from the oracle's (the fp32 sums inside take
    another order). Every element is held to |y - want| <= 2^-7 (sum_i |o_i| + |want|): one step
    of each term plus one of the result (a bf16 step of v is at most 2^-7 |v|). Where terms cancel
    that allows several steps of a small y, so flips (outputs not equal to the oracle's) must also
    stay rare."""
    got = np.asarray(got_bf16, np.float64)
    want = np.asarray(want, np.float64)
    bound = 2.0 ** -7 * (np.asarray(term_abs_sum, np.float64) + np.abs(want))
    assert np.all(np.abs(got - want) <= bound), f"{int(np.sum(np.abs(got - want) > bound))} outputs past the bound"
    u = bf16_ulps(got, want)
    assert np.mean(u > 0) < 0.02, f"{np.mean(u > 0):.4f} of outputs flipped"


def read_device(addr, n):
    """n bytes at device address addr (a slot handed out by an expert cache) as a uint8 tensor,
    through the HIP runtime torch already loaded (the one libstbl_amd.so binds to)."""
    import ctypes
    import os

    hip = ctypes.CDLL(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so"))
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    dst = torch.empty(n, dtype=torch.uint8)
    assert hip.hipMemcpy(ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(addr), n, 2) == 0  # device to host
    return dst
