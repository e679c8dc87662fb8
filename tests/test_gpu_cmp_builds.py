"""The build-comparison harness (stblarge_amd/cmp_builds.py, the role of stbl/cmp_kernels.py:12-64):
two independently loaded copies of this build agree bit for bit on every hot entry point (the kernels
are deterministic run to run), and the harness reports a planted one-bit difference in exactly the
case that has it, and a case that one build rejects, instead of calling either identical."""

import ctypes
import os

import pytest
import torch

from stblarge_amd import _lib, cmp_builds

pytestmark = pytest.mark.gpu


def _hip():
    hip = ctypes.CDLL(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so"))
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return hip


class _Planted:
    """A loaded build whose entry point `name` is changed after the call by `change(first argument)`;
    every other entry point is the build's own."""

    def __init__(self, lib, name, change):
        self._lib, self._name, self._change = lib, name, change

    def __getattr__(self, attr):
        fn = getattr(self._lib, attr)
        if attr != self._name:
            return fn

        def wrapped(*args):
            r = fn(*args)
            self._change(*args)
            return r
        return wrapped


def test_build_against_itself(gpu):
    _lib.load()
    assert cmp_builds.compare(_lib.LIB_PATH, _lib.LIB_PATH, seeds=1) == []


def test_planted_one_bit_difference_is_reported(gpu):
    _lib.load()
    hip = _hip()

    def flip(y, *rest):  # bit 0 of element 5 of stbl_gemv_f32's output
        torch.cuda.synchronize()
        b = (ctypes.c_uint8 * 1)()
        assert hip.hipMemcpy(ctypes.cast(b, ctypes.c_void_p), ctypes.c_void_p(y.value + 20), 1, 2) == 0
        b[0] ^= 1
        assert hip.hipMemcpy(ctypes.c_void_p(y.value + 20), ctypes.cast(b, ctypes.c_void_p), 1, 1) == 0

    old = cmp_builds._load(_lib.LIB_PATH)
    new = _Planted(cmp_builds._load(_lib.LIB_PATH), "stbl_gemv_f32", flip)
    assert cmp_builds.compare(new, old, seeds=1) == [("stbl_gemv_f32 256x5120 seed 0", 1)]


def test_rejected_case_is_reported(gpu):
    # a build that refuses stbl_gemv_mxfp4 (here: called with rows = 0, so it records an error and
    # writes nothing) must not pass as identical to one that refuses it too
    _lib.load()

    class Refusing:
        def __init__(self, lib):
            self._lib = lib

        def __getattr__(self, attr):
            fn = getattr(self._lib, attr)
            if attr != "stbl_gemv_mxfp4":
                return fn
            return lambda y, w, x, rows, k, st: fn(y, w, x, 0, k, st)

    a = Refusing(cmp_builds._load(_lib.LIB_PATH))
    b = Refusing(cmp_builds._load(_lib.LIB_PATH))
    bad = cmp_builds.compare(a, b, seeds=1)
    assert [n for n, _ in bad] == ["stbl_gemv_mxfp4 2304x5120 seed 0", "stbl_gemv_mxfp4 5120x2304 seed 0"]
    assert all(r == "rejected by the new build and the old build" for _, r in bad)
