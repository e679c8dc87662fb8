"""Builds libstbl_amd.so in-tree with hipcc for gfx950 (no JIT cache: the .so travels with the tree).

Run: python -m stblarge_amd.build   (or __graft_entry__.build()).
"""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libstbl_amd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["abi.hip", "quant.hip", "gemv.hip", "moe.hip", "gemm.hip", "expert_cache.hip", "gguf.hip", "calib.hip"]

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 VALU ops are kept out of the generated code (they are not needed here).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Products and sums written in the sources may fuse into FMAs (each kernel's exactness argument
    # allows for it), but not the multiply-subtract pairs inside the compiler's own expansions of
    # expf / log1pf: under -ffp-contract=fast the backend fuses the range reduction's x * log2(e) - n
    # into one FMA, which counts the product's rounding error twice (device expf off by up to 43 fp32
    # ulps at |x| ~ 70, 5 ulps within |x| < 10); fast-honor-pragmas leaves them as written.
    "-ffp-contract=fast-honor-pragmas",
]


def sources():
    return [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]


def build(verbose=False):
    """Compile every HIP source into one shared library. Always recompiles."""
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *FLAGS, "-I", CSRC, "-I", os.path.join(os.path.dirname(HERE), "include"), *sources(), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", LIB)
