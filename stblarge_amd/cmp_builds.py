"""Bitwise comparison of two builds of libstbl_amd.so on the hot entry points (the role of the
reference's stbl/cmp_kernels.py:1-64 for its builds), to guard performance work: a change that only
moves work between lanes, waves or workgroups must leave every output bit unchanged.

    python -m stblarge_amd.cmp_builds NEW.so OLD.so      # two built libraries
    python -m stblarge_amd.cmp_builds --rev REV          # this tree's build against git revision REV,
                                                         # built from a temporary worktree

Both builds must report the same stbl_amd_version() (the same ABI). Runs on one GPU in seconds; the
inputs are seeded, random and bf16-valued where the path needs it. Outputs start as NaN (ids as -1),
and a case that either build rejects (a recorded stbl_amd_last_error, or a v2 status other than 0)
counts as a difference, so two rejected calls never compare equal. Prints each differing case and
exits 1 if any output differs.
"""

import ctypes
import os
import shutil
import subprocess
import sys
import tempfile

import torch

from stblarge_amd import _lib, data, ops

P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float


def _p(t):
    return P(t.data_ptr())


def _load(path):
    """A second, independent handle to a build (a copy, so the loader does not return the first one)."""
    tmp = tempfile.mkdtemp(prefix="stbl_cmp_")
    dst = os.path.join(tmp, os.path.basename(path))
    shutil.copy(path, dst)
    lib = ctypes.CDLL(dst)
    for name, (res, args) in _lib.SIGNATURES.items():
        if hasattr(lib, name):
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
    return lib


def _out(shape, dev, dtype=torch.float32):
    """An output buffer filled with a sentinel (NaN, or -1 for integers) before the call."""
    if dtype.is_floating_point:
        return torch.full(shape if isinstance(shape, tuple) else (shape,), float("nan"), dtype=dtype, device=dev)
    return torch.full(shape if isinstance(shape, tuple) else (shape,), -1, dtype=dtype, device=dev)


def _cases(dev, seed):
    """(name, function(lib) -> list of output tensors) for one seed."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    st = None
    cases = []

    def bf(shape, scale=1.0):
        return (torch.randn(shape, device=dev, generator=g) * scale).to(torch.bfloat16)

    # reference ABI GEMVs at the reference's benchmark shapes
    for rows, k in ((2304, 5120), (5120, 2304)):
        w = torch.randint(0, 256, (rows, k // 32 * 17), dtype=torch.uint8, device=dev, generator=g)
        w[:, ::17] = torch.randint(110, 130, (rows, k // 32), dtype=torch.uint8, device=dev, generator=g)
        x = bf(k).float()

        def mx(lib, w=w, x=x, rows=rows, k=k):
            y = _out(rows, dev)
            lib.stbl_gemv_mxfp4(_p(y), _p(w), _p(x), rows, k, st)
            return [y]
        cases.append((f"stbl_gemv_mxfp4 {rows}x{k}", mx))
    # the engine's expert batches (stbl/model.cu:536-539): 12 gate/up matrices, then 6 down
    for rows, k, n in ((2304, 5120, 12), (5120, 2304, 6)):
        ws = [torch.randint(0, 256, (rows, k // 32 * 17), dtype=torch.uint8, device=dev, generator=g) for _ in range(n)]
        for w in ws:
            w[:, ::17] = torch.randint(110, 130, (rows, k // 32), dtype=torch.uint8, device=dev, generator=g)
        xs = [bf(k).float() for _ in range(n)]

        def mxb(lib, ws=ws, xs=xs, rows=rows, k=k, n=n):
            ys = [_out(rows, dev) for _ in range(n)]
            arr = P * n
            lib.stbl_gemv_mxfp4_batch(arr(*[y.data_ptr() for y in ys]), arr(*[w.data_ptr() for w in ws]),
                                      arr(*[x.data_ptr() for x in xs]), n, rows, k, st)
            return ys
        cases.append((f"stbl_gemv_mxfp4_batch {n}x {rows}x{k}", mxb))
    for rows, k in ((32768, 1280), (5120, 8192), (2304, 5120)):
        w = torch.randint(0, 256, (rows, k), dtype=torch.uint8, device=dev, generator=g)
        w[(w & 0x7f) == 0x7f] = 0
        sc = torch.randint(110, 130, ((rows + 31) // 32, k // 32), dtype=torch.uint8, device=dev, generator=g)
        x = bf(k).float()

        def f8(lib, w=w, sc=sc, x=x, rows=rows, k=k):
            y = _out(rows, dev)
            lib.stbl_gemv_fp8(_p(y), _p(w), _p(sc), _p(x), rows, k, seed % 2, st)
            return [y]
        cases.append((f"stbl_gemv_fp8 {rows}x{k}", f8))
    wb = bf((4096, 5120), 0.02)
    xb = bf(2 * 5120).float()

    def b16(lib):
        y, z = _out(4096, dev), _out(4096, dev)
        lib.stbl_gemv_bf16(_p(y), _p(wb), _p(xb), 4096, 5120, 1, 0, st)
        lib.stbl_gemv_bf16(_p(z), _p(wb), _p(xb), 4096, 5120, 0, 2048, st)
        return [y, z]
    cases.append(("stbl_gemv_bf16 4096x5120", b16))
    wf = torch.randn((256, 5120), device=dev, generator=g) * 0.02
    xf = torch.randn(5120, device=dev, generator=g)

    def f32(lib):
        y = _out(256, dev)
        lib.stbl_gemv_f32(_p(y), _p(wf), _p(xf), 256, 5120, 0, st)
        return [y]
    cases.append(("stbl_gemv_f32 256x5120", f32))

    # v2 GEMVs, single and batched, M = 1 and 4
    for fmt, rows, k in ((ops.FP4, 2048, 7168), (ops.FP4, 7168, 2048), (ops.FP8, 2048, 7168)):
        wt = data.weight(rows, k, seed, dev)
        codes, scales = ops.quant_fp4(wt) if fmt == ops.FP4 else ops.quant_fp8_b128(wt)
        for m in (1, 4):
            x = bf((m, k))

            def v2(lib, fmt=fmt, codes=codes, scales=scales, x=x, m=m, rows=rows, k=k):
                y = _out((m, rows), dev)
                fn = lib.stbl_amd_gemv_fp4 if fmt == ops.FP4 else lib.stbl_amd_gemv_fp8
                assert fn(_p(y), _p(codes), _p(scales), _p(x), m, rows, k, 1, st) == 0
                return [y]
            cases.append((f"gemv v2 fmt {fmt} {rows}x{k} m={m}", v2))
    for rows, k in ((7168, 2048), (2048, 7168)):
        codes, scales = ops.quant_fp4(data.weight(rows, k, seed + 1, dev))
        xs = [bf((1, k)) for _ in range(16)]

        def batch(lib, codes=codes, scales=scales, xs=xs, rows=rows, k=k):
            ys = [_out(rows, dev) for _ in range(16)]
            arr = ctypes.c_void_p * 16
            assert lib.stbl_amd_gemv_fp4_batch(arr(*[y.data_ptr() for y in ys]), arr(*[codes.data_ptr()] * 16),
                                               arr(*[scales.data_ptr()] * 16), arr(*[x.data_ptr() for x in xs]),
                                               16, 1, rows, k, 1, st) == 0
            return ys
        cases.append((f"gemv_fp4_batch 16 x {rows}x{k}", batch))

    # expert FFN and MoE (official numerics, the engine's shared expert format)
    dim, inter = 5120, 2304
    experts = [ops.quant_expert(data.weight(inter, dim, 10 * seed + i, dev), data.weight(inter, dim, 10 * seed + i + 1, dev),
                                data.weight(dim, inter, 10 * seed + i + 2, dev), ops.FP4) for i in range(0, 42, 3)]
    shared = ops.quant_expert(data.weight(inter, dim, 3, dev), data.weight(inter, dim, 4, dev),
                              data.weight(dim, inter, 5, dev), ops.FP8_E8M0)
    # picks (j + 2i) % 7 give every expert three or four tokens; the explicit table gives experts of
    # one, two and four tokens, so the step's jobs span every token class (with the FP8 E8M0 shared
    # expert, or with expert 13 as an FP4 shared one)
    mixed = [[0, 1, 2, 3, 4, 5], [0, 1, 7, 8, 9, 10], [0, 11, 12, 6, 2, 3], [0, 7, 11, 12, 8, 9]]
    for name, t, table, sfmt in (("v41 t=1", 1, None, ops.FP8_E8M0), ("v41 t=4", 4, None, ops.FP8_E8M0),
                                 ("v41 t=4 token classes", 4, mixed, ops.FP8_E8M0),
                                 ("fp4 t=4 token classes", 4, mixed, -1)):
        x = bf((t, dim))

        def moe(lib, x=x, t=t, table=table, sfmt=sfmt):
            pick = table or [[(j + 2 * i) % 7 for j in range(6)] for i in range(t)]
            wts = [[0.3, 0.2, 0.15, 0.15, 0.1, 0.1]] * t
            slots = experts + [shared] if sfmt >= 0 else experts
            sh = 14 if sfmt >= 0 else 13
            y = _out((t, dim), dev, torch.bfloat16)
            work = torch.empty(ops.moe_work_bytes(t, 6, dim, inter), dtype=torch.uint8, device=dev)
            arr = (ctypes.c_void_p * len(slots))(*[s.data_ptr() for s in slots])
            pk = (ctypes.c_int * (6 * t))(*[v for row in pick for v in row])
            wt = (ctypes.c_float * (6 * t))(*[v for row in wts for v in row])
            assert lib.stbl_amd_moe_experts(ops.FP4, _p(y), _p(x), t, dim, inter, arr, len(slots), pk, wt, 6, sh,
                                            sfmt, 10.0, 1, 0, _p(work), st) == 0
            return [y]
        cases.append((f"moe_experts {name}", moe))
    logits = torch.randn((4, 256), device=dev, generator=g) * 3

    def route(lib):
        ids = _out((4, 8), dev, torch.int32)
        w = _out((4, 8), dev)
        assert lib.stbl_amd_route(_p(logits), None, 4, 256, 8, 2.5, 1, _p(ids), _p(w), None, st) == 0
        return [ids, w]
    cases.append(("route sqrt-softplus", route))

    # multi-token GEMM
    gc, gs = ops.quant_fp4(data.weight(2048, 7168, seed + 2, dev))
    xg = bf((64, 7168))

    def gemm(lib):
        y = _out((64, 2048), dev)
        work = torch.empty(int(lib.stbl_amd_gemm_work_bytes(64, 2048, 7168)), dtype=torch.uint8, device=dev)
        assert lib.stbl_amd_gemm(ops.FP4, _p(y), _p(gc), _p(gs), _p(xg), 64, 2048, 7168, 32, 1, _p(work), st) == 0
        return [y]
    cases.append(("gemm fp4 m=64", gemm))
    return cases


def _run(fn, lib):
    """The case's outputs, or None when the build rejected it (a recorded failure or a non-zero v2
    status, which the cases assert)."""
    lib.stbl_amd_last_error(None, 0)  # clear
    try:
        outs = fn(lib)
    except AssertionError:
        return None
    torch.cuda.synchronize()
    return None if lib.stbl_amd_last_error(None, 0) else outs


def compare(new, old, seeds=3):
    """Runs every case on both builds (paths of built libraries, or loaded handles); returns the list
    of (case, differing bytes or "rejected by ...")."""
    new = _load(new) if isinstance(new, str) else new
    old = _load(old) if isinstance(old, str) else old
    if new.stbl_amd_version() != old.stbl_amd_version():
        raise SystemExit(f"ABI versions differ: {new.stbl_amd_version()} vs {old.stbl_amd_version()}")
    dev = torch.device("cuda", torch.cuda.current_device())
    bad = []
    for seed in range(seeds):
        for name, fn in _cases(dev, seed):
            a, b = _run(fn, new), _run(fn, old)
            if a is None or b is None:
                who = " and ".join(w for w, r in (("the new build", a), ("the old build", b)) if r is None)
                bad.append((f"{name} seed {seed}", f"rejected by {who}"))
                print(f"{name} seed {seed}: rejected by {who}", flush=True)
                continue
            d = sum(int((x.view(torch.uint8) != y.view(torch.uint8)).sum()) for x, y in zip(a, b))
            if d:
                bad.append((f"{name} seed {seed}", d))
                print(f"{name} seed {seed}: {d} bytes differ", flush=True)
    return bad


def build_revision(rev):
    """Builds libstbl_amd.so of git revision rev in a temporary worktree; returns its path."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    wt = tempfile.mkdtemp(prefix="stbl_rev_")
    subprocess.run(["git", "-C", root, "worktree", "add", "--detach", wt, rev], check=True, capture_output=True)
    try:
        subprocess.run([sys.executable, "-m", "stblarge_amd.build"], cwd=wt, check=True)
        out = os.path.join(tempfile.mkdtemp(prefix="stbl_revlib_"), "libstbl_amd.so")
        shutil.copy(os.path.join(wt, "stblarge_amd", "libstbl_amd.so"), out)
        return out
    finally:
        subprocess.run(["git", "-C", root, "worktree", "remove", "--force", wt], capture_output=True)


def main(argv):
    if len(argv) == 2 and argv[0] == "--rev":
        new, old = _lib.LIB_PATH, build_revision(argv[1])
    elif len(argv) == 2:
        new, old = argv
    else:
        print(__doc__)
        return 2
    _lib.load()  # torch's HIP runtime first
    bad = compare(new, old)
    print("bitwise identical" if not bad else f"{len(bad)} cases differ")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
