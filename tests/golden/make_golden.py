"""Writes tests/golden/golden.json: known-answer vectors for the CPU oracle.

The expected values here are computed WITHOUT the oracle: by exact rational arithmetic
(fractions.Fraction), brute-force nearest-grid-point search, and numpy float32 for the single fp32
roundings the reference's formulas perform. They restate the reference's own inline known-answer
tests (ref/test_kernel.py:12-57: pow2_ceil, e2m1 ties-to-even, act_quant closed form, fp4 round
trip, fp8_gemm vs brute force) plus the closed forms the path depends on (tools/convert_official.py:
40-48 e4m3 table, :187-201 GGUF MXFP4 repack). No reference code is imported or run.

Run: python tests/golden/make_golden.py   (seconds; deterministic)
"""

import base64
import json
import math
import os
from fractions import Fraction

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.json")


class Lcg:
    """Small deterministic generator so the fixture does not depend on any library's RNG."""

    def __init__(self, seed):
        self.s = seed & 0xFFFFFFFFFFFFFFFF

    def next(self):
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
        return self.s >> 11

    def uniform(self):  # [0, 1)
        return self.next() / float(1 << 53)

    def normal(self):
        u1, u2 = max(self.uniform(), 1e-12), self.uniform()
        return math.sqrt(-2 * math.log(u1)) * math.cos(2 * math.pi * u2)


def f32(v):
    return float(np.float32(v))


def b64(values, dtype):
    """Little-endian raw bytes of a numeric list, base64: keeps the large arrays compact."""
    return base64.b64encode(np.asarray(values, dtype=dtype).astype(np.dtype(dtype).newbyteorder("<")).tobytes()).decode()


def bf16(v):
    """Nearest-even bf16 value of a float (via exact fp32 first)."""
    u = int(np.array([v], np.float32).view(np.uint32)[0])
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return float(np.array([u << 16], np.uint32).view(np.float32)[0])


# ---- e4m3 -------------------------------------------------------------------------------------------

def e4m3_value(c):
    """tools/convert_official.py:40-48 in exact arithmetic; None for the NaN codes."""
    e, m = (c >> 3) & 15, c & 7
    if e == 15 and m == 7:
        return None
    v = Fraction(m, 8) * Fraction(1, 64) if e == 0 else (1 + Fraction(m, 8)) * Fraction(2) ** (e - 7)
    return -v if c & 0x80 else v


POS_GRID = [(c, float(e4m3_value(c))) for c in range(0x7F)]  # codes 0x00..0x7e, increasing values


def e4m3_round(x):
    """Nearest e4m3 code to x (a Fraction or float within +-448), ties to the even code; keeps sign.
    Brute force over all 127 non-negative finite codes; the distances are exact in double because
    every operand is an fp32 value within [2^-30, 448]."""
    neg = math.copysign(1.0, float(x)) < 0
    a = abs(float(x))
    best = min(POS_GRID, key=lambda cv: (abs(cv[1] - a), cv[0] & 1))
    return best[0] | (0x80 if neg else 0)


# ---- e2m1 -------------------------------------------------------------------------------------------

FP4_GRID = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]  # ref/kernel.py:14-16


def fp4_round(v):
    """ref/test_kernel.py:21 brute force: nearest grid value, ties to the even grid index."""
    best = min(FP4_GRID, key=lambda g: (abs(abs(Fraction(v)) - Fraction(g)), FP4_GRID.index(g) % 2))
    return math.copysign(best, v)


def fp4_code(q):
    return FP4_GRID.index(abs(q)) | (8 if math.copysign(1.0, q) < 0 else 0)


def pow2_ceil_exact(t):
    """Smallest power of two >= t (t > 0), exactly."""
    t = Fraction(t)
    e = math.floor(math.log2(float(t))) - 2
    while Fraction(2) ** e < t:
        e += 1
    while e > -200 and Fraction(2) ** (e - 1) >= t:
        e -= 1
    return float(Fraction(2) ** e)


def main():
    g = {}
    # e4m3: every code (NaN codes as null)
    g["e4m3_table"] = [None if e4m3_value(c) is None else float(e4m3_value(c)).hex() for c in range(256)]
    # e4m3 rounding: every midpoint between neighbours, a hair either side, and random points
    cases = []
    vals = [v for _, v in POS_GRID]
    for lo, hi in zip(vals, vals[1:]):
        mid = (lo + hi) / 2
        for x in (float(mid), float(np.nextafter(np.float32(mid), np.float32(0))),
                  float(np.nextafter(np.float32(mid), np.float32(1000)))):
            cases.append(x)
    rng = Lcg(1)
    for _ in range(400):
        cases.append(f32(rng.uniform() * 448.0 * (2.0 ** -int(rng.uniform() * 14))))
    cases += [0.0, 2.0 ** -10, 2.0 ** -10 + 2.0 ** -30, 3 * 2.0 ** -10, 448.0, 464.0 - 2.0 ** -10]
    cases = [f32(c) for c in cases] + [-f32(c) for c in cases[:100]]
    g["e4m3_round"] = [[x.hex(), e4m3_round(min(max(x, -448.0), 448.0))] for x in cases]
    # pow2_ceil KAT of ref/test_kernel.py:13 (float32 inputs)
    kat = [1e-6, 0.25, 0.3, 1.0, 1.0000001, 3.0, 448.0, 1000.0]
    g["pow2_ceil"] = [[f32(v).hex(), pow2_ceil_exact(f32(v)).hex()] for v in kat]
    # e2m1 ties-to-even over the ref/test_kernel.py:20 sweep (i/400 - 6) plus its tie points
    sweep = [f32(Fraction(i, 400) - 6) for i in range(4801)] + [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]
    g["fp4_round"] = {"x": b64(sweep, np.float32), "want": b64([fp4_round(v) for v in sweep], np.float32)}
    # act_quant(x, 32, ue8m0) on x = bf16(randn * logspace(-3, 3, 128)) [3][128] (ref/test_kernel.py:26-35)
    rng = Lcg(2)
    x = [[bf16(rng.normal() * 10 ** (-3 + 6 * j / 127)) for j in range(128)] for _ in range(3)]
    inv448 = np.float32(1.0 / 448.0)
    scales, codes, deq = [], [], []
    for row in x:
        for b in range(4):
            blk = row[b * 32:(b + 1) * 32]
            amax = max(max(abs(v) for v in blk), f32(1e-4))
            t = float(np.float32(amax) * inv448)
            s = pow2_ceil_exact(t)
            scales.append(s)
            for v in blk:
                q = min(max(Fraction(v) / Fraction(s), -448), 448)
                c = e4m3_round(q if v != 0 or math.copysign(1, v) > 0 else -0.0)
                codes.append(c)
                deq.append(bf16(float(e4m3_value(c) * Fraction(s))))
    g["act_quant"] = {"x": [v.hex() for r in x for v in r], "rows": 3, "n": 128, "block": 32,
                      "scales": [s.hex() for s in scales], "codes": codes, "deq": [d.hex() for d in deq]}
    # fp4 weight quantization (fp4_act_quant e8m0 path, ref/kernel.py:55-72): rows of 64 values
    rng = Lcg(3)
    w = [[f32(rng.normal() * 0.02 * (10.0 if (j // 32) == 1 else 1.0)) for j in range(64)] for _ in range(4)]
    w[0][5] = -0.0
    w[1][0:32] = [f32(-1e-9)] * 32          # tiny negative block: scale floor, codes -0 (8)
    w[2][40] = f32(2.0 ** -126 * 3)
    inv6 = np.float32(1.0 / 6.0)
    fcodes, fscales = [], []
    for row in w:
        packed = []
        for b in range(2):
            blk = row[b * 32:(b + 1) * 32]
            amax = max(max(abs(v) for v in blk), f32(6 * 2.0 ** -126))
            s = pow2_ceil_exact(float(np.float32(amax) * inv6))
            fscales.append(int(np.array([s], np.float32).view(np.uint32)[0] >> 23) & 0xFF)
            cs = []
            for v in blk:
                q = float(min(max(Fraction(v) / Fraction(s), -6), 6))
                r = fp4_round(q if q != 0 else math.copysign(0.0, v))
                if r == 0:
                    r = math.copysign(0.0, v)
                cs.append(fp4_code(r))
            packed += [cs[i] | (cs[i + 1] << 4) for i in range(0, 32, 2)]
        fcodes.append(packed)
    g["quant_fp4"] = {"w": [v.hex() for r in w for v in r], "rows": 4, "k": 64,
                      "codes": [c for r in fcodes for c in r], "scales": fscales}
    # fp8 128x128 quantization (s = amax/448 fp32 division), with partial edge blocks: [130][260]
    rng = Lcg(4)
    R, K = 130, 260
    w8 = np.array([[rng.normal() * 0.02 for _ in range(K)] for _ in range(R)], np.float32)
    w8[129, 259] = 0.5  # a lone outlier in the corner (partial) block
    nb, kb = 2, 3
    s8 = np.zeros((nb, kb), np.float32)
    c8 = np.zeros((R, K), np.uint8)
    for bi in range(nb):
        for bj in range(kb):
            blk = w8[bi * 128:(bi + 1) * 128, bj * 128:(bj + 1) * 128]
            amax = np.float32(max(float(np.abs(blk).max()), f32(1e-4)))
            s = np.float32(amax / np.float32(448.0))
            s8[bi, bj] = s
            for r in range(blk.shape[0]):
                for c in range(blk.shape[1]):
                    q = float(np.float32(blk[r, c] / s))
                    c8[bi * 128 + r, bj * 128 + c] = e4m3_round(min(max(q, -448.0), 448.0))
    g["quant_fp8_b128"] = {"w": b64(w8.ravel(), np.float32), "rows": R, "k": K,
                           "codes": b64(c8.ravel(), np.uint8), "scales": b64(s8.ravel(), np.float32)}
    # FP4 GEMV, exact: y[m][n] = sum_k x[m][k] * table[code] * 2^(s-127), small non-square case
    rng = Lcg(5)
    n, k, m = 5, 96, 2
    gc = [[rng.next() & 0xFF for _ in range(k // 2)] for _ in range(n)]
    gs = [[118 + rng.next() % 12 for _ in range(k // 32)] for _ in range(n)]
    gx = [[bf16(rng.normal()) for _ in range(k)] for _ in range(m)]
    tab = [Fraction(v) for v in FP4_GRID] + [-Fraction(v) for v in FP4_GRID]
    gy = []
    for i in range(m):
        for j in range(n):
            acc = Fraction(0)
            for c in range(k):
                byte = gc[j][c // 2]
                nib = (byte >> 4) if c & 1 else (byte & 15)
                acc += Fraction(gx[i][c]) * tab[nib] * Fraction(2) ** (gs[j][c // 32] - 127)
            gy.append(float(acc).hex())
    g["gemv_fp4"] = {"n": n, "k": k, "m": m, "codes": [c for r in gc for c in r], "scales": [s for r in gs for s in r],
                     "x": [v.hex() for r in gx for v in r], "y": gy}
    # GGUF 17-byte repack of the same codes (tools/convert_official.py:187-201)
    blocks = []
    for j in range(n):
        for b in range(k // 32):
            cb = gc[j][b * 16:(b + 1) * 16]
            vals = []
            for byte in cb:
                vals += [byte & 15, byte >> 4]
            blocks += [gs[j][b]] + [vals[i] | (vals[16 + i] << 4) for i in range(16)]
    g["gguf17"] = blocks
    # FP8 GEMV with 128x128 fp32 scales, exact, on the quant_fp8_b128 matrix (codes + scales above)
    rng = Lcg(6)
    x8 = [bf16(rng.normal()) for _ in range(K)]
    y8 = []
    for r in range(R):
        acc = Fraction(0)
        for c in range(K):
            acc += Fraction(x8[c]) * (Fraction(float(np.float32(float(e4m3_value(int(c8[r, c]))) * s8[r // 128, c // 128]))))
        y8.append(float(acc).hex())
    g["gemv_fp8_b128"] = {"x": b64(x8, np.float32), "y": y8}
    # SwiGLU epilogue (stbl/kernels.cu:450-459), numpy float32 exp as the library routine
    rng = Lcg(7)
    sw = []
    for i in range(64):
        gv, uv = f32(rng.normal() * 4), f32(rng.normal() * 4)
        wv, lim = f32(0.37 if i % 2 else 1.0), (10.0 if i % 3 == 0 else 0.0)
        gg, uu = np.float32(gv), np.float32(uv)
        if lim > 0:
            uu = np.float32(min(max(uu, -lim), lim))
            gg = np.float32(min(gg, lim))
        out = np.float32(np.float32(gg / (np.float32(1) + np.exp(-gg))) * uu) * np.float32(wv)
        sw.append([gv.hex(), uv.hex(), wv.hex(), lim, bf16(float(out)).hex()])
    g["swiglu"] = sw
    # Router: sigmoid, top-8 with ties to the lower id, renormalised (stbl/model.cu:444-451)
    rng = Lcg(8)
    logits = [[f32(rng.normal()) for _ in range(32)] for _ in range(3)]
    logits[1][7] = logits[1][3]                     # an exact tie
    logits[2][0:32] = [f32(0.5)] * 32               # everything tied: ids 0..7
    ids_all, w_all = [], []
    for row in logits:
        sc = [float(np.float32(1) / (np.float32(1) + np.exp(-np.float32(v)))) for v in row]
        order = sorted(range(32), key=lambda j: (-sc[j], j))[:8]
        tot = np.float32(0)
        for j in order:
            tot = np.float32(tot + np.float32(sc[j]))
        ws = [float(np.float32(np.float32(sc[j]) / np.float32(tot + np.float32(1e-20)))) for j in order]
        ids_all.append(order)
        w_all.append([v.hex() for v in ws])
    g["route"] = {"logits": [v.hex() for r in logits for v in r], "t": 3, "e": 32, "topk": 8,
                  "ids": ids_all, "weights": w_all}
    with open(OUT, "w") as f:
        json.dump(g, f, separators=(",", ":"))
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
