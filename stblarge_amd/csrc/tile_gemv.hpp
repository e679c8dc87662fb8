// MFMA tile engine for quantized GEMV / skinny GEMM: y[t][r] = sum_k x[t][k] * Wdeq[r][k], t < M <= 16.
//
// One wave computes a 16 x 16 fp32 tile D = A * B with v_mfma_f32_16x16x32_bf16, where the 16 rows of
// A are "virtual rows" and the 16 columns of B are "virtual columns":
//   * K is cut into S segments of L elements (S a power of two, S * M <= 16) and a tile holds
//     R = 16 / S real rows; virtual row v = s * R + r is real row r restricted to segment s;
//   * virtual column c = s * M + t holds token t's activation restricted to segment s;
//   * so D[s R + r][s M + t] is segment s's share of y[t][r], and the S diagonal blocks are summed in
//     the epilogue. Off-diagonal entries are unused.
// This lets one MFMA tile serve 1..16 tokens and 1..16 rows without any cross-lane reduction: the
// contraction over K happens inside the MFMA, and the segments are added once at the end.
//
// A round is one 128-bit weight load per lane. With the gfx950 operand layout (lane l holds
// A[l % 16][8 (l / 16) .. +8], B[8 (l / 16) .. +8][l % 16], D[4 (l / 16) .. +4][l % 16]) lane group
// g = l / 16 loads a CH-element chunk of its virtual row at k = s L + round * RK + g * CH, and the
// chunk feeds NMF consecutive MFMAs, 8 elements each; the B lanes load the matching 8-element pieces
// of x. The k labelling inside an MFMA is arbitrary as long as A and B agree, which they do.
//
// Formats:
//   FP4 e2m1, OCP packing, E8M0 scale per 32: the chunk is 32 elements (16 bytes) with one scale;
//     v_cvt_scalef32_pk_bf16_fp4 converts 2 codes to bf16 and multiplies by the scale exactly (a
//     power of two), so A holds the exact dequantized values (ref/kernel.py:98-101).
//   FP8 e4m3 with fp32 scales per 128x128 block: the chunk is 16 elements, converted exactly to bf16;
//     each round lies inside one 128-column block, so the round's product is scaled by its block
//     scale in fp32 and added to the accumulator (the scale is not a power of two, so it cannot be
//     folded into the bf16 operand without rounding).
// Products of a bf16 activation and an exactly converted weight are exact in fp32; only the order of
// the fp32 additions differs from ref/kernel.py:91,102.
#pragma once

#include "common.hpp"

namespace stbl {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

enum class Fmt { FP4, FP8 };

template <Fmt F>
struct FmtTraits;
template <>
struct FmtTraits<Fmt::FP4> {
    static constexpr int CH = 32;   // elements per lane chunk (16 bytes)
    static constexpr int RK = 128;  // k per virtual row per round
    static constexpr int NMF = 4;   // MFMAs per round
};
template <>
struct FmtTraits<Fmt::FP8> {
    static constexpr int CH = 16;
    static constexpr int RK = 64;
    static constexpr int NMF = 2;
};

// A quantized weight matrix in device memory.
struct QMat {
    const uint8_t *codes;  // FP4: [rows][k/2]; FP8: [rows][k]
    const void *scales;    // FP4: E8M0 bytes [rows][k/32]; FP8: fp32 [ceil(rows/128)][ceil(k/128)]
    int rows, k;
};

// How one launch cuts a [rows x k] matrix into tiles (see the header comment).
struct TileShape {
    int S, R;     // segments per tile, real rows per tile (R * S == 16)
    int L;        // segment length (elements), a multiple of RK
    int rounds;   // rounds per segment, L / RK
    int W;        // waves per workgroup, each taking NRw consecutive rounds of every segment
    int NRw;      // rounds per wave
};

template <Fmt F>
inline TileShape make_shape(int S, int W, int k) {
    constexpr int RK = FmtTraits<F>::RK;
    TileShape t;
    t.S = S;
    t.R = 16 / S;
    t.rounds = (k + S * RK - 1) / (S * RK);
    t.L = t.rounds * RK;
    t.W = W < t.rounds ? W : t.rounds;
    t.NRw = (t.rounds + t.W - 1) / t.W;
    t.W = (t.rounds + t.NRw - 1) / t.NRw;
    return t;
}

// Convert one lane chunk into the A operands of its NMF MFMAs.
template <Fmt F>
__device__ __forceinline__ void chunk_to_bf16(bf16x8 (&a)[FmtTraits<F>::NMF], const u32x4 w, float scale) {
    if constexpr (F == Fmt::FP4) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j], scale, 0);
            const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j], scale, 1);
            const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j], scale, 2);
            const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[j], scale, 3);
            a[j] = bf16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
        }
    } else {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[2 * j], 1.0f, false);
            const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[2 * j], 1.0f, true);
            const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[2 * j + 1], 1.0f, false);
            const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[2 * j + 1], 1.0f, true);
            a[j] = bf16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
        }
    }
}

// Accumulates this wave's share (rounds [wave * NRw, (wave+1) * NRw) of every segment) of the tile
// whose first real row is row0 into acc (the lane's 4 D entries). x is bf16 [M][ldx]. All loads of
// the wave are issued before the first MFMA, so NR rounds of weights are in flight per lane.
template <Fmt F, int NR>
__device__ __forceinline__ void tile_accumulate(f32x4 &acc, const QMat &W, const uint16_t *__restrict__ x, int M,
                                                int ldx, int row0, const TileShape &ts, int wave) {
    using T = FmtTraits<F>;
    const int lane = threadIdx.x & 63, v = lane & 15, g = lane >> 4;
    const int K = W.k;
    // A side: virtual row v = (segment sA, row rA)
    const int sA = v / ts.R, rowA = row0 + v % ts.R;
    const bool rowok = rowA < W.rows;
    // B side: virtual column v = (segment sB, token tB)
    const bool colok = v < ts.S * M;
    const int sB = colok ? v / M : 0, tB = colok ? v % M : 0;
    const int r0 = wave * ts.NRw;

    u32x4 wv[NR];
    float sc[NR];
    u32x4 xv[NR][T::NMF];
#pragma unroll
    for (int i = 0; i < NR; i++) {
        const bool live = i < ts.NRw && r0 + i < ts.rounds;
        const int kA = sA * ts.L + (r0 + i) * T::RK + g * T::CH;
        const bool okA = live && rowok && kA < K;
        if constexpr (F == Fmt::FP4) {
            wv[i] = okA ? *(const u32x4 *)(W.codes + (size_t)rowA * (K >> 1) + (kA >> 1)) : u32x4{0, 0, 0, 0};
            sc[i] = okA ? e8m0_to_f32(((const uint8_t *)W.scales)[(size_t)rowA * (K >> 5) + (kA >> 5)]) : 1.0f;
        } else {
            wv[i] = okA ? *(const u32x4 *)(W.codes + (size_t)rowA * K + kA) : u32x4{0, 0, 0, 0};
        }
        const int kB = sB * ts.L + (r0 + i) * T::RK + g * T::CH;
        const bool okB = live && colok && kB < K;
        const u32x4 *xp = (const u32x4 *)(x + (size_t)tB * ldx + kB);
#pragma unroll
        for (int j = 0; j < T::NMF; j++) xv[i][j] = okB ? xp[j] : u32x4{0, 0, 0, 0};
    }
    if constexpr (F == Fmt::FP8) {
        // block scale of each of the lane's 4 D rows (virtual rows 4 g + e), per round
        const int KB = (K + 127) >> 7;
        const float *s8 = (const float *)W.scales + (size_t)(row0 >> 7) * KB;
#pragma unroll
        for (int i = 0; i < NR; i++) sc[i] = 0.f;  // unused for FP8 (kept for register symmetry)
        float bs[NR][4];
#pragma unroll
        for (int i = 0; i < NR; i++) {
            const bool live = i < ts.NRw && r0 + i < ts.rounds;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int s = (4 * g + e) / ts.R;
                const int kb = (s * ts.L + (r0 + i) * T::RK) >> 7;
                bs[i][e] = live && kb < KB ? s8[kb] : 0.f;
            }
        }
#pragma unroll
        for (int i = 0; i < NR; i++) {
            if (i < ts.NRw) {
                bf16x8 a[T::NMF];
                chunk_to_bf16<F>(a, wv[i], 1.0f);
                f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < T::NMF; j++)
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j], __builtin_bit_cast(bf16x8, xv[i][j]), d, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; e++) acc[e] = fmaf(bs[i][e], d[e], acc[e]);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < NR; i++) {
            if (i < ts.NRw) {
                bf16x8 a[T::NMF];
                chunk_to_bf16<F>(a, wv[i], sc[i]);
#pragma unroll
                for (int j = 0; j < T::NMF; j++)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j], __builtin_bit_cast(bf16x8, xv[i][j]), acc, 0, 0, 0);
            }
        }
    }
}

// Sums the S diagonal blocks of the tile over the W waves of the workgroup. red holds W * 64 f32x4.
// Returns, for thread q < R * M (t = q / R, r = q % R), the value of y[t][row0 + r] in *out.
__device__ __forceinline__ bool tile_reduce(f32x4 (*red)[64], const f32x4 &acc, const TileShape &ts, int M,
                                            float *out, int *t_out, int *r_out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    red[wave][lane] = acc;
    __syncthreads();
    const int q = threadIdx.x;
    if (q >= ts.R * M) return false;
    const int t = q / ts.R, r = q % ts.R;
    float s = 0.f;
    for (int w = 0; w < ts.W; w++)
        for (int seg = 0; seg < ts.S; seg++) {
            const int vr = seg * ts.R + r, vc = seg * M + t;
            s += red[w][(vr >> 2) * 16 + vc][vr & 3];
        }
    *out = s;
    *t_out = t;
    *r_out = r;
    return true;
}

}  // namespace stbl
