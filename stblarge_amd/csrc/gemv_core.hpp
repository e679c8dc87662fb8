// Device building blocks shared by the GEMV, expert-FFN and MoE kernels: weight formats, lane-chunk
// loads of x and weights, exact chunk dot products, and the on-the-fly activation quantization.
//
// Every kernel built from these uses the same work split: lane l of wave w owns one fixed K chunk
// c = 64 w + l of CH elements (16 bytes of FP4 codes, one 17-byte GGUF block, or 16 bytes of FP8
// codes), so a wave-wide load of one row reads a contiguous kilobyte, and per-row partial sums are
// reduced over the lanes with DPP (common.hpp dpp_sum) and over the waves through LDS.
#pragma once

#include "common.hpp"

namespace stbl {

constexpr int kMaxWaves = 8;  // K <= 512 chunks: 16384 FP4 / 8192 FP8 elements
// A tile's OCP FP4 scale block is staged through LDS for tiles of at most kMaxStageRows rows (each
// row at most kMaxWaves * 64 bytes; the block takes R * kMaxWaves * 64 / 16 units of 16 bytes, plus
// one for a block that starts mid-unit and one for its end).
constexpr int kMaxStageRows = 16;
constexpr int kMxBatch = 16;  // matrices per launch of the reference ABI's batch (stbl/kernels.h:18)
constexpr int kMaxJobs = 64;  // matrices per launch of the v2 batches (the MoE step's gate/up launches hold up to 66)

enum class WFmt { FP4_OCP, FP4_GGUF, FP8_B128, FP8_E8M0 };

template <WFmt F>
struct WTraits {
    static constexpr bool fp4 = F == WFmt::FP4_OCP || F == WFmt::FP4_GGUF;
    static constexpr int CH = fp4 ? 32 : 16;  // elements per lane chunk
};

// One matrix of a launch: weights, scales, activations, output.
struct GemvJob {
    const uint8_t *w;
    const void *s;
    const void *x;
    void *y;
};
struct GemvJobs {
    GemvJob j[kMaxJobs];
};

enum OutMode { OUT_BF16 = 0, OUT_F32 = 1, OUT_F32_ROUNDED = 2 };

// A GGUF block c of a row sits at byte 17 c, so it is only byte aligned: read the five dwords that
// cover it from the enclosing 4-byte boundary (each dword starts inside the buffer, and a 4-byte
// aligned dword never crosses a page) and realign with v_alignbyte. The loads and the realignment
// are separate steps so that a kernel can issue every row's loads before it waits for the first.
struct GgufRaw {
    uint32_t v[5];
    uint32_t sh;  // the block's byte offset in its first dword
};

__device__ __forceinline__ void load_gguf_raw(const uint8_t *blk, GgufRaw &raw) {
    // pointer arithmetic, not an integer round trip: the loads stay global loads (as flat loads they
    // cost 2-7% on the reference ABI's GEMVs)
    raw.sh = (uint32_t)((uintptr_t)blk & 3);
    const uint32_t *d = (const uint32_t *)(blk - raw.sh);
#pragma unroll
    for (int i = 0; i < 5; i++) raw.v[i] = d[i];
}

// The same for block `off` bytes into a row at `base` (base wave-uniform, off per lane): the loads
// take a scalar base and a 32-bit lane offset, with no 64-bit address arithmetic per lane (whose
// register reuse once made the compiler wait for earlier loads before issuing the next row's).
__device__ __forceinline__ void load_gguf_raw_at(const uint8_t *base, uint32_t off, GgufRaw &raw) {
    const uint32_t a = (uint32_t)(uintptr_t)base & 3u, o = a + off;
    raw.sh = o & 3u;
    const uint32_t *d = (const uint32_t *)(base - a + (o & ~3u));
#pragma unroll
    for (int i = 0; i < 5; i++) raw.v[i] = d[i];
}

__device__ __forceinline__ void realign_gguf(const GgufRaw &raw, uint32_t &scale, u32x4 &codes) {
    scale = (raw.v[0] >> (8 * raw.sh)) & 0xffu;
    const uint32_t off = raw.sh + 1;  // first code byte, 1..4 bytes past the first dword
#pragma unroll
    for (int j = 0; j < 4; j++) codes[j] = off == 4 ? raw.v[j + 1] : __builtin_amdgcn_alignbyte(raw.v[j + 1], raw.v[j], off);
}

__device__ __forceinline__ void load_gguf_block(const uint8_t *blk, uint32_t &scale, u32x4 &codes) {
    GgufRaw raw;
    load_gguf_raw(blk, raw);
    realign_gguf(raw, scale, codes);
}

// x chunk of CH elements for M tokens, widened to fp32. x is bf16 or fp32 [M][k].
template <bool XF32, int M, int CH>
__device__ __forceinline__ void load_x(float (&xf)[M][CH], const void *x, int k, int k0) {
#pragma unroll
    for (int t = 0; t < M; t++) {
        if constexpr (XF32) {
            const f32x4 *p = (const f32x4 *)((const float *)x + (size_t)t * k + k0);
#pragma unroll
            for (int q = 0; q < CH / 4; q++) {
                const f32x4 v = p[q];
                xf[t][4 * q] = v.x, xf[t][4 * q + 1] = v.y, xf[t][4 * q + 2] = v.z, xf[t][4 * q + 3] = v.w;
            }
        } else {
            const u32x4 *p = (const u32x4 *)((const uint16_t *)x + (size_t)t * k + k0);
#pragma unroll
            for (int q = 0; q < CH / 8; q++) {
                const u32x4 v = p[q];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    xf[t][8 * q + 2 * j] = bf16_lo(v[j]);
                    xf[t][8 * q + 2 * j + 1] = bf16_hi(v[j]);
                }
            }
        }
    }
}

// sum over the chunk of x * weight for each token; FP4 weights are converted times `cs` (their E8M0
// scale as e8m0_cvt_scale, or 1), FP8 weights unscaled.
template <WFmt F, int M, int CH>
__device__ __forceinline__ void chunk_dot(float (&s)[M], const u32x4 w, const float (&xf)[M][CH], float cs = 1.0f) {
#pragma unroll
    for (int t = 0; t < M; t++) s[t] = 0.f;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        if constexpr (WTraits<F>::fp4) {
            const f32x2 a = e2m1x2<0>(w[d], cs), b = e2m1x2<1>(w[d], cs), c = e2m1x2<2>(w[d], cs), e = e2m1x2<3>(w[d], cs);
#pragma unroll
            for (int t = 0; t < M; t++) {
                if constexpr (F == WFmt::FP4_OCP) {  // byte b: elements 2b, 2b+1
                    const float *xv = &xf[t][8 * d];
                    s[t] = fmaf(xv[0], a.x, s[t]);
                    s[t] = fmaf(xv[1], a.y, s[t]);
                    s[t] = fmaf(xv[2], b.x, s[t]);
                    s[t] = fmaf(xv[3], b.y, s[t]);
                    s[t] = fmaf(xv[4], c.x, s[t]);
                    s[t] = fmaf(xv[5], c.y, s[t]);
                    s[t] = fmaf(xv[6], e.x, s[t]);
                    s[t] = fmaf(xv[7], e.y, s[t]);
                } else {  // GGUF byte b: elements b, 16 + b
                    const float *lo = &xf[t][4 * d], *hi = &xf[t][16 + 4 * d];
                    s[t] = fmaf(lo[0], a.x, s[t]);
                    s[t] = fmaf(hi[0], a.y, s[t]);
                    s[t] = fmaf(lo[1], b.x, s[t]);
                    s[t] = fmaf(hi[1], b.y, s[t]);
                    s[t] = fmaf(lo[2], c.x, s[t]);
                    s[t] = fmaf(hi[2], c.y, s[t]);
                    s[t] = fmaf(lo[3], e.x, s[t]);
                    s[t] = fmaf(hi[3], e.y, s[t]);
                }
            }
        } else {
            const f32x2 a = e4m3x2(w[d], false), b = e4m3x2(w[d], true);
#pragma unroll
            for (int t = 0; t < M; t++) {
                const float *xv = &xf[t][4 * d];
                s[t] = fmaf(xv[0], a.x, s[t]);
                s[t] = fmaf(xv[1], a.y, s[t]);
                s[t] = fmaf(xv[2], b.x, s[t]);
                s[t] = fmaf(xv[3], b.y, s[t]);
            }
        }
    }
}

// ---- packed-bf16 path (v2 formats): weights converted to bf16 pairs, v_dot2_f32_bf16 ---------------
//
// With bf16 activations the lane keeps its x chunk as packed bf16 words (word i = elements 2i, 2i+1)
// and each pair of weights is converted straight to a bf16 pair (exactly: e2m1 and e4m3 values are
// bf16 values) and multiplied into the sum by one v_dot2_f32_bf16: per 32 FP4 elements 16
// conversions + 16 dot2 instead of 16 conversions + 32 FMAs, which is what keeps a CU ahead of its
// share of HBM bandwidth. The dot2 products are exact; its internal sum can differ from an IEEE fp32
// addition in the last bits.

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <int M, int CH>
__device__ __forceinline__ void load_x_packed(uint32_t (&xw)[M][CH / 2], const uint16_t *x, int k, int k0) {
#pragma unroll
    for (int t = 0; t < M; t++) {
        const u32x4 *p = (const u32x4 *)(x + (size_t)t * k + k0);
#pragma unroll
        for (int q = 0; q < CH / 8; q++) {
            const u32x4 v = p[q];
#pragma unroll
            for (int j = 0; j < 4; j++) xw[t][4 * q + j] = v[j];
        }
    }
}

// In-register act_quant(x, 32, "ue8m0", inplace=True) of the lane's chunk of packed bf16 words
// (word i = elements 2i, 2i + 1; ref/kernel.py:35-45, the reference engine's stbl_act_quant_fp8,
// stbl/kernels.cu:54-63): per 32 values s = 2^ceil(log2(max(amax, 1e-4) / 448)), x = bf16(e4m3(
// clamp(x / s, +-448)) * s). A 16-element chunk shares its 32-block with the neighbouring lane
// (lanes 2b and 2b+1), whose amax comes over by DPP. 1/s is a power of two too (s lies in [2^-22,
// 2^120]), so x * inv is x / s exactly; v_cvt_pk_fp8_f32 rounds to nearest even like the
// reference's cast (it equals the software encoder f32_to_e4m3 on every bf16 input, and x / s of a
// bf16 x is a bf16 value). bf16(e4m3(q) * s) of each pair is one scaled conversion
// (v_cvt_scalef32_pk_bf16_fp8 multiplies by the power of two whose exponent field its scale operand
// carries: s itself; e4m3 * s is a bf16 value, so the product is exact), so the words are rebuilt
// without widening, multiplying and repacking.
template <int M, int CH>
__device__ __forceinline__ void act_quant_packed(uint32_t (&xw)[M][CH / 2]) {
    static_assert(CH == 32 || CH == 16, "chunk must be one or half an act_quant block");
#pragma unroll
    for (int t = 0; t < M; t++) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < CH / 2; i++) a = fmaxf(fmaxf(a, fabsf(bf16_lo(xw[t][i]))), fabsf(bf16_hi(xw[t][i])));
        if constexpr (CH == 16)
            a = fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0xB1, 0xF, 0xF, false)));
        const float s = pow2_ceil(fmaxf(a, 1e-4f) * (1.0f / 448.0f));
        const float inv = __uint_as_float((254u - ((__float_as_uint(s) >> 23) & 0xffu)) << 23);
#pragma unroll
        for (int i = 0; i < CH / 2; i += 2) {
            const float q0 = fminf(fmaxf(bf16_lo(xw[t][i]) * inv, -448.f), 448.f);
            const float q1 = fminf(fmaxf(bf16_hi(xw[t][i]) * inv, -448.f), 448.f);
            const float q2 = fminf(fmaxf(bf16_lo(xw[t][i + 1]) * inv, -448.f), 448.f);
            const float q3 = fminf(fmaxf(bf16_hi(xw[t][i + 1]) * inv, -448.f), 448.f);
            int p = __builtin_amdgcn_cvt_pk_fp8_f32(q0, q1, 0, false);
            p = __builtin_amdgcn_cvt_pk_fp8_f32(q2, q3, p, true);
            xw[t][i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((uint32_t)p, s, false));
            xw[t][i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((uint32_t)p, s, true));
        }
    }
}

__device__ __forceinline__ float dot2(bf16x2 w, uint32_t x, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(w, __builtin_bit_cast(bf16x2, x), acc, false);
}

// sum over the chunk of x * weight for each token; OCP FP4 or FP8 weights converted times `cs` (an
// E8M0 scale as e8m0_cvt_scale, or 1).
template <WFmt F, int M, int CH>
__device__ __forceinline__ void chunk_dot_packed(float (&s)[M], const u32x4 w, const uint32_t (&xw)[M][CH / 2],
                                                 float cs = 1.0f) {
    static_assert(F == WFmt::FP4_OCP || F == WFmt::FP8_B128 || F == WFmt::FP8_E8M0, "packed path: OCP FP4 or FP8");
    float s2[M];
#pragma unroll
    for (int t = 0; t < M; t++) s[t] = 0.f, s2[t] = 0.f;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        if constexpr (F == WFmt::FP4_OCP) {  // byte b of dword d: elements 8d + 2b, +1 = x word 4d + b
            const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], cs, 0);
            const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], cs, 1);
            const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], cs, 2);
            const bf16x2 e = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], cs, 3);
#pragma unroll
            for (int t = 0; t < M; t++) {
                s[t] = dot2(a, xw[t][4 * d], s[t]);
                s2[t] = dot2(b, xw[t][4 * d + 1], s2[t]);
                s[t] = dot2(c, xw[t][4 * d + 2], s[t]);
                s2[t] = dot2(e, xw[t][4 * d + 3], s2[t]);
            }
        } else {  // bytes 0,1 / 2,3 of dword d: elements 4d, 4d+1 / 4d+2, 4d+3 = x words 2d / 2d+1
            const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[d], cs, false);
            const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[d], cs, true);
#pragma unroll
            for (int t = 0; t < M; t++) {
                s[t] = dot2(a, xw[t][2 * d], s[t]);
                s2[t] = dot2(b, xw[t][2 * d + 1], s2[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < M; t++) s[t] += s2[t];
}

// GGUF block codes (byte j: elements j and j + 16) times bf16-exact x packed as x[j] = elements j,
// j + 16: one scaled conversion and one dot2 per code byte.
__device__ __forceinline__ float gguf_dot_bf16(const u32x4 w, const uint32_t (&x)[16], float cs) {
    float s = 0.f, s2 = 0.f;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        s = dot2(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], cs, 0), x[4 * d], s);
        s2 = dot2(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], cs, 1), x[4 * d + 1], s2);
        s = dot2(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], cs, 2), x[4 * d + 2], s);
        s2 = dot2(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], cs, 3), x[4 * d + 3], s2);
    }
    return s + s2;
}

}  // namespace stbl
