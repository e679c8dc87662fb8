// Shared device helpers for the quantized expert-GEMV kernels (gfx950 / CDNA4, wave64).
//
// Formats handled here (each decode is exact; the reference arithmetic they restate is cited):
//   e4m3 (OCP "fn"): sign, 4 exponent bits (bias 7), 3 mantissa bits, subnormal m/8 * 2^-6, codes
//        0x7f/0xff NaN, no infinities (tools/convert_official.py:40-48, ref/kernel.py:41).
//   e2m1: the 16-entry table {0, .5, 1, 1.5, 2, 3, 4, 6} with bit 3 the sign (ref/kernel.py:14-16);
//        two codes per byte, element 2i in the low nibble (ref/kernel.py:70-71, :98-100).
//   e8m0: 2^(s-127); s = 0 reads as 2^-127 and s = 255 as NaN, as torch's float8_e8m0fnu does
//        (ref/kernel.py:45,72,101).
//   bf16: the high half of an fp32, rounded to nearest even (torch .to(bfloat16)).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace stbl {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));  // an f8f6f4 MFMA operand

// Loads of weights, which are read once per launch: the non-temporal hint lets the caches evict
// them first (measured: a plain streaming read of 128 MiB to 1 GiB runs 10-14% faster with it).
__device__ __forceinline__ u32x4 ld_stream(const void *p) { return __builtin_nontemporal_load((const u32x4 *)p); }
__device__ __forceinline__ uint32_t ld_stream_u8(const uint8_t *p) { return __builtin_nontemporal_load(p); }

constexpr int kWave = 64;

constexpr int pow2_at_least(int n) { return n <= 1 ? 1 : 2 * pow2_at_least((n + 1) / 2); }
constexpr int log2_exact(int n) { return n <= 1 ? 0 : 1 + log2_exact(n / 2); }

// ---- bf16 <-> fp32 -------------------------------------------------------------------------------

__host__ __device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __builtin_bit_cast(float, h << 16); }

// Round to nearest even; a NaN stays a (quiet) NaN.
__host__ __device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// Low / high bf16 of a packed pair as fp32.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ---- scale codecs --------------------------------------------------------------------------------

// Selects, not branches: a branch on a loaded scale byte makes the compiler wait for that load
// before issuing the loads after it.
__device__ __forceinline__ float e8m0_to_f32(uint32_t s) {
    s &= 0xffu;
    uint32_t b = s << 23;
    b = s == 0 ? 0x00400000u : b;    // 2^-127
    b = s == 255 ? 0x7fc00000u : b;  // NaN
    return __uint_as_float(b);
}

// The scaled conversions (v_cvt_scalef32_pk_{f32,bf16}_fp4, _bf16_fp8) multiply by 2^(e - 127) for a
// scale operand whose exponent field is e, exactly as E8M0 defines it: measured on gfx950 against
// e2m1 / e4m3 code x 2^(s - 127) for every scale byte s and code (s = 0 gives 2^-127, s = 255 NaN,
// results rounded like a single product). So an E8M0 byte placed in the exponent field is the scale
// operand, and a chunk's scale is applied inside its conversions instead of by a decode and a multiply.
__device__ __forceinline__ float e8m0_cvt_scale(uint32_t s) { return __uint_as_float((s & 0xffu) << 23); }

// 2^ceil(log2 t) for positive normal t by its exponent and mantissa bits (ref/kernel.py:22-26).
__device__ __forceinline__ float pow2_ceil(float t) {
    const uint32_t b = __float_as_uint(t);
    const int e = (int)((b >> 23) & 0xffu) - 127 + ((b & 0x7fffffu) != 0);
    return __uint_as_float((uint32_t)(e + 127) << 23);
}

// ---- element decoders (CDNA4 conversion instructions) -------------------------------------------

// Two e4m3 codes (bytes 0,1 of w when hi == false, bytes 2,3 when true) -> fp32, exactly.
__device__ __forceinline__ f32x2 e4m3x2(uint32_t w, bool hi) {
    return hi ? __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true) : __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
}

// The two e2m1 codes of byte `sel` of w -> fp32 (low nibble in .x), exactly, times `cs` (a conversion
// scale from e8m0_cvt_scale, or 1).
template <int sel>
__device__ __forceinline__ f32x2 e2m1x2(uint32_t w, float cs = 1.0f) {
    return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, cs, sel);
}

// Scalar e4m3 decode (closed form), used where a single value is needed.
__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
    const f32x2 v = __builtin_amdgcn_cvt_pk_f32_fp8((int)(c & 0xffu), false);
    return v.x;
}

// fp32 -> e4m3 code, round to nearest even. `x` is already clamped to [-448, 448]; NaN -> 0x7f.
// Built on the e4m3 grid directly: the quantum of |x| is 2^(max(E,-6)-3) for |x| in [2^E, 2^(E+1)),
// the quotient |x| / quantum is exact in fp32 and rintf rounds it to even.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return 0x7fu;
    if (a >= 0x43e00000u) return sign | 0x7eu;  // 448
    int E = (int)(a >> 23) - 127;
    if (E < -6) E = -6;
    const float q = rintf(__uint_as_float(a) * __uint_as_float((uint32_t)(127 - (E - 3)) << 23));
    int qi = (int)q;
    if (E == -6 && qi < 8) return sign | (uint32_t)qi;
    if (qi == 16) E += 1, qi = 8;
    return sign | (uint32_t)(((E + 7) << 3) | (qi - 8));
}

// e2m1 value table (ref/kernel.py:14-16).
__device__ __forceinline__ float e2m1_value(uint32_t c) {
    const uint32_t m = c & 7u;
    const float mag = m < 4 ? 0.5f * (float)m : (m < 6 ? (float)(m - 2) : (m == 6 ? 4.0f : 6.0f));
    return (c & 8u) ? -mag : mag;
}

// Onto the e2m1 grid, ties to even (ref/kernel.py:48-52); v is within [-6, 6].
__device__ __forceinline__ float round_fp4(float v) {
    const float a = fabsf(v);
    const float step = a < 2.f ? .5f : (a < 4.f ? 1.f : 2.f);
    return copysignf(rintf(a / step) * step, v);
}

// e2m1 code of a grid value (ref/kernel.py:75-77): magnitude index | sign bit << 3.
__device__ __forceinline__ uint32_t fp4_code(float q) {
    const float a = fabsf(q);
    const uint32_t m = a <= 1.5f ? (uint32_t)(a * 2.f) : (a <= 3.f ? (uint32_t)(a + 2.f) : (a <= 4.f ? 6u : 7u));
    return m | ((__float_as_uint(q) >> 28) & 8u);
}

// ---- wave reductions -----------------------------------------------------------------------------

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

// Sum over the 64 lanes of a wave with DPP data movement only (no LDS crossbar): pairs, quads,
// half rows, rows, then the row broadcasts. The total is valid in lane 63.
__device__ __forceinline__ float dpp_sum(float v) {
#define STBL_DPP_ADD(ctrl, rmask) \
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, rmask, 0xF, false))
    STBL_DPP_ADD(0xB1, 0xF);   // quad_perm [1,0,3,2]
    STBL_DPP_ADD(0x4E, 0xF);   // quad_perm [2,3,0,1]
    STBL_DPP_ADD(0x141, 0xF);  // row_half_mirror
    STBL_DPP_ADD(0x140, 0xF);  // row_mirror
    STBL_DPP_ADD(0x142, 0xA);  // row_bcast:15 into rows 1 and 3
    STBL_DPP_ADD(0x143, 0xC);  // row_bcast:31 into rows 2 and 3
#undef STBL_DPP_ADD
    return v;
}

// One DPP step of wave_sum_rows: with HALF > 0 the lane keeps v[i] (or v[i + HALF] when `up`) for
// i < HALF and adds the DPP partner's copy of it; with HALF == 0 it adds the partner's v[0].
template <int CTRL, int HALF, int N>
__device__ __forceinline__ void dpp_keep_step(float (&v)[N], bool up) {
#pragma unroll
    for (int i = 0; i < (HALF > 0 ? HALF : 1); i++) {
        const float keep = HALF > 0 ? (up ? v[i + HALF] : v[i]) : v[i];
        const float give = HALF > 0 ? (up ? v[i] : v[i + HALF]) : v[i];
        v[i] = keep + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, give), CTRL, 0xF, 0xF, false));
    }
}

// Sums each of N values over the 64 lanes of a wave (N a power of two, <= 32) in N - 1 + 6 - log2 N
// exchange-and-add steps instead of 6 N. Each step pairs the lanes that differ in one lane bit (5,
// 4, 3, 2, 1, 0 in that order): while more than one value is left, the lanes with the bit clear keep
// the lower half of their list and the others the upper half, and each adds its partner's copy of
// the half it keeps. Partners over bit 5 / bit 4 come from v_permlane32_swap / v_permlane16_swap,
// which exchange two whole lists in one instruction (swap(A, B) = {A lo | B lo}, {A hi | B hi} over
// 32- / 16-lane halves); over bits 3, 2, 1, 0 from DPP row_ror:8, row_half_mirror and quad_perm. Every
// N pairs the same lanes in the same order (a sum of two lanes is the same whichever lane forms it),
// so a value's total does not depend on N. On return lane L holds the total of value L >> (6 - log2
// N), as do the other 64 / N lanes of its group.
template <int N>
__device__ __forceinline__ float wave_sum_rows(float (&v)[N]) {
    static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16 || N == 32, "N: a power of two <= 32");
    const int lane = __lane_id();
    auto bits = [](float f) { return __builtin_bit_cast(uint32_t, f); };
    auto flt = [](uint32_t u) { return __builtin_bit_cast(float, u); };
    // bits 5 and 4: partner copies by lane swaps
    constexpr int h5 = N >= 2 ? N / 2 : 1;
#pragma unroll
    for (int i = 0; i < h5; i++) {
        const auto r = __builtin_amdgcn_permlane32_swap(bits(v[i]), bits(v[N >= 2 ? i + N / 2 : i]), false, false);
        v[i] = flt(r[0]) + flt(r[1]);
    }
    constexpr int h4 = N >= 4 ? N / 4 : 1;
#pragma unroll
    for (int i = 0; i < h4; i++) {
        const auto r = __builtin_amdgcn_permlane16_swap(bits(v[i]), bits(v[N >= 4 ? i + N / 4 : i]), false, false);
        v[i] = flt(r[0]) + flt(r[1]);
    }
    // bits 3, 2, 1, 0: DPP; a lane keeps one value of each pair and adds its partner's copy of it
    dpp_keep_step<0x128, N / 8>(v, lane & 8);   // row_ror:8 = lane ^ 8
    dpp_keep_step<0x141, N / 16>(v, lane & 4);  // row_half_mirror: lane ^ 7 within 8
    dpp_keep_step<0x4E, N / 32>(v, lane & 2);   // quad_perm [2,3,0,1] = lane ^ 2
    dpp_keep_step<0xB1, 0>(v, lane & 1);        // quad_perm [1,0,3,2] = lane ^ 1
    return v[0];
}

}  // namespace stbl
