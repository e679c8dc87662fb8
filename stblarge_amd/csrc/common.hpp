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

// Loads of weights, which are read once per launch: the non-temporal hint lets the caches evict
// them first (measured: a plain streaming read of 128 MiB to 1 GiB runs 10-14% faster with it).
__device__ __forceinline__ u32x4 ld_stream(const void *p) { return __builtin_nontemporal_load((const u32x4 *)p); }
__device__ __forceinline__ uint32_t ld_stream_u8(const uint8_t *p) { return __builtin_nontemporal_load(p); }

constexpr int kWave = 64;

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

// The two e2m1 codes of byte `sel` of w -> fp32 (low nibble in .x), exactly.
template <int sel>
__device__ __forceinline__ f32x2 e2m1x2(uint32_t w) {
    return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, sel);
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

// Sums N values per lane over the 64 lanes of a wave with N-1+6-log2(N) exchanges instead of 6N:
// at each halving step a lane keeps one half of its list and adds the partner's copy of that half.
// On return lane L holds the full sum of value index ((L >> 3) & 7) >> (3 - log2 N)... concretely
// `reduced_index(L)` below; every lane of a group of 64/N lanes holds the same sum. N is a power
// of two, 1 <= N <= 8.
template <int N>
__device__ __forceinline__ float wave_sum_transposed(float (&v)[N], int lane) {
    if constexpr (N >= 8) {
        const bool up = lane & 32;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float keep = up ? v[i + 4] : v[i], give = up ? v[i] : v[i + 4];
            v[i] = keep + __shfl_xor(give, 32, kWave);
        }
    }
    if constexpr (N >= 4) {
        constexpr int o = N >= 8 ? 16 : 32;
        const bool up = lane & o;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const float keep = up ? v[i + 2] : v[i], give = up ? v[i] : v[i + 2];
            v[i] = keep + __shfl_xor(give, o, kWave);
        }
    }
    if constexpr (N >= 2) {
        constexpr int o = N >= 8 ? 8 : (N >= 4 ? 16 : 32);
        const bool up = lane & o;
        const float keep = up ? v[1] : v[0], give = up ? v[0] : v[1];
        v[0] = keep + __shfl_xor(give, o, kWave);
    }
    constexpr int first = N >= 8 ? 4 : (N >= 4 ? 8 : (N >= 2 ? 16 : 32));
    float s = v[0];
#pragma unroll
    for (int o = first; o > 0; o >>= 1) s += __shfl_xor(s, o, kWave);
    return s;
}

// Which value index lane L holds after wave_sum_transposed<N>.
template <int N>
__device__ __forceinline__ int reduced_index(int lane) {
    if constexpr (N == 8) return ((lane >> 5) & 1) * 4 + ((lane >> 4) & 1) * 2 + ((lane >> 3) & 1);
    if constexpr (N == 4) return ((lane >> 5) & 1) * 2 + ((lane >> 4) & 1);
    if constexpr (N == 2) return (lane >> 5) & 1;
    return 0;
}

// Lane that holds value index i after wave_sum_transposed<N> (the lowest such lane).
template <int N>
__device__ __forceinline__ int holder_lane(int i) {
    if constexpr (N == 8) return ((i >> 2) & 1) * 32 + ((i >> 1) & 1) * 16 + (i & 1) * 8;
    if constexpr (N == 4) return ((i >> 1) & 1) * 32 + (i & 1) * 16;
    if constexpr (N == 2) return (i & 1) * 32;
    return 0;
}

}  // namespace stbl
