// Quantizers, dequantizers and the elementwise epilogues of the expert-GEMV path.
//
//   act_quant          ref/kernel.py:35-45 (v2, bf16 in, codes + scales out) and the reference
//                      engine's in-place fp32 form stbl/kernels.cu:54-63 (stbl_act_quant_fp8).
//   weight quantizers  FP4: fp4_act_quant's E8M0 path, ref/kernel.py:55-72, on weight rows.
//                      FP8: one fp32 scale per 128x128 block, s = max(amax, 1e-4) / 448.
//   dequantizers       one fp32 product per element, ref/kernel.py:89-90 and :98-101.
//   epilogues          round_bf16 / swiglu / axpy, stbl/kernels.cu:86-89, :444-464.
// None of these is bandwidth-critical at the configs' sizes; they are written for exactness first.
#include "common.hpp"
#include "abi_util.hpp"

namespace stbl {

// ---- activation quantization ---------------------------------------------------------------------

// The reference engine's form: per 32 values in place, s = pow2_ceil(max(amax, 1e-4) * (1/448)),
// x = bf16(e4m3(clamp(x / s, +-448)) * s). One 32-lane half-wave per block of 32.
// The block's amax comes from its 32 lanes (half a wave) by four DPP moves and one lane shuffle
// (instead of five shuffles, each an LDS round trip); x / s is x times the exact inverse of the power of two s; the e4m3 rounding is the
// hardware v_cvt_pk_fp8_f32 (round to nearest even, equal to the software encoder f32_to_e4m3 on
// fp32 inputs), and e4m3 * s is exact.
__device__ __forceinline__ float dpp_max(float a, int ctrl_sel) {
    int m;
    switch (ctrl_sel) {  // compile-time after inlining
        case 0: m = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0xB1, 0xF, 0xF, false); break;   // lane ^ 1
        case 1: m = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x4E, 0xF, 0xF, false); break;   // lane ^ 2
        case 2: m = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x141, 0xF, 0xF, false); break;  // 7 - lane in 8
        default: m = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x140, 0xF, 0xF, false); break; // 15 - lane in 16
    }
    return fmaxf(a, __builtin_bit_cast(float, m));
}

__global__ void k_act_quant_fp8_inplace(float *x, int n_blocks) {
    const int b = (blockIdx.x * blockDim.x + threadIdx.x) >> 5;
    const int i = (blockIdx.x * blockDim.x + threadIdx.x) & 31;
    const bool ok = b < n_blocks;
    const float v = ok ? x[(size_t)b * 32 + i] : 0.f;
    float a = fabsf(v);
    a = dpp_max(a, 0);
    a = dpp_max(a, 1);
    a = dpp_max(a, 2);
    a = dpp_max(a, 3);
    a = fmaxf(a, __shfl_xor(a, 16, kWave));  // lanes l and l ^ 16
    const float s = pow2_ceil(fmaxf(a, 1e-4f) * (1.0f / 448.0f));
    // 1/s, exact; 0 for s = +Inf (a block holding an infinity), where v * 0 is v / s: a signed zero for
    // a finite v, NaN for an infinite one
    const float inv = __builtin_isinf(s) ? 0.f : __uint_as_float((254u - ((__float_as_uint(s) >> 23) & 0xffu)) << 23);
    if (ok) {
        const float q = fminf(fmaxf(v * inv, -448.f), 448.f);
        const uint32_t c = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q, q, 0, false) & 0xffu;
        x[(size_t)b * 32 + i] = bf16_round(e4m3_to_f32(c) * s);
    }
}

// ref/kernel.py:35-45 on bf16 rows: one thread per block of `block` values. codes [rows][n] e4m3,
// scales [rows][n/block] fp32, and (optional) the dequantized bf16 values bf16(e4m3 * s).
__global__ void k_act_quant(const uint16_t *x, int n_blocks, int block, int pow2, uint8_t *codes, float *scales,
                            uint16_t *deq) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blocks) return;
    const uint16_t *xb = x + (size_t)b * block;
    float amax = 0.f;
    for (int i = 0; i < block; i++) amax = fmaxf(amax, fabsf(bf16_bits_to_f32(xb[i])));
    const float t = fmaxf(amax, 1e-4f) * (float)(1.0 / 448.0);
    const float s = pow2 ? pow2_ceil(t) : t;
    if (scales) scales[b] = s;
    for (int i = 0; i < block; i++) {
        const float q = fminf(fmaxf(__fdiv_rn(bf16_bits_to_f32(xb[i]), s), -448.f), 448.f);
        const uint32_t c = f32_to_e4m3(q);
        if (codes) codes[(size_t)b * block + i] = (uint8_t)c;
        if (deq) deq[(size_t)b * block + i] = f32_to_bf16_bits(e4m3_to_f32(c) * s);
    }
}

// ---- weight quantizers ---------------------------------------------------------------------------

// FP4 e2m1 with E8M0 scales per 32 along K. One thread per group of 32: reads 128 bytes, writes
// 16 bytes of codes (element 2i in the low nibble) and one scale byte.
__global__ void k_quant_fp4(const float *w, int n_groups, uint8_t *codes, uint8_t *scales) {
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_groups) return;
    const f32x4 *src = (const f32x4 *)(w + (size_t)g * 32);
    float v[32];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        const f32x4 t = src[q];
        v[4 * q] = t.x, v[4 * q + 1] = t.y, v[4 * q + 2] = t.z, v[4 * q + 3] = t.w;
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, 6.0f * 0x1p-126f);
    const float s = pow2_ceil(amax * (float)(1.0 / 6.0));
    scales[g] = (uint8_t)((__float_as_uint(s) >> 23) & 0xffu);
    u32x4 out;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float q = round_fp4(fminf(fmaxf(v[8 * d + j] / s, -6.f), 6.f));  // exact division
            word |= fp4_code(q) << (4 * j);
        }
        out[d] = word;
    }
    *(u32x4 *)(codes + (size_t)g * 16) = out;
}

// FP8 e4m3 with one fp32 scale per 128x128 block (partial blocks at the edges). One workgroup of
// 256 threads per block: amax by a block reduction, then s = amax / 448 and e4m3(clamp(w / s)),
// both true fp32 divisions.
__global__ __launch_bounds__(256) void k_quant_fp8_b128(const float *w, int rows, int k, uint8_t *codes,
                                                        float *scales) {
    __shared__ float red[4];
    const int bi = blockIdx.y, bj = blockIdx.x, kb = gridDim.x;
    const int r0 = bi * 128, c0 = bj * 128;
    const int nr = min(128, rows - r0), nc = min(128, k - c0);
    float amax = 0.f;
    for (int i = threadIdx.x; i < nr * nc; i += 256) amax = fmaxf(amax, fabsf(w[(size_t)(r0 + i / nc) * k + c0 + i % nc]));
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = __fdiv_rn(fmaxf(amax, 1e-4f), 448.0f);
    if (threadIdx.x == 0) scales[(size_t)bi * kb + bj] = s;
    for (int i = threadIdx.x; i < nr * nc; i += 256) {
        const size_t at = (size_t)(r0 + i / nc) * k + c0 + i % nc;
        codes[at] = (uint8_t)f32_to_e4m3(fminf(fmaxf(__fdiv_rn(w[at], s), -448.f), 448.f));
    }
}

// FP8 e4m3 with one E8M0 scale per 32x32 block (the reference engine's FP8 layout, stbl/kernels.cu:
// 98-103): s = pow2_ceil(max(amax, 1e-4) * fp32(1/448)) as act_quant's power-of-two rule
// (ref/kernel.py:38-40), q = e4m3_rne(clamp(w / s, +-448)) (w / s is exact). One 256-thread
// workgroup per block; scales [(rows+31)/32][k/32] bytes.
__global__ __launch_bounds__(256) void k_quant_fp8_e8m0(const float *w, int rows, int k, uint8_t *codes,
                                                        uint8_t *scales) {
    __shared__ float red[4];
    const int bi = blockIdx.y, bj = blockIdx.x, kb = gridDim.x;
    const int r0 = bi * 32, c0 = bj * 32, nr = min(32, rows - r0);
    float amax = 0.f;
    for (int i = threadIdx.x; i < nr * 32; i += 256) amax = fmaxf(amax, fabsf(w[(size_t)(r0 + i / 32) * k + c0 + i % 32]));
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = pow2_ceil(fmaxf(amax, 1e-4f) * (1.0f / 448.0f));
    if (threadIdx.x == 0) scales[(size_t)bi * kb + bj] = (uint8_t)((__float_as_uint(s) >> 23) & 0xffu);
    for (int i = threadIdx.x; i < nr * 32; i += 256) {
        const size_t at = (size_t)(r0 + i / 32) * k + c0 + i % 32;
        codes[at] = (uint8_t)f32_to_e4m3(fminf(fmaxf(__fdiv_rn(w[at], s), -448.f), 448.f));
    }
}

// ---- dequantizers (the bit-exactness check of the decoders the GEMVs use) ------------------------

// FP4 OCP: out[r][c] = e2m1(code) * 2^(s-127), one fp32 product. One thread per 32-group.
__global__ void k_dequant_fp4(const uint8_t *codes, const uint8_t *scales, int n_groups, float *out) {
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_groups) return;
    const u32x4 w = *(const u32x4 *)(codes + (size_t)g * 16);
    const float s = e8m0_to_f32(scales[g]);
    float *o = out + (size_t)g * 32;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const f32x2 a = e2m1x2<0>(w[d]), b = e2m1x2<1>(w[d]), c = e2m1x2<2>(w[d]), e = e2m1x2<3>(w[d]);
        *(f32x4 *)(o + 8 * d) = f32x4{a.x * s, a.y * s, b.x * s, b.y * s};
        *(f32x4 *)(o + 8 * d + 4) = f32x4{c.x * s, c.y * s, e.x * s, e.y * s};
    }
}

// GGUF MXFP4 rows of 17-byte blocks (byte 0: E8M0 scale; bytes 1..16: element i in the low nibble
// and element 16+i in the high nibble of byte 1+i). One thread per block, byte reads.
__global__ void k_dequant_gguf17(const uint8_t *w, int n_blocks, float *out) {
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_blocks) return;
    const uint8_t *blk = w + (size_t)g * 17;
    const float s = e8m0_to_f32(blk[0]);
    float *o = out + (size_t)g * 32;
    for (int i = 0; i < 16; i++) {
        const uint32_t byte = blk[1 + i];
        const f32x2 v = e2m1x2<0>(byte);
        o[i] = v.x * s;
        o[16 + i] = v.y * s;
    }
}

// FP8 e4m3 with fp32 128x128 block scales (scale_e8m0 == 0), or with E8M0 bytes per 32x32 block, the
// reference engine's layout [(rows+31)/32][k/32] (scale_e8m0 == 1). One thread per 16 values.
__global__ void k_dequant_fp8(const uint8_t *codes, const void *scales, int rows, int k, int scale_e8m0, float *out) {
    const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16;
    if (i >= (size_t)rows * k) return;
    const int r = (int)(i / k), c = (int)(i % k);
    const u32x4 w = *(const u32x4 *)(codes + i);
    float s;
    if (scale_e8m0) s = e8m0_to_f32(((const uint8_t *)scales)[(size_t)(r >> 5) * (k >> 5) + (c >> 5)]);
    else s = ((const float *)scales)[(size_t)(r >> 7) * ((k + 127) >> 7) + (c >> 7)];
    float *o = out + i;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const f32x2 a = e4m3x2(w[d], false), b = e4m3x2(w[d], true);
        *(f32x4 *)(o + 4 * d) = f32x4{a.x * s, a.y * s, b.x * s, b.y * s};
    }
}

// ---- epilogues (stbl/kernels.cu:86-89, 444-464) --------------------------------------------------

__global__ void k_round_bf16(float *x, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = bf16_round(x[i]);
}

constexpr int kSegMax = 16;
struct SegWeights {
    float w[kSegMax];
};

// out = bf16(silu(min(g, lim)) * clamp(u, +-lim) * w), no clamps when lim <= 0; segment blockIdx.y
// of `count` consecutive n-long segments uses weight w[blockIdx.y]. silu(g) = g / (1 + exp(-g)).
__global__ void k_swiglu(float *out, const float *g, const float *u, SegWeights ws, float limit, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const size_t at = (size_t)blockIdx.y * n + i;
    float gv = g[at], uv = u[at];
    if (limit > 0) {
        uv = fminf(fmaxf(uv, -limit), limit);
        gv = fminf(gv, limit);
    }
    out[at] = bf16_round(__fdiv_rn(gv, 1.f + expf(-gv)) * uv * ws.w[blockIdx.y]);
}

// y += a * x as one fused multiply-add (nvcc contracts the reference's `y[i] += a * x[i]`).
__global__ void k_axpy(float *y, const float *x, float a, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = fmaf(a, x[i], y[i]);
}

static inline unsigned grid_for(size_t n, int b) { return (unsigned)((n + b - 1) / b); }

}  // namespace stbl

using namespace stbl;

extern "C" {

// stbl/kernels.h:9. n % 32 == 0.
void stbl_act_quant_fp8(float *x, int n, hipStream_t st) {
    if (!x || n <= 0 || n % 32) {
        abi_fail(hipErrorInvalidValue, "stbl_act_quant_fp8: need n %% 32 == 0 (n=%d)", n);
        return;
    }
    hipLaunchKernelGGL(k_act_quant_fp8_inplace, dim3(grid_for((size_t)n, 256)), dim3(256), 0, st, x, n / 32);
    abi_status(hipGetLastError(), "stbl_act_quant_fp8 launch");
}

// stbl/kernels.h:11.
void stbl_round_bf16(float *x, int n, hipStream_t st) {
    if (!x || n <= 0) {
        abi_fail(hipErrorInvalidValue, "stbl_round_bf16: bad arguments (n=%d)", n);
        return;
    }
    hipLaunchKernelGGL(k_round_bf16, dim3(grid_for((size_t)n, 256)), dim3(256), 0, st, x, n);
    abi_status(hipGetLastError(), "stbl_round_bf16 launch");
}

// stbl/kernels.h:37-38. `weights` is a host array of `count` <= 16 floats.
void stbl_swiglu_batch(float *out, const float *g, const float *u, const float *weights, int count, float limit, int n,
                       hipStream_t st) {
    if (!out || !g || !u || !weights || count <= 0 || count > kSegMax || n <= 0) {
        abi_fail(hipErrorInvalidValue, "stbl_swiglu_batch: bad arguments (count=%d n=%d)", count, n);
        return;
    }
    SegWeights ws = {};
    for (int j = 0; j < count; j++) ws.w[j] = weights[j];
    hipLaunchKernelGGL(k_swiglu, dim3(grid_for((size_t)n, 256), count), dim3(256), 0, st, out, g, u, ws, limit, n);
    abi_status(hipGetLastError(), "stbl_swiglu_batch launch");
}

// stbl/kernels.h:35.
void stbl_swiglu(float *out, const float *g, const float *u, float weight, float limit, int n, hipStream_t st) {
    stbl_swiglu_batch(out, g, u, &weight, 1, limit, n, st);
}

// stbl/kernels.h:39.
void stbl_axpy(float *y, const float *x, float a, int n, hipStream_t st) {
    if (!y || !x || n <= 0) {
        abi_fail(hipErrorInvalidValue, "stbl_axpy: bad arguments (n=%d)", n);
        return;
    }
    hipLaunchKernelGGL(k_axpy, dim3(grid_for((size_t)n, 256)), dim3(256), 0, st, y, x, a, n);
    abi_status(hipGetLastError(), "stbl_axpy launch");
}

int stbl_amd_act_quant(const void *x, int rows, int n, int block, int pow2, void *codes, float *scales, void *deq,
                       hipStream_t st) {
    if (!x || rows <= 0 || n <= 0 || block <= 0 || n % block) return abi_fail(hipErrorInvalidValue, "act_quant: need n %% block == 0");
    const int nb = rows * (n / block);
    hipLaunchKernelGGL(k_act_quant, dim3(grid_for((size_t)nb, 128)), dim3(128), 0, st, (const uint16_t *)x, nb, block,
                       pow2, (uint8_t *)codes, scales, (uint16_t *)deq);
    return abi_status(hipGetLastError(), "act_quant launch");
}

int stbl_amd_quant_fp4(void *codes, void *scales, const float *w, int rows, int k, hipStream_t st) {
    if (!codes || !scales || !w || rows <= 0 || k <= 0 || k % 32) return abi_fail(hipErrorInvalidValue, "quant_fp4: need k %% 32 == 0");
    if (!aligned16(codes) || !aligned16(w)) return abi_fail(hipErrorInvalidValue, "quant_fp4: codes and w must be 16-byte aligned");
    const int ng = rows * (k / 32);
    hipLaunchKernelGGL(k_quant_fp4, dim3(grid_for((size_t)ng, 256)), dim3(256), 0, st, w, ng, (uint8_t *)codes,
                       (uint8_t *)scales);
    return abi_status(hipGetLastError(), "quant_fp4 launch");
}

int stbl_amd_quant_fp8_b128(void *codes, float *scales, const float *w, int rows, int k, hipStream_t st) {
    if (!codes || !scales || !w || rows <= 0 || k <= 0) return abi_fail(hipErrorInvalidValue, "quant_fp8_b128: bad arguments");
    hipLaunchKernelGGL(k_quant_fp8_b128, dim3((k + 127) / 128, (rows + 127) / 128), dim3(256), 0, st, w, rows, k,
                       (uint8_t *)codes, scales);
    return abi_status(hipGetLastError(), "quant_fp8_b128 launch");
}

// FP8 e4m3 with E8M0 scales per 32x32 block: codes [rows][k], scales [(rows+31)/32][k/32]. k % 32 == 0.
int stbl_amd_quant_fp8_e8m0(void *codes, void *scales, const float *w, int rows, int k, hipStream_t st) {
    if (!codes || !scales || !w || rows <= 0 || k <= 0 || k % 32)
        return abi_fail(hipErrorInvalidValue, "quant_fp8_e8m0: need k %% 32 == 0");
    hipLaunchKernelGGL(k_quant_fp8_e8m0, dim3(k / 32, (rows + 31) / 32), dim3(256), 0, st, w, rows, k, (uint8_t *)codes,
                       (uint8_t *)scales);
    return abi_status(hipGetLastError(), "quant_fp8_e8m0 launch");
}

int stbl_amd_dequant_fp4(float *out, const void *codes, const void *scales, int rows, int k, hipStream_t st) {
    if (!out || !codes || !scales || rows <= 0 || k <= 0 || k % 32) return abi_fail(hipErrorInvalidValue, "dequant_fp4: need k %% 32 == 0");
    if (!aligned16(codes) || !aligned16(out)) return abi_fail(hipErrorInvalidValue, "dequant_fp4: codes and out must be 16-byte aligned");
    const int ng = rows * (k / 32);
    hipLaunchKernelGGL(k_dequant_fp4, dim3(grid_for((size_t)ng, 256)), dim3(256), 0, st, (const uint8_t *)codes,
                       (const uint8_t *)scales, ng, out);
    return abi_status(hipGetLastError(), "dequant_fp4 launch");
}

int stbl_amd_dequant_gguf17(float *out, const void *w, int rows, int k, hipStream_t st) {
    if (!out || !w || rows <= 0 || k <= 0 || k % 32) return abi_fail(hipErrorInvalidValue, "dequant_gguf17: need k %% 32 == 0");
    const int nb = rows * (k / 32);
    hipLaunchKernelGGL(k_dequant_gguf17, dim3(grid_for((size_t)nb, 256)), dim3(256), 0, st, (const uint8_t *)w, nb, out);
    return abi_status(hipGetLastError(), "dequant_gguf17 launch");
}

int stbl_amd_dequant_fp8(float *out, const void *codes, const void *scales, int rows, int k, int scale_e8m0,
                         hipStream_t st) {
    if (!out || !codes || !scales || rows <= 0 || k <= 0 || k % 16 || (scale_e8m0 && k % 32))
        return abi_fail(hipErrorInvalidValue, "dequant_fp8: need k %% 16 == 0 (k %% 32 for E8M0 scales)");
    if (!aligned16(codes) || !aligned16(out)) return abi_fail(hipErrorInvalidValue, "dequant_fp8: codes and out must be 16-byte aligned");
    hipLaunchKernelGGL(k_dequant_fp8, dim3(grid_for((size_t)rows * k / 16, 256)), dim3(256), 0, st,
                       (const uint8_t *)codes, scales, rows, k, scale_e8m0, out);
    return abi_status(hipGetLastError(), "dequant_fp8 launch");
}

}  // extern "C"
