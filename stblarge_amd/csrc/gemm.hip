// Multi-token expert GEMM on CDNA4 scaled MFMA: Y[m][n] = sum_k Aq[m][k] * Wdeq[n][k], M <= 64.
//
// Reference: fp8_gemm / fp4_gemm of ref/kernel.py:85-102 with M = 64 rows of activations:
//   A = act_quant(X, block, "ue8m0") (e4m3 codes, power-of-two scales per `block` along K),
//   FP8 W: e4m3 with fp32 scales per 128x128 block; FP4 W: e2m1 with E8M0 scales per 32 along K;
//   fp32 accumulation, bf16 output.
// Three launches:
//   k_act_quant_e4m3  X bf16 -> e4m3 codes + E8M0 scale bytes, one 16-lane group per block of 128
//                     (or 4 lanes per block of 32); the e4m3 rounding uses v_cvt_pk_fp8_f32, which
//                     equals the round-to-nearest-even encoder bit for bit on every bf16 input;
//   k_gemm            v_mfma_scale_f32_16x16x128_f8f6f4 with A = e4m3 activations and B = the e4m3 or
//                     e2m1 weights. The activation scales (powers of two) and the FP4 weight scales
//                     (E8M0) are the MFMA's own per-32 scale operands, so the hardware applies them
//                     exactly; the FP8 weights' fp32 block scale multiplies each 128-K step's product
//                     in fp32. A workgroup owns 64 output columns (one 16-column MFMA tile per wave)
//                     and a K slice; its activation slice is staged once in LDS in MFMA operand order
//                     and shared by the 4 waves; each wave streams its weights straight into
//                     registers, all of its slice's loads in flight at once;
//   k_gemm_reduce     sums the K slices' fp32 partials in slice order (deterministic) and rounds to
//                     bf16.
// Operand layout of the 16x16x128 f8f6f4 MFMA (probed on gfx950): lane l = r + 16 g holds row r of A
// (column r of B); e4m3 operands hold K bytes [16g, 16g+16) and [64+16g, 64+16g+16) of the 128-K
// step, e2m1 operands K elements [32g, 32g+32) (low nibble first); the lane's E8M0 scale covers K
// block [32g, 32g+32); D lane l holds rows 4g..4g+3 of column r.
#include "abi_util.hpp"
#include "common.hpp"

namespace stbl {

typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr int kGemmMaxM = 64;
constexpr int kGemmMaxSteps = 8;  // 128-K steps per workgroup slice

// ---- activation quantization --------------------------------------------------------------------

// x bf16 [rows][k] -> codes e4m3 [rows][k], scales E8M0 bytes [rows][k / block]. Each thread takes 8
// consecutive values; block / 8 threads share a block (8 or 16 lanes of one wave).
__global__ __launch_bounds__(256) void k_act_quant_e4m3(const uint16_t *__restrict__ x, int n8, int block,
                                                        uint8_t *__restrict__ codes, uint8_t *__restrict__ scales) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const bool ok = i < n8;
    const u32x4 v = *(const u32x4 *)(x + (size_t)(ok ? i : 0) * 8);
    float f[8];
#pragma unroll
    for (int j = 0; j < 4; j++) f[2 * j] = bf16_lo(v[j]), f[2 * j + 1] = bf16_hi(v[j]);
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) a = fmaxf(a, fabsf(f[j]));
    const int lanes = block >> 3;  // 4 or 16, a power of two
    for (int o = 1; o < lanes; o <<= 1) a = fmaxf(a, __shfl_xor(a, o, kWave));
    const float s = pow2_ceil(fmaxf(a, 1e-4f) * (1.0f / 448.0f));
    const float inv = __uint_as_float((uint32_t)(254 - ((__float_as_uint(s) >> 23) & 0xffu)) << 23);  // 1/s, exact
    uint32_t w[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        // x / s is exact (s is a power of two); the clamp is ref/kernel.py:41's
        float q[4];
#pragma unroll
        for (int e = 0; e < 4; e++) q[e] = fminf(fmaxf(f[4 * j + e] * inv, -448.f), 448.f);
        int p = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
        p = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], p, true);
        w[j] = (uint32_t)p;
    }
    if (!ok) return;
    *(u32x2 *)(codes + (size_t)i * 8) = u32x2{w[0], w[1]};
    if ((threadIdx.x & (lanes - 1)) == 0) scales[(size_t)i * 8 / block] = (uint8_t)((__float_as_uint(s) >> 23) & 0xffu);
}

// ---- GEMM ---------------------------------------------------------------------------------------

template <bool FP4W>
__global__ __launch_bounds__(256) void k_gemm(const uint8_t *__restrict__ wc, const void *__restrict__ ws,
                                              const uint8_t *__restrict__ aq, const uint8_t *__restrict__ as_,
                                              float *__restrict__ part, int M, int N, int K, int act_shift,
                                              int steps_per_slice) {
    // A operands of the slice, in MFMA order, as two planes of 16 bytes per lane (so that a wave's
    // ds_read_b128 reads one contiguous kilobyte, free of bank conflicts): plane p holds
    // [m-tile][step][lane] the lane's bytes [16p, 16p+16); scales [m-tile][step][lane]
    __shared__ u32x4 lds_a[4 * kGemmMaxSteps * 64 * 2];
    __shared__ uint32_t lds_s[4 * kGemmMaxSteps * 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 64, slice = blockIdx.y;
    const int KS = K >> 7, step0 = slice * steps_per_slice;
    const int nsteps = min(steps_per_slice, KS - step0);

    // 1. activation slice loads (issued first: they come from L2 and gate the LDS stage)
    //    unit q = (m-tile, step, lane): 2 x 16 bytes of row 16 mt + r at step k-offsets 16g and 64+16g.
    //    Every load is unconditional, from an address clamped into the buffers; dead units are
    //    zeroed afterwards, so no load sits behind a branch and all of them are in flight together.
    constexpr int kUnits = 4 * kGemmMaxSteps * 64;
    u32x4 av[kUnits / 256][2];
    uint32_t sv[kUnits / 256];
    bool aok[kUnits / 256];
#pragma unroll
    for (int j = 0; j < kUnits / 256; j++) {
        const int q = tid + 256 * j, mt = q / (kGemmMaxSteps * 64), st = (q / 64) % kGemmMaxSteps, l = q & 63;
        const int m = 16 * mt + (l & 15), gg = l >> 4;
        aok[j] = m < M && st < nsteps;
        const size_t kb = (size_t)(step0 + (aok[j] ? st : 0)) * 128;
        const uint8_t *row = aq + (size_t)(aok[j] ? m : 0) * K + kb;
        av[j][0] = *(const u32x4 *)(row + 16 * gg);
        av[j][1] = *(const u32x4 *)(row + 64 + 16 * gg);
        sv[j] = as_[(size_t)(aok[j] ? m : 0) * (K >> act_shift) + ((kb + 32 * gg) >> act_shift)];
    }
    // 2. this wave's weights for every step of the slice: column n = n0 + 16 wave + r
    const int n = min(n0 + 16 * wave + r, N - 1);
    u32x4 bw[kGemmMaxSteps][2];
    uint32_t bsc[kGemmMaxSteps];
    float wsc[kGemmMaxSteps];
#pragma unroll
    for (int s = 0; s < kGemmMaxSteps; s++) {
        const size_t kb = (size_t)(step0 + (s < nsteps ? s : 0)) * 128;
        if constexpr (FP4W) {
            bw[s][0] = *(const u32x4 *)(wc + (size_t)n * (K >> 1) + ((kb + 32 * g) >> 1));
            bsc[s] = ((const uint8_t *)ws)[(size_t)n * (K >> 5) + ((kb + 32 * g) >> 5)];
        } else {
            const uint8_t *row = wc + (size_t)n * K + kb;
            bw[s][0] = *(const u32x4 *)(row + 16 * g);
            bw[s][1] = *(const u32x4 *)(row + 64 + 16 * g);
            wsc[s] = ((const float *)ws)[(size_t)(n0 >> 7) * KS + (kb >> 7)];
        }
    }
    // 3. stage the activation operands (dead units as zeros)
    const u32x4 z4 = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < kUnits / 256; j++) {
        const int q = tid + 256 * j;
        lds_a[q] = aok[j] ? av[j][0] : z4;
        lds_a[kUnits + q] = aok[j] ? av[j][1] : z4;
        lds_s[q] = aok[j] ? sv[j] : 127u;
    }
    __syncthreads();
    // 4. MFMAs: 4 m-tiles x kGemmMaxSteps steps; a step past the slice has zero operands (and a zero
    //    block scale for FP8), so it adds nothing and needs no branch
    f32x4 acc[4];
#pragma unroll
    for (int mt = 0; mt < 4; mt++) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kGemmMaxSteps; s++) {
        const bool live = s < nsteps;
        const u32x4 b0 = live ? bw[s][0] : z4;
        i32x8 b;
        if constexpr (FP4W) {
            b = i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], 0, 0, 0, 0};
        } else {
            const u32x4 b1 = live ? bw[s][1] : z4;
            b = i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
        }
#pragma unroll
        for (int mt = 0; mt < 4; mt++) {
            const int q = (mt * kGemmMaxSteps + s) * 64 + lane;
            const u32x4 a0 = lds_a[q], a1 = lds_a[kUnits + q];
            const i32x8 a = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
            const int sa = (int)lds_s[q];
            if constexpr (FP4W) {
                acc[mt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[mt], 0, 4, 0, sa, 0,
                                                                           live ? (int)bsc[s] : 127);
            } else {
                const f32x4 d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0,
                                                                                  0, sa, 0, 127);
                const float sw = live ? wsc[s] : 0.f;
#pragma unroll
                for (int e = 0; e < 4; e++) acc[mt][e] = fmaf(sw, d[e], acc[mt][e]);
            }
        }
    }
    // 5. partials [slice][m][n]
    const int ncol = n0 + 16 * wave + r;
    if (ncol >= N) return;
#pragma unroll
    for (int mt = 0; mt < 4; mt++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = 16 * mt + 4 * g + e;
            if (m < M) part[((size_t)slice * M + m) * N + ncol] = acc[mt][e];
        }
}

// y[m][n] = bf16(sum over slices in order of part[slice][m][n]) (or the fp32 sum when y_f32).
__global__ void k_gemm_reduce(const float *__restrict__ part, int slices, int mn, void *__restrict__ y, int y_f32) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= mn) return;
    float s = part[i];
    for (int sl = 1; sl < slices; sl++) s += part[(size_t)sl * mn + i];
    if (y_f32) ((float *)y)[i] = s;
    else ((uint16_t *)y)[i] = f32_to_bf16_bits(s);
}

// Slicing of K: about 2 workgroups per CU in total, each slice at most kGemmMaxSteps 128-K steps.
static void gemm_plan(int n, int k, int *slices, int *steps) {
    const int ntiles = (n + 63) / 64, ks = k / 128;
    int want = 256 / ntiles;
    if (want < 1) want = 1;
    int st = (ks + want - 1) / want;
    if (st > kGemmMaxSteps) st = kGemmMaxSteps;
    if (st < 1) st = 1;
    *steps = st;
    *slices = (ks + st - 1) / st;
}

static uint64_t a256(uint64_t v) { return (v + 255) & ~(uint64_t)255; }

}  // namespace stbl

using namespace stbl;

extern "C" {

uint64_t stbl_amd_gemm_work_bytes(int m, int n, int k) {
    int slices, steps;
    gemm_plan(n, k, &slices, &steps);
    return a256((uint64_t)m * k) + a256((uint64_t)m * (k / 32)) + a256((uint64_t)slices * m * n * 4);
}

int stbl_amd_gemm(int fmt, void *y, const void *codes, const void *scales, const void *x, int m, int n, int k,
                  int act_block, int y_f32, void *work, hipStream_t st) {
    if (fmt != 0 && fmt != 1) return abi_fail(hipErrorInvalidValue, "gemm: unknown format %d", fmt);
    if (!y || !codes || !scales || !x || !work) return abi_fail(hipErrorInvalidValue, "gemm: null pointer");
    if (m < 1 || m > kGemmMaxM || n < 1 || k < 128 || k % 128 || (act_block != 32 && act_block != 128))
        return abi_fail(hipErrorInvalidValue, "gemm: need 1 <= m <= 64, k %% 128 == 0, act_block 32 or 128 (m=%d k=%d)", m, k);
    if (!aligned16(codes) || !aligned16(x) || !aligned16(work)) return abi_fail(hipErrorInvalidValue, "gemm: codes, x, work must be 16-byte aligned");
    int slices, steps;
    gemm_plan(n, k, &slices, &steps);
    uint8_t *aq = (uint8_t *)work;
    uint8_t *as_ = aq + a256((uint64_t)m * k);
    float *part = (float *)(as_ + a256((uint64_t)m * (k / 32)));
    const int n8 = m * k / 8;
    hipLaunchKernelGGL(k_act_quant_e4m3, dim3((n8 + 255) / 256), dim3(256), 0, st, (const uint16_t *)x, n8, act_block, aq, as_);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) {
        const dim3 grid((n + 63) / 64, slices);
        if (fmt == 0)
            hipLaunchKernelGGL(k_gemm<true>, grid, dim3(256), 0, st, (const uint8_t *)codes, scales, aq, as_, part, m, n, k,
                               act_block == 32 ? 5 : 7, steps);
        else
            hipLaunchKernelGGL(k_gemm<false>, grid, dim3(256), 0, st, (const uint8_t *)codes, scales, aq, as_, part, m, n,
                               k, act_block == 32 ? 5 : 7, steps);
        e = hipGetLastError();
    }
    if (e == hipSuccess) {
        hipLaunchKernelGGL(k_gemm_reduce, dim3((m * n + 255) / 256), dim3(256), 0, st, part, slices, m * n, y, y_f32);
        e = hipGetLastError();
    }
    return abi_status(e, "gemm launch");
}

// act_quant(x, block, "ue8m0") of ref/kernel.py:35-45 with the codes and E8M0 scale bytes it feeds
// the GEMM: x bf16 [rows][k] -> codes [rows][k], scales [rows][k / block]. k % block == 0.
int stbl_amd_act_quant_e4m3(const void *x, int rows, int k, int block, void *codes, void *scales, hipStream_t st) {
    if (!x || !codes || !scales || rows < 1 || (block != 32 && block != 128) || k % block)
        return abi_fail(hipErrorInvalidValue, "act_quant_e4m3: need block 32 or 128 and k %% block == 0");
    if (!aligned16(x) || ((uintptr_t)codes & 7)) return abi_fail(hipErrorInvalidValue, "act_quant_e4m3: x 16-byte, codes 8-byte aligned");
    const int n8 = rows * k / 8;
    hipLaunchKernelGGL(k_act_quant_e4m3, dim3((n8 + 255) / 256), dim3(256), 0, st, (const uint16_t *)x, n8, block,
                       (uint8_t *)codes, (uint8_t *)scales);
    return abi_status(hipGetLastError(), "act_quant_e4m3 launch");
}

}  // extern "C"
