// Multi-token expert GEMM on CDNA4 scaled MFMA: Y[m][n] = sum_k Aq[m][k] * Wdeq[n][k], M <= 64.
//
// Reference: fp8_gemm / fp4_gemm of ref/kernel.py:85-102 with M = 64 rows of activations:
//   A = act_quant(X, block, "ue8m0") (e4m3 codes, power-of-two scales per `block` along K),
//   FP8 W: e4m3 with fp32 scales per 128x128 block; FP4 W: e2m1 with E8M0 scales per 32 along K;
//   fp32 accumulation, bf16 output.
// Kernels:
//   k_act_quant_e4m3  X bf16 -> e4m3 codes + E8M0 scale bytes, one 16-lane group per block of 128
//                     (or 4 lanes per block of 32); the e4m3 rounding uses v_cvt_pk_fp8_f32, which
//                     equals the round-to-nearest-even encoder bit for bit on every bf16 input;
//                     k_act_quant_e4m3_ops the same codes in MFMA operand order, for k_gemm_one;
//   k_gemm            v_mfma_scale_f32_16x16x128_f8f6f4 with A = e4m3 activations and B = the e4m3 or
//                     e2m1 weights. The activation scales (powers of two) and the FP4 weight scales
//                     (E8M0) are the MFMA's own per-32 scale operands, so the hardware applies them
//                     exactly; the FP8 weights' fp32 block scale multiplies each 128-K step's product
//                     in fp32. Split K: each workgroup writes its K slice's partial tile and
//                     k_gemm_reduce adds the slices in order (the kernel boundary is the
//                     synchronization point); stbl_amd_gemm_q takes already quantized activations,
//                     stbl_amd_gemm quantizes X first (one more launch).
//   k_gemm_one        the same products in one launch over all of K, for m > 32 and K % 512 == 0
//                     (the configurations' shapes): small tiles, half-line-balanced operand loads
//                     and scales loaded four steps at a time;
//   k_gemm_pack       the weight codes rearranged once into MFMA operand order (WOPS below), which
//                     both GEMM kernels then read as one contiguous kilobyte per wave load.
// Operand layout of the 16x16x128 f8f6f4 MFMA (probed on gfx950): lane l = r + 16 g holds row r of A
// (column r of B); e4m3 operands hold K bytes [16g, 16g+16) and [64+16g, 64+16g+16) of the 128-K
// step, e2m1 operands K elements [32g, 32g+32) (low nibble first); the lane's E8M0 scale covers K
// block [32g, 32g+32); D lane l holds rows 4g..4g+3 of column r.
#include <algorithm>

#include "abi_util.hpp"
#include "common.hpp"

namespace stbl {

constexpr int kGemmMaxM = 64;
constexpr int kGemmMaxN = 1 << 20;

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
    // 1/s, exact; 0 for s = +Inf (a block holding an infinity), where x * 0 is x / s: a signed zero for
    // a finite x, NaN for an infinite one
    const float inv = __builtin_isinf(s) ? 0.f : __uint_as_float((uint32_t)(254 - ((__float_as_uint(s) >> 23) & 0xffu)) << 23);
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

// The same quantization written in MFMA operand order (stbl_amd_gemm's one-launch plans, whose
// operand loads then each read one contiguous kilobyte): per group of 16 rows and 128-K step, 2 KB,
// in which the 16 bytes lane l = r + 16 g of an operand load takes (row r, bytes [16 g, 16 g + 16) of
// the step's first 64, then of its second 64) sit at l * 16 of the first, then of the second
// kilobyte. One wave per group and step: lane l reads row r's 16 values at [16 g, 16 g + 16) of each
// half of the step and stores their codes as that piece, so each store instruction writes a
// contiguous kilobyte (measured against 8-byte stores scattered into the same layout by
// k_act_quant_e4m3's lanes: full FP4 GEMM at 2048x7168 10.14 -> 9.75 us, FP8 12.83 -> 12.43). A block's amax
// comes from the lanes of the same row: all four for a 128-block (xor 16, 32), the pair g, g ^ 1 of
// one half for a 32-block (block 2 h + g / 2 of the step). Rows past m (up to the group's 16) store
// zero codes and no scales. The codes and scales of rows < m are k_act_quant_e4m3's, byte for byte.
__global__ __launch_bounds__(64) void k_act_quant_e4m3_ops(const uint16_t *__restrict__ x, int m, int k, int block,
                                                          uint8_t *__restrict__ codes, uint8_t *__restrict__ scales) {
    const int ks = k >> 7;
    const int w = blockIdx.x, mg = w / ks, s = w % ks;  // grid: ceil(m / 16) * ks waves
    const int lane = threadIdx.x, r = lane & 15, g = lane >> 4;
    const int row = mg * 16 + r;
    const bool ok = row < m;
    const uint16_t *src = x + (size_t)(ok ? row : 0) * k + (size_t)s * 128 + 16 * g;
    float f[2][16];
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const u32x4 v = *(const u32x4 *)(src + 64 * h + 8 * q);
#pragma unroll
            for (int j = 0; j < 4; j++) f[h][8 * q + 2 * j] = bf16_lo(v[j]), f[h][8 * q + 2 * j + 1] = bf16_hi(v[j]);
        }
    }
    float a[2] = {0.f, 0.f};
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int j = 0; j < 16; j++) a[h] = fmaxf(a[h], fabsf(f[h][j]));
#pragma unroll
    for (int h = 0; h < 2; h++) a[h] = fmaxf(a[h], __shfl_xor(a[h], 16, kWave));  // the lane pair g, g ^ 1
    if (block == 128) {
        const float t = fmaxf(a[0], a[1]);
        a[0] = a[1] = fmaxf(t, __shfl_xor(t, 32, kWave));
    }
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const float sc = pow2_ceil(fmaxf(a[h], 1e-4f) * (1.0f / 448.0f));
        // 1/sc, exact, or 0 for sc = +Inf, as in k_act_quant_e4m3
        const float inv =
            __builtin_isinf(sc) ? 0.f : __uint_as_float((uint32_t)(254 - ((__float_as_uint(sc) >> 23) & 0xffu)) << 23);
        u32x4 out;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // x / sc is exact (sc is a power of two); the clamp is ref/kernel.py:41's
            float q[4];
#pragma unroll
            for (int e = 0; e < 4; e++) q[e] = fminf(fmaxf(f[h][4 * j + e] * inv, -448.f), 448.f);
            int p = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
            p = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], p, true);
            out[j] = ok ? (uint32_t)p : 0u;
        }
        *(u32x4 *)(codes + (((size_t)mg * ks + s) * 2 + h) * 1024 + lane * 16) = out;
        const uint8_t sbyte = (uint8_t)((__float_as_uint(sc) >> 23) & 0xffu);
        if (ok && block == 128 && h == 0 && g == 0) scales[(size_t)row * ks + s] = sbyte;
        if (ok && block == 32 && (g & 1) == 0) scales[(size_t)row * (k >> 5) + 4 * s + 2 * h + (g >> 1)] = sbyte;
    }
}

// ---- GEMM ---------------------------------------------------------------------------------------

// WOPS: weights in MFMA operand order. Per group G of 16 columns and 128-K step s, the 64 lanes'
// 16-byte operand pieces lie in lane order: FP4 one kilobyte, lane r + 16 g holding bytes [16g,
// 16g + 16) of column 16 G + r's 64-byte step; FP8 two kilobytes, the first holding bytes [16g, 16g
// + 16) and the second [64 + 16g, 64 + 16g + 16) of the column's 128-byte step. Blocks run over the
// steps of a group, then over the groups, so a column group's weights stay one contiguous run and
// the packed array has the size of the codes. Byte offset of the block (G, s):
__device__ __forceinline__ size_t ops_block(int G, int s, int KS, bool fp4) {
    return ((size_t)G * KS + s) * (fp4 ? 1024 : 2048);
}

// codes [n][k / 2] (FP4) or [n][k] (FP8), n % 16 == 0, k % 128 == 0 -> the same codes in operand
// order. Thread t moves the 16-byte piece t of the packed array.
__global__ __launch_bounds__(256) void k_gemm_pack(const uint8_t *__restrict__ codes, uint8_t *__restrict__ packed,
                                                   int n, int k, int fp4, size_t pieces) {
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= pieces) return;
    const int KS = k >> 7, lane = (int)(t & 63), r = lane & 15, g = lane >> 4;
    size_t src;
    if (fp4) {
        const size_t blk = t >> 6;  // G * KS + s
        const size_t G = blk / KS, st = blk % KS;
        src = (16 * G + r) * (size_t)(k >> 1) + st * 64 + 16 * g;
    } else {
        const size_t blk = t >> 7, half = (t >> 6) & 1;  // (G * KS + s) * 2 + half
        const size_t G = blk / KS, st = blk % KS;
        src = (16 * G + r) * (size_t)k + st * 128 + 64 * half + 16 * g;
    }
    *(u32x4 *)(packed + 16 * t) = *(const u32x4 *)(codes + src);
}

// One workgroup owns a 16 MT x 16 NT output tile (MT m-tiles x NT n-tiles of 16 x 16, rows m0 ..) and
// a slice of up to NW * SW 128-K steps; wave w takes SW consecutive steps of the slice and accumulates
// its MT * NT tiles in registers, loading its activations and weights straight from global memory
// (no operand is shared between waves, so nothing is staged through LDS). All loads of a wave are
// issued before its first MFMA, from addresses clamped into the buffers; a step past the slice gets
// zero operands instead of a branch. The waves' tiles are summed through LDS in wave order. With one
// slice the workgroup writes Y; otherwise it writes its slice's partial tile and k_gemm_reduce adds
// the slices in order. (Summing the slices in the last workgroup to finish needs an agent-scope
// release/acquire per workgroup, which writes back and invalidates the XCD's L2 each time: measured
// at about 4x the whole GEMM, so the kernel boundary is the synchronization point.) The workgroup
// order is gemm_plan's. A rows are lda bytes apart. Partial tiles and the LDS sum hold f32x4
// q = t * 64 + lane with t = m-tile * NT + n-tile.
template <bool FP4W, int MT, int NT, int NW, int SW, bool WOPS>
__global__ __launch_bounds__(NW * 64) void k_gemm(const uint8_t *__restrict__ wc, const void *__restrict__ ws,
                                                  const uint8_t *__restrict__ aq, const uint8_t *__restrict__ as_,
                                                  f32x4 *__restrict__ part, void *__restrict__ y, int y_f32, int M,
                                                  int N, int K, int lda, int act_shift, int ntiles, int mgroups,
                                                  int slices, int steps_wg) {
    constexpr int kTileVecs = MT * NT * 64;
    constexpr int kThreads = NW * 64;
    __shared__ f32x4 red[NW * kTileVecs];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r = lane & 15, g = lane >> 4;
    const int u = blockIdx.x % (ntiles * mgroups), slice = blockIdx.x / (ntiles * mgroups);
    const int tile = u % ntiles, m0 = (u / ntiles) * 16 * MT;
    const int n0 = tile * 16 * NT, KS = K >> 7;
    const int wsteps = (steps_wg + NW - 1) / NW;
    const int s0 = slice * steps_wg + wave * wsteps;
    const int nst = max(0, min(wsteps, min(KS, (slice + 1) * steps_wg) - s0));  // wave-uniform

    // 1. loads: lane (r, g) holds, per step, rows 16 mt + r of A and columns n0 + 16 nt + r of W
    u32x4 av[SW][MT][2];
    uint32_t asc[SW][MT];
    u32x4 bv[SW][NT][FP4W ? 1 : 2];
    uint32_t bsc[SW][NT];
    float wsc[SW];
#pragma unroll
    for (int s = 0; s < SW; s++) {
        const size_t kb = (size_t)(s < nst ? s0 + s : 0) * 128;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int m = min(m0 + 16 * mt + r, M - 1);
            const uint8_t *row = aq + (size_t)m * lda + kb;
            av[s][mt][0] = *(const u32x4 *)(row + 16 * g);
            av[s][mt][1] = *(const u32x4 *)(row + 64 + 16 * g);
            asc[s][mt] = as_[(size_t)m * (K >> act_shift) + ((kb + 32 * g) >> act_shift)];
        }
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int n = min(n0 + 16 * nt + r, N - 1);
            if constexpr (WOPS) {  // operand order: one contiguous kilobyte (two for FP8) per load
                const uint8_t *blk = wc + ops_block(min((n0 >> 4) + nt, (N >> 4) - 1), (int)(kb >> 7), KS, FP4W) + 16 * lane;
                bv[s][nt][0] = *(const u32x4 *)blk;
                if constexpr (!FP4W) bv[s][nt][1] = *(const u32x4 *)(blk + 1024);
                if constexpr (FP4W) bsc[s][nt] = ((const uint8_t *)ws)[(size_t)n * (K >> 5) + (kb >> 5) + g];
            } else if constexpr (FP4W) {
                bv[s][nt][0] = *(const u32x4 *)(wc + (size_t)n * (K >> 1) + (kb >> 1) + 16 * g);
                bsc[s][nt] = ((const uint8_t *)ws)[(size_t)n * (K >> 5) + (kb >> 5) + g];
            } else {
                const uint8_t *row = wc + (size_t)n * K + kb;
                bv[s][nt][0] = *(const u32x4 *)(row + 16 * g);
                bv[s][nt][1] = *(const u32x4 *)(row + 64 + 16 * g);
            }
        }
        if constexpr (!FP4W) wsc[s] = ((const float *)ws)[(size_t)(n0 >> 7) * KS + (kb >> 7)];
    }
    // 2. MFMAs, 4 NT independent accumulators per step
    f32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const u32x4 z4 = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < SW; s++) {
        const bool live = s < nst;
        i32x8 b[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const u32x4 b0 = live ? bv[s][nt][0] : z4;
            if constexpr (FP4W) {
                b[nt] = i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], 0, 0, 0, 0};
            } else {
                const u32x4 b1 = live ? bv[s][nt][1] : z4;
                b[nt] = i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
            }
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const u32x4 a0 = live ? av[s][mt][0] : z4, a1 = live ? av[s][mt][1] : z4;
            const i32x8 a = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                if constexpr (FP4W) {
                    acc[mt][nt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b[nt], acc[mt][nt], 0, 4, 0,
                                                                                   (int)asc[s][mt], 0, (int)bsc[s][nt]);
                } else {
                    const f32x4 d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b[nt], f32x4{0.f, 0.f, 0.f, 0.f},
                                                                                      0, 0, 0, (int)asc[s][mt], 0, 127);
                    const float sw = live ? wsc[s] : 0.f;
#pragma unroll
                    for (int e = 0; e < 4; e++) acc[mt][nt][e] = fmaf(sw, d[e], acc[mt][nt][e]);
                }
            }
        }
    }
    // 3. the workgroup's sum, in wave order; thread tid takes q = tid + kThreads j
#pragma unroll
    for (int t = 0; t < MT * NT; t++) red[(wave * MT * NT + t) * 64 + lane] = acc[t / NT][t % NT];
    __syncthreads();
    constexpr int kPer = (kTileVecs + kThreads - 1) / kThreads;
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        const int q = tid + kThreads * j;
        if (q >= kTileVecs) break;
        f32x4 v = red[q];
#pragma unroll
        for (int w = 1; w < NW; w++) v += red[w * kTileVecs + q];
        if (slices > 1) {  // (split K only with mgroups == 1: u is the tile)
            part[((size_t)u * slices + slice) * kTileVecs + q] = v;
            continue;
        }
        // Y: element e of v is row 16 mt + 4 g' + e, column n0 + 16 nt + r' of the lane q % 64
        const int t = q >> 6, ql = q & 63, mt = t / NT, nt = t % NT;
        const int n = n0 + 16 * nt + (ql & 15);
        if (n >= N) continue;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = m0 + 16 * mt + 4 * (ql >> 4) + e;
            if (m >= M) continue;
            if (y_f32) ((float *)y)[(size_t)m * N + n] = v[e];
            else ((uint16_t *)y)[(size_t)m * N + n] = f32_to_bf16_bits(v[e]);
        }
    }
}

// Y = the slices' partial tiles added in slice order; thread i takes f32x4 i of every tile (the
// layout k_gemm stored them in), so partial reads are contiguous per slice.
template <int NT>
__global__ __launch_bounds__(256) void k_gemm_reduce(const f32x4 *__restrict__ part, int slices, int ntiles,
                                                     void *__restrict__ y, int y_f32, int M, int N) {
    constexpr int kTileVecs = 4 * NT * 64;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= ntiles * kTileVecs) return;
    const int tile = i / kTileVecs, q = i % kTileVecs;
    const f32x4 *tp = part + (size_t)tile * slices * kTileVecs + q;
    // slices are loaded up to 8 at a time, all loads issued before the first add (a plain loop waits
    // for each load in turn), and added in slice order
    constexpr int kBatch = 8;
    f32x4 s = tp[0];
    for (int sl0 = 1; sl0 < slices; sl0 += kBatch) {
        f32x4 v[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; i++)
            if (sl0 + i < slices) v[i] = tp[(size_t)(sl0 + i) * kTileVecs];
#pragma unroll
        for (int i = 0; i < kBatch; i++)
            if (sl0 + i < slices) s += v[i];
    }
    const int t = q >> 6, ql = q & 63, mt = t / NT, nt = t % NT;
    const int n = tile * 16 * NT + 16 * nt + (ql & 15);
    if (n >= N) return;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const int m = 16 * mt + 4 * (ql >> 4) + e;
        if (m >= M) continue;
        if (y_f32) ((float *)y)[(size_t)m * N + n] = s[e];
        else ((uint16_t *)y)[(size_t)m * N + n] = f32_to_bf16_bits(s[e]);
    }
}

// One-launch GEMM for K % 512 == 0: a workgroup owns a 16 MT x 16 NT output tile over all of K; wave w
// takes the 4 SW consecutive 128-K steps [4 SW w, 4 SW w + 4 SW) (waves past K do nothing), and the
// waves' tiles are summed through LDS in wave order, so the result does not depend on timing.
// Three things keep the loads, which bound this kernel, few and cheap (each measured):
//  - every load of a wave is issued before its first MFMA (a scheduling fence keeps the compiler
//    from interleaving waits with the loads);
//  - the operand loads alternate 64-byte halves: an MFMA operand load reads 16 rows x 64 bytes, all
//    in the same half of their 128-byte lines, which the vector L1 serves at half rate. Lanes of odd
//    rows (odd columns for W) read the other half first, and a per-lane select puts the halves back
//    in operand order. For FP4 W, whose step is 64 bytes, steps s and s + 1 of a column are the two
//    halves of one line, so steps come in pairs;
//  - scales are loaded four steps per instruction (one dword of A scale bytes per row with
//    act_block 128, 16 bytes per row or column for the per-32 scales), not one byte per step: a
//    one-byte wave load costs the L1 as much as a 1 KB one. The MFMA reads the low byte of its scale
//    operand, so each lane shifts its byte down.
template <bool FP4W, int MT, int NT, int NW, int QW, bool AARR, bool WOPS>
__global__ __launch_bounds__(NW * 64) void k_gemm_one(const uint8_t *__restrict__ wc, const void *__restrict__ ws,
                                                      const uint8_t *__restrict__ aq, const uint8_t *__restrict__ as_,
                                                      void *__restrict__ y, int y_f32, int M, int N, int K, int lda,
                                                      int act32, int ntiles) {
    constexpr int SW = 4 * QW;  // steps per wave
    constexpr int kTileVecs = MT * NT * 64;
    constexpr int kThreads = NW * 64;
    __shared__ f32x4 red[NW * kTileVecs];
    const int tid = threadIdx.x, lane = tid & 63, r = lane & 15, g = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool odd = r & 1;
    const int h0 = odd ? 64 : 0, h1 = 64 - h0;
    const int tile = blockIdx.x % ntiles, m0 = (blockIdx.x / ntiles) * 16 * MT;
    const int n0 = tile * 16 * NT, KS = K >> 7;
    const int s0 = wave * SW;
    const int nst = max(0, min(SW, KS - s0));  // wave-uniform; a multiple of 4

    f32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (nst > 0) {
        // 1. loads: lane (r, g) holds rows 16 mt + r of A and columns n0 + 16 nt + r of W; step
        // s < nst is step s0 + s of K (nst is a multiple of 4: KS % 4 == 0; steps past nst read
        // step s0 again and are not used). Issued in order of their latency:
        // the scales, then W (from HBM: a column tile's weights are first read by one of its row
        // groups), then A (the activations, resident in L2): 2048x7168 FP4 8.55 -> 8.15 us, FP8
        // 11.04 -> 10.60, 7168x2048 6.86 -> 6.33 against A, W, then the scales.
        u32x4 av[SW][MT][2];
        u32x4 bv[SW][NT][FP4W ? 1 : 2];
        u32x4 asw[QW][MT];  // A scale bytes: dword 0 (act_block 128) or 16 bytes (act_block 32)
        u32x4 bsw[QW][NT];  // FP4 W scale bytes, 16 per column per 4 steps
        float wsc[SW];      // FP8 W: the 128 x 128 block scale of each step
#pragma unroll
        for (int q = 0; q < QW; q++) {
            // groups of 4 steps past nst (the last wave of a K with KS % SW == 4) reload the last
            // group's words, in range, and are not used
            const int sq = s0 + 4 * min(q, (nst >> 2) - 1);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const size_t m = min(m0 + 16 * mt + r, M - 1);
                if (act32) asw[q][mt] = *(const u32x4 *)(as_ + m * (K >> 5) + 4 * sq);
                else asw[q][mt][0] = *(const uint32_t *)(as_ + m * KS + sq);
            }
            if constexpr (FP4W) {
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    bsw[q][nt] = *(const u32x4 *)((const uint8_t *)ws + (size_t)min(n0 + 16 * nt + r, N - 1) * (K >> 5) + 4 * sq);
            }
        }
#pragma unroll
        for (int s = 0; s < SW; s++) {
            const size_t kb = (size_t)(s < nst ? s0 + s : s0) * 128;
            if constexpr (WOPS) {  // operand order: steps s and s + 1 of a group are adjacent blocks
                if (!FP4W || s % 2 == 0) {
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        const uint8_t *blk = wc + ops_block(min((n0 >> 4) + nt, (N >> 4) - 1), (int)(kb >> 7), KS, FP4W) + 16 * lane;
                        bv[s][nt][0] = *(const u32x4 *)blk;
                        if constexpr (FP4W) bv[s + 1][nt][0] = *(const u32x4 *)(blk + 1024);
                        else bv[s][nt][1] = *(const u32x4 *)(blk + 1024);
                    }
                }
                if constexpr (!FP4W) wsc[s] = ((const float *)ws)[(size_t)(n0 >> 7) * KS + (kb >> 7)];
            } else if constexpr (FP4W) {
                if (s % 2 == 0) {
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        const uint8_t *row = wc + (size_t)min(n0 + 16 * nt + r, N - 1) * (K >> 1) + (kb >> 1);
                        bv[s][nt][0] = *(const u32x4 *)(row + h0 + 16 * g);
                        bv[s + 1][nt][0] = *(const u32x4 *)(row + h1 + 16 * g);
                    }
                }
            } else {
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    const uint8_t *row = wc + (size_t)min(n0 + 16 * nt + r, N - 1) * K + kb;
                    bv[s][nt][0] = *(const u32x4 *)(row + h0 + 16 * g);
                    bv[s][nt][1] = *(const u32x4 *)(row + h1 + 16 * g);
                }
                wsc[s] = ((const float *)ws)[(size_t)(n0 >> 7) * KS + (kb >> 7)];
            }
        }
#pragma unroll
        for (int s = 0; s < SW; s++) {
            const size_t kb = (size_t)(s < nst ? s0 + s : s0) * 128;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                if constexpr (AARR) {  // operand order (k_act_quant_e4m3_ops): two contiguous kilobytes
                    const uint8_t *blk = aq + (((size_t)((m0 >> 4) + mt) * KS + (kb >> 7)) * 2) * 1024 + lane * 16;
                    av[s][mt][0] = *(const u32x4 *)blk;
                    av[s][mt][1] = *(const u32x4 *)(blk + 1024);
                } else {
                    const uint8_t *row = aq + (size_t)min(m0 + 16 * mt + r, M - 1) * lda + kb;
                    av[s][mt][0] = *(const u32x4 *)(row + h0 + 16 * g);
                    av[s][mt][1] = *(const u32x4 *)(row + h1 + 16 * g);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // 2. halves back in operand order, then the MFMAs, NT independent accumulators per step
        // (steps past nst, in the last wave of a K with KS % SW == 4, take zero weights: a branch
        // there made the compiler wait for each step's loads before its MFMAs)
        const int gsh = 8 * g;
        const u32x4 z4 = {0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < SW; s++) {
            const bool live = SW == 4 || s < nst;  // SW == 4: nst is 0 or 4
            i32x8 b[NT];
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                if constexpr (FP4W) {
                    const u32x4 x0 = bv[s & ~1][nt][0], x1 = bv[s | 1][nt][0];
                    const u32x4 b0 = live ? (WOPS ? bv[s][nt][0] : (odd == (s & 1)) ? x0 : x1) : z4;
                    b[nt] = i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], 0, 0, 0, 0};
                } else {
                    const u32x4 x0 = bv[s][nt][0], x1 = bv[s][nt][1];
                    const bool sw = odd && !WOPS;  // operand-order weights need no half swap
                    const u32x4 b0 = live ? (sw ? x1 : x0) : z4, b1 = live ? (sw ? x0 : x1) : z4;
                    b[nt] = i32x8{(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
                }
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const u32x4 x0 = av[s][mt][0], x1 = av[s][mt][1];
                const u32x4 a0 = odd && !AARR ? x1 : x0, a1 = odd && !AARR ? x0 : x1;
                const i32x8 a = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
                const uint32_t aw = asw[s / 4][mt][act32 ? s % 4 : 0];
                const int ascale = (int)(act32 ? aw >> gsh : aw >> (8 * (s % 4)));
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    if constexpr (FP4W) {
                        const int bscale = (int)(bsw[s / 4][nt][s % 4] >> gsh);
                        acc[mt][nt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b[nt], acc[mt][nt], 0, 4, 0,
                                                                                       ascale, 0, bscale);
                    } else {
                        const f32x4 d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                            a, b[nt], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, ascale, 0, 127);
#pragma unroll
                        for (int e = 0; e < 4; e++) acc[mt][nt][e] = fmaf(wsc[s], d[e], acc[mt][nt][e]);
                    }
                }
            }
        }
    }
    // 3. the workgroup's sum in wave order (idle waves add zeros); thread tid takes q = tid + kThreads j
#pragma unroll
    for (int t = 0; t < MT * NT; t++) red[(wave * MT * NT + t) * 64 + lane] = acc[t / NT][t % NT];
    __syncthreads();
    constexpr int kPer = (kTileVecs + kThreads - 1) / kThreads;
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        const int q = tid + kThreads * j;
        if (q >= kTileVecs) break;
        f32x4 v = red[q];
#pragma unroll
        for (int w = 1; w < NW; w++) v += red[w * kTileVecs + q];
        // element e of v is row 16 mt + 4 g' + e, column n0 + 16 nt + r' of the lane q % 64
        const int t = q >> 6, ql = q & 63, mt = t / NT, nt = t % NT;
        const int n = n0 + 16 * nt + (ql & 15);
        if (n >= N) continue;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int m = m0 + 16 * mt + 4 * (ql >> 4) + e;
            if (m >= M) continue;
            if (y_f32) ((float *)y)[(size_t)m * N + n] = v[e];
            else ((uint16_t *)y)[(size_t)m * N + n] = f32_to_bf16_bits(v[e]);
        }
    }
}

// Tile shape and split of K, chosen per shape (each choice measured fastest for its shape):
//   variant 4, k_gemm_one with 32 x 64 tiles on 4 waves of 4 steps, when K % 512 == 0, K <= 2048, m > 32
//     and the tiles give >= 192 workgroups (7168 x 2048: 9.0 -> 6.6 us against variant 2);
//   variant 3, k_gemm_one with 16 x 32 tiles on up to 8 waves of 8 steps (FP4 weights: 8.2 -> 7.9 us
//     against 16 waves of 4, 8.9 with 4 waves of 16) or 16 waves of 4 steps (FP8), when K % 512 == 0,
//     K <= 8192, m > 32 and the tiles give >= 192 workgroups (2048 x 7168: 11.7 -> 8.3 us against
//     variant 0, and no partial tiles or second launch);
//   variant 2, 32 x 64 tiles (two workgroups per 64 columns when m > 32) and 16 waves of one step
//     each, when one slice covers K (<= 16 steps) and the tiles give >= 192 workgroups: per
//     workgroup 32 rows of activations and 64 columns of weights instead of 64 and 32 (7168 x 2048);
//   variant 1, 64 x 32 tiles and 16 waves of one step each, when one slice covers K and the tiles
//     alone give >= 192 workgroups (m <= 32 at 7168 x 2048: no partials and no second launch,
//     11.6 -> 9.3 us against variant 0);
//   variant 0 otherwise, 64 x 64 tiles and 8 waves of one step each, K split into slices of <= 8
//     steps, as many as it takes to give >= 200 workgroups (2048 x 7168: 7 slices, 224 workgroups;
//     against the earlier 4 waves of 2 steps, FP4 11.9 -> 11.6 us, FP8 12.7 -> 11.8 us).
// Workgroup b takes column tile u % ntiles and row group u / ntiles, u = b % (ntiles * mgroups), and
// slice b / (ntiles * mgroups): with ntiles % 8 == 0 the row groups and slices of a column tile run
// on one XCD.
struct GemmPlan {
    int variant, mt, nt, ntiles, mgroups, slices, steps;
};

// one_launch: variants 3 and 4 allowed (their scale loads need 16-byte aligned scale arrays).
static GemmPlan gemm_plan(int m, int n, int k, bool one_launch = true) {
    GemmPlan p;
    const int ks = k / 128;
    p.mgroups = 1;
    if (one_launch && ks % 4 == 0 && ks <= 16 && m > 32 && ((n + 63) / 64) * ((m + 31) / 32) >= 192) {
        p.variant = 4, p.mt = 2, p.nt = 4, p.ntiles = (n + 63) / 64, p.mgroups = (m + 31) / 32, p.slices = 1, p.steps = ks;
        return p;
    }
    if (one_launch && ks % 4 == 0 && ks <= 64 && m > 32 && ((n + 31) / 32) * ((m + 15) / 16) >= 192) {
        p.variant = 3, p.mt = 1, p.nt = 2, p.ntiles = (n + 31) / 32, p.mgroups = (m + 15) / 16, p.slices = 1, p.steps = ks;
        return p;
    }
    if (ks <= 16 && m > 32 && 2 * ((n + 63) / 64) >= 192) {
        p.variant = 2, p.mt = 2, p.nt = 4, p.ntiles = (n + 63) / 64, p.mgroups = 2, p.slices = 1, p.steps = ks;
        return p;
    }
    if (ks <= 16 && (n + 31) / 32 >= 192) {
        p.variant = 1, p.mt = 4, p.nt = 2, p.ntiles = (n + 31) / 32, p.slices = 1, p.steps = ks;
        return p;
    }
    p.variant = 0, p.mt = 4, p.nt = 4, p.ntiles = (n + 63) / 64;
    const int slices = std::max((ks + 7) / 8, std::min(ks, (200 + p.ntiles - 1) / p.ntiles));
    p.steps = (ks + slices - 1) / slices;
    p.slices = (ks + p.steps - 1) / p.steps;
    return p;
}

static uint64_t a256(uint64_t v) { return (v + 255) & ~(uint64_t)255; }

static uint64_t part_bytes(const GemmPlan &p) {
    return p.slices > 1 ? (uint64_t)p.ntiles * p.slices * (p.mt * p.nt * 64) * 16 : 0;
}

// Bytes the partial tiles take at the front of `work`: the larger of the plans for m and for m <= 32
// (the only way m changes the plan), so a workspace sized for m also serves every smaller m. Both
// are the plans without variants 3 and 4, which need no partials: a call whose scale arrays are not
// 16-byte aligned falls back to those plans.
static uint64_t part_reserve(int m, int n, int k) {
    return a256(std::max(part_bytes(gemm_plan(m, n, k, false)), part_bytes(gemm_plan(1, n, k, false))));
}

template <int MT, int NT, int NW, bool WOPS>
static hipError_t launch_gemm_t(const GemmPlan &p, int fmt, void *y, const void *codes, const void *scales,
                                const uint8_t *aq, int lda, const uint8_t *as_, int m, int n, int k, int shift,
                                int y_f32, f32x4 *part, hipStream_t st) {
    static_assert(MT == 4 || NW == 16, "split K (the reduce kernel) takes 64-row tiles only");
    const dim3 grid(p.ntiles * p.mgroups * p.slices);
    if (fmt == 0)
        hipLaunchKernelGGL((k_gemm<true, MT, NT, NW, 1, WOPS>), grid, dim3(NW * 64), 0, st, (const uint8_t *)codes, scales, aq,
                           as_, part, y, y_f32, m, n, k, lda, shift, p.ntiles, p.mgroups, p.slices, p.steps);
    else
        hipLaunchKernelGGL((k_gemm<false, MT, NT, NW, 1, WOPS>), grid, dim3(NW * 64), 0, st, (const uint8_t *)codes, scales, aq,
                           as_, part, y, y_f32, m, n, k, lda, shift, p.ntiles, p.mgroups, p.slices, p.steps);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && p.slices > 1) {
        hipLaunchKernelGGL(k_gemm_reduce<NT>, dim3(p.ntiles * (4 * NT * 64) / 256), dim3(256), 0, st, part, p.slices,
                           p.ntiles, y, y_f32, m, n);
        e = hipGetLastError();
    }
    return e;
}

// Requires p.steps <= the variant's steps per workgroup and p.slices * p.steps covering k / 128, and
// split K (slices > 1) only in variant 0; A rows lda bytes apart.
// arr: the activations are in operand order (k_act_quant_e4m3_ops; variants 3 and 4 only).
template <bool ARR, bool WOPS>
static hipError_t launch_gemm_one(const GemmPlan &p, int fmt, void *y, const void *codes, const void *scales,
                                  const uint8_t *aq, int lda, const uint8_t *as_, int m, int n, int k, int act_block,
                                  int y_f32, hipStream_t st) {
    const dim3 grid(p.ntiles * p.mgroups);
    const int a32 = act_block == 32;
    if (p.variant == 3 && fmt == 0)
        hipLaunchKernelGGL((k_gemm_one<true, 1, 2, 8, 2, ARR, WOPS>), grid, dim3(512), 0, st, (const uint8_t *)codes, scales, aq,
                           as_, y, y_f32, m, n, k, lda, a32, p.ntiles);
    else if (p.variant == 3)
        hipLaunchKernelGGL((k_gemm_one<false, 1, 2, 16, 1, ARR, WOPS>), grid, dim3(1024), 0, st, (const uint8_t *)codes, scales,
                           aq, as_, y, y_f32, m, n, k, lda, a32, p.ntiles);
    else if (fmt == 0)
        hipLaunchKernelGGL((k_gemm_one<true, 2, 4, 4, 1, ARR, WOPS>), grid, dim3(256), 0, st, (const uint8_t *)codes, scales, aq,
                           as_, y, y_f32, m, n, k, lda, a32, p.ntiles);
    else
        hipLaunchKernelGGL((k_gemm_one<false, 2, 4, 4, 1, ARR, WOPS>), grid, dim3(256), 0, st, (const uint8_t *)codes, scales,
                           aq, as_, y, y_f32, m, n, k, lda, a32, p.ntiles);
    return hipGetLastError();
}

template <bool WOPS>
static hipError_t launch_gemm_plan_w(const GemmPlan &p, int fmt, void *y, const void *codes, const void *scales,
                                     const uint8_t *aq, int lda, const uint8_t *as_, int m, int n, int k, int act_block,
                                     int y_f32, void *work, hipStream_t st, bool arr) {
    f32x4 *part = (f32x4 *)work;
    const int shift = act_block == 32 ? 5 : 7;
    if (p.variant >= 3)
        return arr ? launch_gemm_one<true, WOPS>(p, fmt, y, codes, scales, aq, lda, as_, m, n, k, act_block, y_f32, st)
                   : launch_gemm_one<false, WOPS>(p, fmt, y, codes, scales, aq, lda, as_, m, n, k, act_block, y_f32, st);
    if (p.variant == 0)
        return launch_gemm_t<4, 4, 8, WOPS>(p, fmt, y, codes, scales, aq, lda, as_, m, n, k, shift, y_f32, part, st);
    if (p.variant == 1)
        return launch_gemm_t<4, 2, 16, WOPS>(p, fmt, y, codes, scales, aq, lda, as_, m, n, k, shift, y_f32, part, st);
    return launch_gemm_t<2, 4, 16, WOPS>(p, fmt, y, codes, scales, aq, lda, as_, m, n, k, shift, y_f32, part, st);
}

// wops: the weight codes are in operand order (k_gemm_pack)
static hipError_t launch_gemm_plan(const GemmPlan &p, int fmt, void *y, const void *codes, const void *scales,
                                   const uint8_t *aq, int lda, const uint8_t *as_, int m, int n, int k, int act_block,
                                   int y_f32, void *work, hipStream_t st, bool arr = false, bool wops = false) {
    return wops ? launch_gemm_plan_w<true>(p, fmt, y, codes, scales, aq, lda, as_, m, n, k, act_block, y_f32, work, st, arr)
                : launch_gemm_plan_w<false>(p, fmt, y, codes, scales, aq, lda, as_, m, n, k, act_block, y_f32, work, st, arr);
}

// variants 3 and 4 load scale words 16 bytes at a time; unaligned scale arrays take the other plans
static GemmPlan plan_for(int fmt, const void *scales, const uint8_t *as_, int m, int n, int k) {
    return gemm_plan(m, n, k, aligned16(as_) && (fmt != 0 || aligned16(scales)));
}

static hipError_t launch_gemm(int fmt, void *y, const void *codes, const void *scales, const uint8_t *aq,
                              const uint8_t *as_, int m, int n, int k, int act_block, int y_f32, void *work,
                              hipStream_t st, bool wops = false) {
    return launch_gemm_plan(plan_for(fmt, scales, as_, m, n, k), fmt, y, codes, scales, aq, k, as_, m, n, k, act_block,
                            y_f32, work, st, false, wops);
}

// Rows of the activation codes in the workspace: a whole number of 16-row groups (operand order).
static uint64_t aq_bytes(int m, int k) { return a256((uint64_t)(m + 15) / 16 * 16 * k); }

static int check_gemm(const char *name, int fmt, const void *y, const void *codes, const void *scales, int m, int n,
                      int k, int act_block, const void *work) {
    if (fmt != 0 && fmt != 1) return abi_fail(hipErrorInvalidValue, "%s: unknown format %d", name, fmt);
    if (!y || !codes || !scales || !work) return abi_fail(hipErrorInvalidValue, "%s: null pointer", name);
    if (m < 1 || m > kGemmMaxM || n < 1 || n > kGemmMaxN || k < 128 || k % 128 || (act_block != 32 && act_block != 128))
        return abi_fail(hipErrorInvalidValue,
                        "%s: need 1 <= m <= 64, n <= %d, k %% 128 == 0, act_block 32 or 128 (m=%d n=%d k=%d)", name,
                        kGemmMaxN, m, n, k);
    if (!aligned16(codes) || !aligned16(work)) return abi_fail(hipErrorInvalidValue, "%s: codes and work must be 16-byte aligned", name);
    return 0;
}

}  // namespace stbl

using namespace stbl;

extern "C" {

uint64_t stbl_amd_gemm_work_bytes(int m, int n, int k) {
    if (m < 1 || n < 1 || k < 128) return 256;
    return part_reserve(m, n, k) + aq_bytes(m, k) + a256((uint64_t)m * (k / 32)) + 256;
}

}  // extern "C"

namespace stbl {

static int gemm_q_any(const char *name, bool wops, int fmt, void *y, const void *codes, const void *scales,
                      const void *aq, const void *as, int m, int n, int k, int act_block, int y_f32, void *work,
                      hipStream_t st) {
    if (int e = check_gemm(name, fmt, y, codes, scales, m, n, k, act_block, work)) return e;
    if (wops && n % 16) return abi_fail(hipErrorInvalidValue, "%s: packed weights need n %% 16 == 0 (n=%d)", name, n);
    if (!aq || !as || !aligned16(aq)) return abi_fail(hipErrorInvalidValue, "%s: aq (16-byte aligned) and as needed", name);
    return abi_status(launch_gemm(fmt, y, codes, scales, (const uint8_t *)aq, (const uint8_t *)as, m, n, k, act_block,
                                  y_f32, work, st, wops),
                      name);
}

static int gemm_any(const char *name, bool wops, int fmt, void *y, const void *codes, const void *scales,
                    const void *x, int m, int n, int k, int act_block, int y_f32, void *work, hipStream_t st) {
    if (int e = check_gemm(name, fmt, y, codes, scales, m, n, k, act_block, work)) return e;
    if (wops && n % 16) return abi_fail(hipErrorInvalidValue, "%s: packed weights need n %% 16 == 0 (n=%d)", name, n);
    if (!x || !aligned16(x)) return abi_fail(hipErrorInvalidValue, "%s: x must be 16-byte aligned", name);
    uint8_t *aq = (uint8_t *)work + part_reserve(m, n, k);
    uint8_t *as_ = aq + aq_bytes(m, k);
    // the one-launch plans read activations this call quantizes in operand order (one contiguous
    // kilobyte per load instead of 16 rows x 64 bytes)
    const GemmPlan p = plan_for(fmt, scales, as_, m, n, k);
    const bool arr = p.variant >= 3;
    if (arr) {
        hipLaunchKernelGGL(k_act_quant_e4m3_ops, dim3((m + 15) / 16 * (k / 128)), dim3(64), 0, st, (const uint16_t *)x, m,
                           k, act_block, aq, as_);
    } else {
        const int n8 = m * k / 8;
        hipLaunchKernelGGL(k_act_quant_e4m3, dim3((n8 + 255) / 256), dim3(256), 0, st, (const uint16_t *)x, n8, act_block,
                           aq, as_);
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess)
        e = launch_gemm_plan(p, fmt, y, codes, scales, aq, k, as_, m, n, k, act_block, y_f32, work, st, arr, wops);
    return abi_status(e, name);
}

}  // namespace stbl

extern "C" {

int stbl_amd_gemm_q(int fmt, void *y, const void *codes, const void *scales, const void *aq, const void *as, int m,
                    int n, int k, int act_block, int y_f32, void *work, hipStream_t st) {
    return gemm_q_any("gemm_q", false, fmt, y, codes, scales, aq, as, m, n, k, act_block, y_f32, work, st);
}

int stbl_amd_gemm(int fmt, void *y, const void *codes, const void *scales, const void *x, int m, int n, int k,
                  int act_block, int y_f32, void *work, hipStream_t st) {
    return gemm_any("gemm", false, fmt, y, codes, scales, x, m, n, k, act_block, y_f32, work, st);
}

int stbl_amd_gemm_pack(int fmt, void *packed, const void *codes, int n, int k, hipStream_t st) {
    if (fmt != 0 && fmt != 1) return abi_fail(hipErrorInvalidValue, "gemm_pack: unknown format %d", fmt);
    if (!packed || !codes || n < 16 || n % 16 || n > kGemmMaxN || k < 128 || k % 128)
        return abi_fail(hipErrorInvalidValue, "gemm_pack: need n %% 16 == 0 and k %% 128 == 0 (n=%d k=%d)", n, k);
    if (!aligned16(packed) || !aligned16(codes) || packed == codes)
        return abi_fail(hipErrorInvalidValue, "gemm_pack: codes and packed must be distinct 16-byte aligned buffers");
    const size_t pieces = (size_t)n * k / (fmt == 0 ? 32 : 16);
    hipLaunchKernelGGL(k_gemm_pack, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, st, (const uint8_t *)codes,
                       (uint8_t *)packed, n, k, fmt == 0 ? 1 : 0, pieces);
    return abi_status(hipGetLastError(), "gemm_pack launch");
}

int stbl_amd_gemm_q_packed(int fmt, void *y, const void *packed, const void *scales, const void *aq, const void *as,
                           int m, int n, int k, int act_block, int y_f32, void *work, hipStream_t st) {
    return gemm_q_any("gemm_q_packed", true, fmt, y, packed, scales, aq, as, m, n, k, act_block, y_f32, work, st);
}

int stbl_amd_gemm_packed(int fmt, void *y, const void *packed, const void *scales, const void *x, int m, int n, int k,
                         int act_block, int y_f32, void *work, hipStream_t st) {
    return gemm_any("gemm_packed", true, fmt, y, packed, scales, x, m, n, k, act_block, y_f32, work, st);
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
