// Decode GEMVs over FP4 e2m1 and FP8 e4m3 weights: y[t][r] = sum_k x[t][k] * Wdeq[r][k], M <= 4 rows
// of activations (tokens).
//
// Reference arithmetic: ref/kernel.py:85-102 (fp8_gemm / fp4_gemm: exact dequant, fp32 accumulate)
// and the engine kernels stbl/kernels.cu:92-191 whose C-ABI names are exported at the end.
//
// Work split (one design for every weight format): a workgroup owns R consecutive output rows and
// the whole K extent. Lane l of wave w owns one fixed K chunk c = 64 w + l of CH elements (16 bytes
// of FP4 codes, one 17-byte GGUF block, or 16 bytes of FP8 codes), so one wave-wide load of one row
// reads a contiguous kilobyte. Each lane
//   1. issues its x chunk loads and then all R row loads at once, from addresses clamped into the
//      buffers (lanes past K or rows past the matrix read row 0 / chunk 0 and are masked later), so
//      no load sits behind a branch and every load of the workgroup is in flight together;
//   2. forms the exact products of each row's chunk (bf16 x times a converted weight is exact in
//      fp32), applies the chunk's scale (E8M0: exact; FP8 block scale: one fp32 multiply), and
//      masks dead lanes;
//   3. reduces each (token, row) partial over the 64 lanes with DPP moves only, and over the waves
//      through LDS in wave order, so the result is the same on every run.
#include "abi_util.hpp"
#include "common.hpp"

namespace stbl {

constexpr int kMaxWaves = 8;  // K <= 512 chunks: 16384 FP4 / 8192 FP8 elements
constexpr int kMaxJobs = 16;  // matrices per launch (the reference's kMxBatch, stbl/kernels.h:18)

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
// aligned dword never crosses a page) and realign with v_alignbyte.
__device__ __forceinline__ void load_gguf_block(const uint8_t *blk, uint32_t &scale, u32x4 &codes) {
    const uintptr_t a = (uintptr_t)blk;
    const uint32_t *d = (const uint32_t *)(a & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)(a & 3);
    uint32_t v[5];
#pragma unroll
    for (int i = 0; i < 5; i++) v[i] = d[i];
    scale = (v[0] >> (8 * sh)) & 0xffu;
    const uint32_t off = sh + 1;  // first code byte, 1..4 bytes past d
#pragma unroll
    for (int j = 0; j < 4; j++) codes[j] = off == 4 ? v[j + 1] : __builtin_amdgcn_alignbyte(v[j + 1], v[j], off);
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

// sum over the chunk of x * (unscaled) weight, for each token.
template <WFmt F, int M, int CH>
__device__ __forceinline__ void chunk_dot(float (&s)[M], const u32x4 w, const float (&xf)[M][CH]) {
#pragma unroll
    for (int t = 0; t < M; t++) s[t] = 0.f;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        if constexpr (WTraits<F>::fp4) {
            const f32x2 a = e2m1x2<0>(w[d]), b = e2m1x2<1>(w[d]), c = e2m1x2<2>(w[d]), e = e2m1x2<3>(w[d]);
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

template <WFmt F, bool XF32, int M, int R>
__global__ __launch_bounds__(512) void k_gemv(GemvJobs jobs, int rows, int k, int out_mode) {
    using T = WTraits<F>;
    constexpr int CH = T::CH;
    static_assert(32 % R == 0, "a row tile must sit inside one scale block");
    const GemvJob J = jobs.j[blockIdx.y];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const int nch = k / CH, c = wave * 64 + lane;
    const bool active = c < nch;
    const int cc = active ? c : 0;
    const int row0 = blockIdx.x * R;

    // 1. loads: x first (it is needed by every row), then every row of the tile
    float xf[M][CH];
    load_x<XF32, M, CH>(xf, J.x, k, cc * CH);
    u32x4 w[R];
    uint32_t sb[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const size_t row = (size_t)min(row0 + r, rows - 1);
        if constexpr (F == WFmt::FP4_OCP) {
            w[r] = *(const u32x4 *)(J.w + row * (k >> 1) + (size_t)cc * 16);
            sb[r] = ((const uint8_t *)J.s)[row * nch + cc];
        } else if constexpr (F == WFmt::FP4_GGUF) {
            load_gguf_block(J.w + (row * nch + cc) * 17, sb[r], w[r]);
        } else {
            w[r] = *(const u32x4 *)(J.w + row * k + (size_t)cc * 16);
        }
    }
    float lscale = 1.f;  // FP8: one block scale per lane for the whole tile
    if constexpr (F == WFmt::FP8_B128)
        lscale = ((const float *)J.s)[(size_t)(row0 >> 7) * ((k + 127) >> 7) + ((cc * 16) >> 7)];
    uint32_t lsb = 0;
    if constexpr (F == WFmt::FP8_E8M0) lsb = ((const uint8_t *)J.s)[(size_t)(row0 >> 5) * (k >> 5) + ((cc * 16) >> 5)];

    // 2. products, scales, masking; 3. lane reduction
    __shared__ float red[kMaxWaves][M * R];
    float tot[M * R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float s[M];
        chunk_dot<F, M, CH>(s, w[r], xf);
        float scale;
        if constexpr (T::fp4) scale = e8m0_to_f32(sb[r]);
        else if constexpr (F == WFmt::FP8_B128) scale = lscale;
        else scale = e8m0_to_f32(lsb);
#pragma unroll
        for (int t = 0; t < M; t++) tot[t * R + r] = dpp_sum(active ? s[t] * scale : 0.f);
    }
    auto store = [&](int i, float v) {
        const int t = i / R, r = i % R;
        if (row0 + r >= rows) return;
        const size_t at = (size_t)t * rows + row0 + r;
        if (out_mode == OUT_BF16) ((uint16_t *)J.y)[at] = f32_to_bf16_bits(v);
        else if (out_mode == OUT_F32) ((float *)J.y)[at] = v;
        else ((float *)J.y)[at] = bf16_round(v);
    };
    if (waves == 1) {
        if (lane == 63) {
#pragma unroll
            for (int i = 0; i < M * R; i++) store(i, tot[i]);
        }
        return;
    }
    if (lane == 63) {
#pragma unroll
        for (int i = 0; i < M * R; i++) red[wave][i] = tot[i];
    }
    __syncthreads();
    if ((int)threadIdx.x < M * R) {
        const int i = threadIdx.x;
        float acc = red[0][i];
        for (int v = 1; v < waves; v++) acc += red[v][i];
        store(i, acc);
    }
}

static inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

template <WFmt F, bool XF32, int M>
static hipError_t launch(const GemvJobs &jobs, int njobs, int rows, int k, int out_mode, hipStream_t st) {
    constexpr int R = M <= 2 ? 2 : 1;
    const int waves = ceil_div(k / WTraits<F>::CH, 64);
    hipLaunchKernelGGL((k_gemv<F, XF32, M, R>), dim3(ceil_div(rows, R), njobs), dim3(64 * waves), 0, st, jobs, rows,
                       k, out_mode);
    return hipGetLastError();
}

// v2 dispatch over the token count.
template <WFmt F>
static int gemv_v2(const char *name, void *y, const void *w, const void *s, const void *x, int m, int rows, int k,
                   int y_f32, hipStream_t st) {
    constexpr int CH = WTraits<F>::CH;
    if (!y || !w || !s || !x) return abi_fail(hipErrorInvalidValue, "%s: null pointer", name);
    if (rows <= 0 || k <= 0 || k % CH != 0 || k / CH > kMaxWaves * 64)
        return abi_fail(hipErrorInvalidValue, "%s: need k %% %d == 0 and 0 < k <= %d (k=%d)", name, CH,
                        kMaxWaves * 64 * CH, k);
    if (m < 1 || m > 4) return abi_fail(hipErrorInvalidValue, "%s: m must be 1..4 (m=%d); use the GEMM for more", name, m);
    if (!aligned16(w) || !aligned16(x)) return abi_fail(hipErrorInvalidValue, "%s: weights and x must be 16-byte aligned", name);
    GemvJobs jobs = {};
    jobs.j[0] = GemvJob{(const uint8_t *)w, s, x, y};
    const int mode = y_f32 ? OUT_F32 : OUT_BF16;
    hipError_t e;
    switch (m) {
        case 1: e = launch<F, false, 1>(jobs, 1, rows, k, mode, st); break;
        case 2: e = launch<F, false, 2>(jobs, 1, rows, k, mode, st); break;
        case 3: e = launch<F, false, 3>(jobs, 1, rows, k, mode, st); break;
        default: e = launch<F, false, 4>(jobs, 1, rows, k, mode, st); break;
    }
    return abi_status(e, name);
}

}  // namespace stbl

using namespace stbl;

extern "C" {

int stbl_amd_gemv_fp4(void *y, const void *codes, const void *scales, const void *x, int m, int rows, int k,
                      int y_f32, hipStream_t st) {
    return gemv_v2<WFmt::FP4_OCP>("gemv_fp4", y, codes, scales, x, m, rows, k, y_f32, st);
}

int stbl_amd_gemv_fp8(void *y, const void *codes, const float *scales, const void *x, int m, int rows, int k,
                      int y_f32, hipStream_t st) {
    return gemv_v2<WFmt::FP8_B128>("gemv_fp8", y, codes, scales, x, m, rows, k, y_f32, st);
}

// stbl/kernels.h:14-15. Requires k % 32 == 0 and 16-byte aligned rows, as the reference does.
void stbl_gemv_fp8(float *y, const void *w, const void *scale, const float *x, int rows, int k, int round_out,
                   hipStream_t st) {
    if (!y || !w || !scale || !x || rows <= 0 || k <= 0 || k % 32 != 0 || k / 16 > kMaxWaves * 64 || !aligned16(w) ||
        !aligned16(x)) {
        abi_fail(hipErrorInvalidValue, "stbl_gemv_fp8: bad arguments (rows=%d k=%d)", rows, k);
        return;
    }
    GemvJobs jobs = {};
    jobs.j[0] = GemvJob{(const uint8_t *)w, scale, x, y};
    abi_status(launch<WFmt::FP8_E8M0, true, 1>(jobs, 1, rows, k, round_out ? OUT_F32_ROUNDED : OUT_F32, st),
               "stbl_gemv_fp8 launch");
}

// stbl/kernels.h:19-20. n <= 16 same-shape matrices in one launch; needs k % 256 == 0 and w 8-byte
// aligned (the reference's preconditions, stbl/kernels.cu:138-139). y, w, x are host arrays.
void stbl_gemv_mxfp4_batch(float *const *y, const void *const *w, const float *const *x, int n, int rows, int k,
                           hipStream_t st) {
    if (!y || !w || !x || n <= 0 || n > kMaxJobs || rows <= 0 || k <= 0 || k % 256 != 0 || k / 32 > kMaxWaves * 64) {
        abi_fail(hipErrorInvalidValue, "stbl_gemv_mxfp4_batch: bad arguments (n=%d rows=%d k=%d)", n, rows, k);
        return;
    }
    GemvJobs jobs = {};
    for (int j = 0; j < n; j++) {
        if (!y[j] || !w[j] || !x[j] || ((uintptr_t)w[j] & 7) || !aligned16(x[j])) {
            abi_fail(hipErrorInvalidValue, "stbl_gemv_mxfp4_batch: matrix %d: null or misaligned pointer", j);
            return;
        }
        jobs.j[j] = GemvJob{(const uint8_t *)w[j], nullptr, x[j], y[j]};
    }
    abi_status(launch<WFmt::FP4_GGUF, true, 1>(jobs, n, rows, k, OUT_F32_ROUNDED, st), "stbl_gemv_mxfp4_batch launch");
}

// stbl/kernels.h:16.
void stbl_gemv_mxfp4(float *y, const void *w, const float *x, int rows, int k, hipStream_t st) {
    stbl_gemv_mxfp4_batch(&y, &w, &x, 1, rows, k, st);
}

}  // extern "C"
