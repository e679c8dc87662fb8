// Batch-1 (M <= 4 tokens) GEMVs over FP4 e2m1 and FP8 e4m3 weights, y[m][r] = sum_k x[m][k] W[r][k].
//
// Reference arithmetic: ref/kernel.py:85-102 (fp8_gemm / fp4_gemm: exact dequant, fp32 accumulate)
// and the engine kernels stbl/kernels.cu:92-191 that the C ABI names below replace.
//
// Work split (one design for every format): a workgroup owns R consecutive output rows and the
// whole K extent. Lane l of wave w owns one fixed K chunk, c = 64 w + l: 32 elements (16 bytes of
// FP4 codes, or one 17-byte GGUF block) or 16 elements (16 bytes of FP8 codes). The lane first
// issues all R row loads of its chunk (R independent 128-bit loads in flight per lane), then loads
// and widens its slice of x once and reuses it for the R rows, so x is read from L2 once per
// workgroup instead of once per row. Per row the lane forms the exact products of its chunk,
// applies the chunk's scale (exactly, a power of two, or the fp32 block scale), then the R partial
// sums are reduced over the 64 lanes with one transposed butterfly and over the waves through LDS
// in a fixed order, so results are deterministic run to run.
#include "common.hpp"
#include "abi_util.hpp"

namespace stbl {

constexpr int kMaxWaves = 8;  // K <= 8 * 64 chunks (512 threads, up to 256 VGPRs a lane)

// ---- x staging: the lane's chunk of x for M tokens, widened to fp32 -----------------------------

template <int M, int E>
struct XChunk {
    float v[M][E];
};

// bf16 x, E elements starting at element k0 of each token row (16-byte aligned).
template <int M, int E>
__device__ __forceinline__ void load_x_bf16(XChunk<M, E> &xc, const uint16_t *x, int k, int k0, bool active) {
#pragma unroll
    for (int t = 0; t < M; t++) {
        const u32x4 *p = (const u32x4 *)(x + (size_t)t * k + k0);
#pragma unroll
        for (int q = 0; q < E / 8; q++) {
            const u32x4 w = active ? p[q] : u32x4{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                xc.v[t][q * 8 + 2 * j] = bf16_lo(w[j]);
                xc.v[t][q * 8 + 2 * j + 1] = bf16_hi(w[j]);
            }
        }
    }
}

// fp32 x (the reference ABI's activation buffers), E elements from k0 (16-byte aligned).
template <int M, int E>
__device__ __forceinline__ void load_x_f32(XChunk<M, E> &xc, const float *x, int k, int k0, bool active) {
#pragma unroll
    for (int t = 0; t < M; t++) {
        const f32x4 *p = (const f32x4 *)(x + (size_t)t * k + k0);
#pragma unroll
        for (int q = 0; q < E / 4; q++) {
            const f32x4 w = active ? p[q] : f32x4{0.f, 0.f, 0.f, 0.f};
            xc.v[t][q * 4] = w.x, xc.v[t][q * 4 + 1] = w.y, xc.v[t][q * 4 + 2] = w.z, xc.v[t][q * 4 + 3] = w.w;
        }
    }
}

// ---- per-row partial products -------------------------------------------------------------------

// 32 FP4 values in OCP order (byte b: element 2b low nibble, 2b+1 high nibble) times x.
template <int M>
__device__ __forceinline__ void dot_fp4_ocp(float (&s)[M], const u32x4 w, const XChunk<M, 32> &xc) {
#pragma unroll
    for (int t = 0; t < M; t++) s[t] = 0.f;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const f32x2 a = e2m1x2<0>(w[d]), b = e2m1x2<1>(w[d]), c = e2m1x2<2>(w[d]), e = e2m1x2<3>(w[d]);
#pragma unroll
        for (int t = 0; t < M; t++) {
            const float *xv = &xc.v[t][8 * d];
            s[t] = fmaf(xv[0], a.x, s[t]);
            s[t] = fmaf(xv[1], a.y, s[t]);
            s[t] = fmaf(xv[2], b.x, s[t]);
            s[t] = fmaf(xv[3], b.y, s[t]);
            s[t] = fmaf(xv[4], c.x, s[t]);
            s[t] = fmaf(xv[5], c.y, s[t]);
            s[t] = fmaf(xv[6], e.x, s[t]);
            s[t] = fmaf(xv[7], e.y, s[t]);
        }
    }
}

// 32 FP4 values in GGUF block order (byte b: element b low nibble, 16+b high nibble) times x.
template <int M>
__device__ __forceinline__ void dot_fp4_gguf(float (&s)[M], const u32x4 w, const XChunk<M, 32> &xc) {
#pragma unroll
    for (int t = 0; t < M; t++) s[t] = 0.f;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const f32x2 a = e2m1x2<0>(w[d]), b = e2m1x2<1>(w[d]), c = e2m1x2<2>(w[d]), e = e2m1x2<3>(w[d]);
#pragma unroll
        for (int t = 0; t < M; t++) {
            const float *lo = &xc.v[t][4 * d], *hi = &xc.v[t][16 + 4 * d];
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
}

// 16 e4m3 values times x.
template <int M>
__device__ __forceinline__ void dot_fp8(float (&s)[M], const u32x4 w, const XChunk<M, 16> &xc) {
#pragma unroll
    for (int t = 0; t < M; t++) s[t] = 0.f;
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const f32x2 a = e4m3x2(w[d], false), b = e4m3x2(w[d], true);
#pragma unroll
        for (int t = 0; t < M; t++) {
            const float *xv = &xc.v[t][4 * d];
            s[t] = fmaf(xv[0], a.x, s[t]);
            s[t] = fmaf(xv[1], a.y, s[t]);
            s[t] = fmaf(xv[2], b.x, s[t]);
            s[t] = fmaf(xv[3], b.y, s[t]);
        }
    }
}

// ---- the reduction epilogue ---------------------------------------------------------------------

// part[t * R + r] of every lane -> out(t, row0 + r), summed over lanes and waves in a fixed order.
template <int M, int R, typename Store>
__device__ __forceinline__ void reduce_store(float (&part)[M * R], int row0, int rows, Store store) {
    constexpr int N = M * R;
    static_assert(N == 1 || N == 2 || N == 4 || N == 8, "M * R must be a power of two <= 8");
    __shared__ float red[kMaxWaves][N];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const float s = wave_sum_transposed<N>(part, lane);
    if (waves == 1) {
        if ((lane & (64 / N - 1)) == 0) {
            const int i = reduced_index<N>(lane), t = i / R, r = i % R;
            if (row0 + r < rows) store(t, row0 + r, s);
        }
        return;
    }
    if ((lane & (64 / N - 1)) == 0) red[wave][reduced_index<N>(lane)] = s;
    __syncthreads();
    if ((int)threadIdx.x < N) {
        const int i = threadIdx.x, t = i / R, r = i % R;
        float acc = red[0][i];
        for (int w = 1; w < waves; w++) acc += red[w][i];
        if (row0 + r < rows) store(t, row0 + r, acc);
    }
}

struct StoreBf16OrF32 {
    void *y;
    int rows, y_f32;
    __device__ void operator()(int t, int row, float v) const {
        if (y_f32) ((float *)y)[(size_t)t * rows + row] = v;
        else ((uint16_t *)y)[(size_t)t * rows + row] = f32_to_bf16_bits(v);
    }
};

struct StoreF32 {  // the reference ABI: fp32 output, bf16-rounded when `round`
    float *y;
    int round;
    __device__ void operator()(int, int row, float v) const { y[row] = round ? bf16_round(v) : v; }
};

// ---- FP4, OCP layout: codes [rows][k/2], e8m0 scales [rows][k/32]; x bf16 [M][k] -----------------

template <int M, int R>
__global__ __launch_bounds__(512) void k_gemv_fp4(void *__restrict__ y, const uint8_t *__restrict__ codes,
                                                   const uint8_t *__restrict__ scales, const uint16_t *__restrict__ x,
                                                   int rows, int k, int y_f32) {
    const int lane = threadIdx.x & 63, c = (threadIdx.x >> 6) * 64 + lane, G = k >> 5;
    const bool active = c < G;
    const int row0 = blockIdx.x * R;
    u32x4 w[R];
    uint32_t sc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = row0 + r;
        const bool ok = active && row < rows;
        w[r] = ok ? *(const u32x4 *)(codes + (size_t)row * (k >> 1) + (size_t)c * 16) : u32x4{0, 0, 0, 0};
        sc[r] = ok ? scales[(size_t)row * G + c] : 127u;
    }
    XChunk<M, 32> xc;
    load_x_bf16<M, 32>(xc, x, k, c * 32, active);
    float part[M * R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float s[M];
        dot_fp4_ocp<M>(s, w[r], xc);
        const float scale = e8m0_to_f32(sc[r]);
#pragma unroll
        for (int t = 0; t < M; t++) part[t * R + r] = s[t] * scale;
    }
    reduce_store<M, R>(part, row0, rows, StoreBf16OrF32{y, rows, y_f32});
}

// ---- FP8 e4m3 with fp32 scales per 128x128 block; x bf16 [M][k] ---------------------------------

template <int M, int R>
__global__ __launch_bounds__(512) void k_gemv_fp8(void *__restrict__ y, const uint8_t *__restrict__ codes,
                                                   const float *__restrict__ scales, const uint16_t *__restrict__ x,
                                                   int rows, int k, int y_f32) {
    static_assert(128 % R == 0, "a row tile must sit inside one 128-row scale block");
    const int lane = threadIdx.x & 63, c = (threadIdx.x >> 6) * 64 + lane;
    const int k0 = c * 16;
    const bool active = k0 < k;
    const int row0 = blockIdx.x * R;
    u32x4 w[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = row0 + r;
        w[r] = active && row < rows ? *(const u32x4 *)(codes + (size_t)row * k + k0) : u32x4{0, 0, 0, 0};
    }
    const int kb = (k + 127) >> 7;
    const float scale = active ? scales[(size_t)(row0 >> 7) * kb + (k0 >> 7)] : 0.f;
    XChunk<M, 16> xc;
    load_x_bf16<M, 16>(xc, x, k, k0, active);
    float part[M * R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float s[M];
        dot_fp8<M>(s, w[r], xc);
#pragma unroll
        for (int t = 0; t < M; t++) part[t * R + r] = s[t] * scale;
    }
    reduce_store<M, R>(part, row0, rows, StoreBf16OrF32{y, rows, y_f32});
}

// ---- reference ABI: FP8 with E8M0 scales per 32x32 block, fp32 x and y (stbl/kernels.cu:92-132) --

template <int R>
__global__ __launch_bounds__(512) void k_gemv_fp8_e8m0(float *__restrict__ y, const uint8_t *__restrict__ w8,
                                                        const uint8_t *__restrict__ scales, const float *__restrict__ x,
                                                        int rows, int k, int round_out) {
    static_assert(32 % R == 0, "a row tile must sit inside one 32-row scale block");
    const int lane = threadIdx.x & 63, c = (threadIdx.x >> 6) * 64 + lane;
    const int k0 = c * 16;
    const bool active = k0 < k;
    const int row0 = blockIdx.x * R;
    u32x4 w[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = row0 + r;
        w[r] = active && row < rows ? *(const u32x4 *)(w8 + (size_t)row * k + k0) : u32x4{0, 0, 0, 0};
    }
    const float scale = active ? e8m0_to_f32(scales[(size_t)(row0 >> 5) * (k >> 5) + (k0 >> 5)]) : 0.f;
    XChunk<1, 16> xc;
    load_x_f32<1, 16>(xc, x, k, k0, active);
    float part[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float s[1];
        dot_fp8<1>(s, w[r], xc);
        part[r] = s[0] * scale;
    }
    reduce_store<1, R>(part, row0, rows, StoreF32{y, round_out});
}

// ---- reference ABI: MXFP4 as GGUF 17-byte blocks, fp32 x, bf16-rounded fp32 y (kernels.cu:134-191)

constexpr int kMxBatch = 16;
struct MxBatch {
    float *y[kMxBatch];
    const uint8_t *w[kMxBatch];
    const float *x[kMxBatch];
};

// Block c of a row sits at byte 17 c, so it is only byte aligned: read the five dwords that cover
// it from the enclosing 4-byte boundary (every dword starts inside the buffer) and realign.
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

template <int R>
__global__ __launch_bounds__(512) void k_gemv_mxfp4_gguf(MxBatch b, int rows, int k) {
    float *y = b.y[blockIdx.y];
    const uint8_t *w = b.w[blockIdx.y];
    const float *x = b.x[blockIdx.y];
    const int lane = threadIdx.x & 63, c = (threadIdx.x >> 6) * 64 + lane, G = k >> 5;
    const bool active = c < G;
    const int row0 = blockIdx.x * R;
    u32x4 wc[R];
    uint32_t sc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int row = row0 + r;
        if (active && row < rows) {
            load_gguf_block(w + ((size_t)row * G + c) * 17, sc[r], wc[r]);
        } else {
            wc[r] = u32x4{0, 0, 0, 0};
            sc[r] = 127u;
        }
    }
    XChunk<1, 32> xc;
    load_x_f32<1, 32>(xc, x, k, c * 32, active);
    float part[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        float s[1];
        dot_fp4_gguf<1>(s, wc[r], xc);
        part[r] = s[0] * e8m0_to_f32(sc[r]);
    }
    reduce_store<1, R>(part, row0, rows, StoreF32{y, 1});
}

// ---- launchers ------------------------------------------------------------------------------------

static inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

template <int M>
static hipError_t launch_fp4(void *y, const void *codes, const void *scales, const void *x, int rows, int k,
                             int y_f32, hipStream_t st) {
    constexpr int R = 8 / M;
    const int waves = ceil_div(k / 32, 64);
    hipLaunchKernelGGL((k_gemv_fp4<M, R>), dim3(ceil_div(rows, R)), dim3(64 * waves), 0, st, y,
                       (const uint8_t *)codes, (const uint8_t *)scales, (const uint16_t *)x, rows, k, y_f32);
    return hipGetLastError();
}

template <int M>
static hipError_t launch_fp8(void *y, const void *codes, const float *scales, const void *x, int rows, int k,
                             int y_f32, hipStream_t st) {
    constexpr int R = 8 / M;
    const int waves = ceil_div(k / 16, 64);
    hipLaunchKernelGGL((k_gemv_fp8<M, R>), dim3(ceil_div(rows, R)), dim3(64 * waves), 0, st, y,
                       (const uint8_t *)codes, scales, (const uint16_t *)x, rows, k, y_f32);
    return hipGetLastError();
}

}  // namespace stbl

using namespace stbl;

extern "C" {

int stbl_amd_gemv_fp4(void *y, const void *codes, const void *scales, const void *x, int m, int rows, int k,
                      int y_f32, hipStream_t st) {
    if (!y || !codes || !scales || !x) return abi_fail(hipErrorInvalidValue, "gemv_fp4: null pointer");
    if (rows <= 0 || k <= 0 || k % 32 != 0 || k / 32 > kMaxWaves * 64)
        return abi_fail(hipErrorInvalidValue, "gemv_fp4: need k %% 32 == 0 and 0 < k <= 16384 (k=%d)", k);
    if (!aligned16(codes) || !aligned16(x)) return abi_fail(hipErrorInvalidValue, "gemv_fp4: codes and x must be 16-byte aligned");
    hipError_t e;
    switch (m) {
        case 1: e = launch_fp4<1>(y, codes, scales, x, rows, k, y_f32, st); break;
        case 2: e = launch_fp4<2>(y, codes, scales, x, rows, k, y_f32, st); break;
        case 3:
        case 4:
            // m = 3 runs as two launches of 2 tokens and 1 token; m = 4 as one launch.
            if (m == 4) { e = launch_fp4<4>(y, codes, scales, x, rows, k, y_f32, st); break; }
            e = launch_fp4<2>(y, codes, scales, x, rows, k, y_f32, st);
            if (e == hipSuccess)
                e = launch_fp4<1>((char *)y + (size_t)2 * rows * (y_f32 ? 4 : 2), codes, scales,
                                  (const uint16_t *)x + (size_t)2 * k, rows, k, y_f32, st);
            break;
        default: return abi_fail(hipErrorInvalidValue, "gemv_fp4: m must be 1..4 (m=%d); use the GEMM for more", m);
    }
    return abi_status(e, "gemv_fp4 launch");
}

int stbl_amd_gemv_fp8(void *y, const void *codes, const float *scales, const void *x, int m, int rows, int k,
                      int y_f32, hipStream_t st) {
    if (!y || !codes || !scales || !x) return abi_fail(hipErrorInvalidValue, "gemv_fp8: null pointer");
    if (rows <= 0 || k <= 0 || k % 16 != 0 || k / 16 > kMaxWaves * 64)
        return abi_fail(hipErrorInvalidValue, "gemv_fp8: need k %% 16 == 0 and 0 < k <= 8192 (k=%d)", k);
    if (!aligned16(codes) || !aligned16(x)) return abi_fail(hipErrorInvalidValue, "gemv_fp8: codes and x must be 16-byte aligned");
    hipError_t e;
    switch (m) {
        case 1: e = launch_fp8<1>(y, codes, scales, x, rows, k, y_f32, st); break;
        case 2: e = launch_fp8<2>(y, codes, scales, x, rows, k, y_f32, st); break;
        case 3:
        case 4:
            if (m == 4) { e = launch_fp8<4>(y, codes, scales, x, rows, k, y_f32, st); break; }
            e = launch_fp8<2>(y, codes, scales, x, rows, k, y_f32, st);
            if (e == hipSuccess)
                e = launch_fp8<1>((char *)y + (size_t)2 * rows * (y_f32 ? 4 : 2), codes, scales,
                                  (const uint16_t *)x + (size_t)2 * k, rows, k, y_f32, st);
            break;
        default: return abi_fail(hipErrorInvalidValue, "gemv_fp8: m must be 1..4 (m=%d); use the GEMM for more", m);
    }
    return abi_status(e, "gemv_fp8 launch");
}

// stbl/kernels.h:14-15. Requires k % 32 == 0 and 16-byte aligned rows, as the reference does.
void stbl_gemv_fp8(float *y, const void *w, const void *scale, const float *x, int rows, int k, int round_out,
                   hipStream_t st) {
    if (!y || !w || !scale || !x || rows <= 0 || k <= 0 || k % 32 != 0 || k / 16 > kMaxWaves * 64 || !aligned16(w) ||
        !aligned16(x)) {
        abi_fail(hipErrorInvalidValue, "stbl_gemv_fp8: bad arguments (rows=%d k=%d)", rows, k);
        return;
    }
    constexpr int R = 8;
    hipLaunchKernelGGL((k_gemv_fp8_e8m0<R>), dim3(ceil_div(rows, R)), dim3(64 * ceil_div(k / 16, 64)), 0, st, y,
                       (const uint8_t *)w, (const uint8_t *)scale, x, rows, k, round_out);
    abi_status(hipGetLastError(), "stbl_gemv_fp8 launch");
}

// stbl/kernels.h:19-20. n <= 16 same-shape matrices in one launch; needs k % 256 == 0 and w 8-byte
// aligned (the reference's preconditions, stbl/kernels.cu:138-139).
void stbl_gemv_mxfp4_batch(float *const *y, const void *const *w, const float *const *x, int n, int rows, int k,
                           hipStream_t st) {
    if (!y || !w || !x || n <= 0 || n > kMxBatch || rows <= 0 || k <= 0 || k % 256 != 0 || k / 32 > kMaxWaves * 64) {
        abi_fail(hipErrorInvalidValue, "stbl_gemv_mxfp4_batch: bad arguments (n=%d rows=%d k=%d)", n, rows, k);
        return;
    }
    MxBatch b = {};
    for (int j = 0; j < n; j++) {
        if (!y[j] || !w[j] || !x[j] || ((uintptr_t)w[j] & 7) || !aligned16(x[j])) {
            abi_fail(hipErrorInvalidValue, "stbl_gemv_mxfp4_batch: matrix %d: null or misaligned pointer", j);
            return;
        }
        b.y[j] = y[j], b.w[j] = (const uint8_t *)w[j], b.x[j] = x[j];
    }
    constexpr int R = 8;
    hipLaunchKernelGGL((k_gemv_mxfp4_gguf<R>), dim3(ceil_div(rows, R), n), dim3(64 * ceil_div(k / 32, 64)), 0, st, b,
                       rows, k);
    abi_status(hipGetLastError(), "stbl_gemv_mxfp4_batch launch");
}

// stbl/kernels.h:16.
void stbl_gemv_mxfp4(float *y, const void *w, const float *x, int rows, int k, hipStream_t st) {
    stbl_gemv_mxfp4_batch(&y, &w, &x, 1, rows, k, st);
}

}  // extern "C"
