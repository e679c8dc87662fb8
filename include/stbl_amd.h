/*
 * libstbl_amd.so -- MI355X (gfx950) quantized expert-GEMV path, C ABI.
 *
 * Two surfaces:
 *  1. The reference's operator names and signatures (stbl/kernels.h), so existing ctypes call sites
 *     (stbl/bench_gemv.py:40,48, stbl/test_kernels.py:68,95-97,114-116,206) bind unchanged:
 *     fp32 activation buffers holding bf16-representable values, raw weight bytes, a stream last.
 *     These return void, as the reference's do; a failure is recorded per thread and read with
 *     stbl_amd_last_error().
 *  2. v2 entry points (prefix stbl_amd_) for the formats of the path's configurations: bf16
 *     activations, FP8 e4m3 with fp32 128x128 block scales, FP4 e2m1 in the OCP packing (element 2i
 *     in the low nibble) with E8M0 scales per 32 along K. They return 0 on success or a negative
 *     hipError_t, and also record the failure for stbl_amd_last_error().
 *
 * Conventions: every pointer argument except host arrays named as such is device memory allocated
 * by the caller; no entry point allocates device memory unless it says so. `st` is a hipStream_t
 * (NULL = the null stream). bf16 buffers are arrays of uint16 bit patterns. Every kernel is
 * stateless, so entry points may be called concurrently on different streams.
 */
#ifndef STBL_AMD_H
#define STBL_AMD_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- reference surface (stbl/kernels.h) ---------------------------------------------------------- */

/* stbl/kernels.h:9 -- in place, per 32 values: s = 2^ceil(log2(max(amax,1e-4)/448)),
 * x = bf16(e4m3(x/s)*s). n % 32 == 0. */
void stbl_act_quant_fp8(float *x, int n, hipStream_t st);

/* stbl/kernels.h:11 -- x = bf16(x) in place. */
void stbl_round_bf16(float *x, int n, hipStream_t st);

/* stbl/kernels.h:14-15 -- y[r] = sum_k x[k] * e4m3(w[r][k]) * 2^(scale[r/32][k/32]-127); y rounded
 * to bf16 when round_out. w [rows][k] e4m3, scale E8M0 [(rows+31)/32][k/32], x fp32 [k], y fp32
 * [rows]. k % 32 == 0, k <= 8192, w and x 16-byte aligned. */
void stbl_gemv_fp8(float *y, const void *w, const void *scale, const float *x, int rows, int k, int round_out,
                   hipStream_t st);

/* stbl/kernels.h:16 -- MXFP4 rows of GGUF 17-byte blocks ([E8M0][16 bytes: element i low nibble,
 * 16+i high nibble]); y = bf16(W x) stored as fp32. k % 256 == 0, k <= 16384, w 8-byte aligned. */
void stbl_gemv_mxfp4(float *y, const void *w, const float *x, int rows, int k, hipStream_t st);

/* stbl/kernels.h:18-20 -- n <= 16 same-shape stbl_gemv_mxfp4 products in one launch. y, w and x are
 * HOST arrays of n device pointers. */
enum { kMxBatch = 16 };
void stbl_gemv_mxfp4_batch(float *const *y, const void *const *w, const float *const *x, int n, int rows, int k,
                           hipStream_t st);

/* stbl/kernels.h:35 -- out = bf16(silu(min(g,lim)) * clamp(u,-lim,lim) * weight); no clamp if
 * limit <= 0. */
void stbl_swiglu(float *out, const float *g, const float *u, float weight, float limit, int n, hipStream_t st);

/* stbl/kernels.h:37-38 -- count <= 16 consecutive n-long segments, segment j scaled by weights[j]
 * (a HOST array). */
void stbl_swiglu_batch(float *out, const float *g, const float *u, const float *weights, int count, float limit, int n,
                       hipStream_t st);

/* stbl/kernels.h:39 -- y += a * x (fp32). */
void stbl_axpy(float *y, const float *x, float a, int n, hipStream_t st);

/* ---- v2: quantized GEMV (ref/kernel.py:85-102 with M <= 4 activation rows) ------------------------- */

/* y[m][rows] = x[m][k] . Wdeq^T with fp32 accumulation, Wdeq = e2m1(codes) * 2^(scales-127).
 * codes [rows][k/2] (OCP nibble order), scales E8M0 [rows][k/32], x bf16 [m][k], y bf16 [m][rows]
 * (fp32 when y_f32). 1 <= m <= 4, k % 32 == 0, k <= 16384, codes and x 16-byte aligned.
 * Replaces fp4_gemm (ref/kernel.py:94-102) with unit activation scales and, for the engine,
 * stbl_gemv_mxfp4 (stbl/kernels.h:16). */
int stbl_amd_gemv_fp4(void *y, const void *codes, const void *scales, const void *x, int m, int rows, int k,
                      int y_f32, hipStream_t st);

/* y[m][rows] = x[m][k] . Wdeq^T, Wdeq = e4m3(codes) * scales[r/128][k/128] (fp32 scales,
 * [ceil(rows/128)][ceil(k/128)]). 1 <= m <= 4, k % 16 == 0, k <= 8192, codes and x 16-byte aligned.
 * Replaces fp8_gemm (ref/kernel.py:85-91) and stbl_gemv_fp8 (stbl/kernels.h:14-15). */
int stbl_amd_gemv_fp8(void *y, const void *codes, const float *scales, const void *x, int m, int rows, int k,
                      int y_f32, hipStream_t st);

/* ---- v2: quantizers and dequantizers ----------------------------------------------------------------- */

/* act_quant (ref/kernel.py:35-45) on bf16 x [rows][n]: per `block` values amax >= 1e-4,
 * t = amax * fp32(1/448), s = pow2 ? 2^ceil(log2 t) : t, codes = e4m3(clamp(x/s, +-448)).
 * Outputs (each optional): codes e4m3 [rows][n], scales fp32 [rows][n/block], deq bf16 [rows][n]
 * = bf16(e4m3 * s) (the inplace=True form). */
int stbl_amd_act_quant(const void *x, int rows, int n, int block, int pow2, void *codes, float *scales, void *deq,
                       hipStream_t st);

/* FP4 weight quantization: fp4_act_quant(w, 32) E8M0 path (ref/kernel.py:55-72) on w fp32
 * [rows][k]: s = 2^ceil(log2(max(amax, 6*2^-126)/6)), codes = e2m1_rne(clamp(w/s, +-6)).
 * codes [rows][k/2], scales E8M0 bytes [rows][k/32]. k % 32 == 0. */
int stbl_amd_quant_fp4(void *codes, void *scales, const float *w, int rows, int k, hipStream_t st);

/* FP8 weight quantization with one fp32 scale per 128x128 block: s = max(amax, 1e-4) / 448,
 * codes = e4m3_rne(clamp(w/s, +-448)). scales [ceil(rows/128)][ceil(k/128)]. No reference function
 * quantizes 128x128 weights; this follows the configs' definition with act_quant's clamp. */
int stbl_amd_quant_fp8_b128(void *codes, float *scales, const float *w, int rows, int k, hipStream_t st);

/* out fp32 [rows][k] = e2m1(code) * 2^(s-127), one fp32 product per element (ref/kernel.py:98-101). */
int stbl_amd_dequant_fp4(float *out, const void *codes, const void *scales, int rows, int k, hipStream_t st);

/* out fp32 [rows][k] from GGUF MXFP4 17-byte blocks (tools/convert_official.py:187-201 layout). */
int stbl_amd_dequant_gguf17(float *out, const void *w, int rows, int k, hipStream_t st);

/* out fp32 [rows][k] = e4m3(code) * scale (ref/kernel.py:89-90): fp32 128x128 scales, or with
 * scale_e8m0 the reference engine's E8M0 bytes per 32x32 block [(rows+31)/32][k/32]. */
int stbl_amd_dequant_fp8(float *out, const void *codes, const void *scales, int rows, int k, int scale_e8m0,
                         hipStream_t st);

/* ---- library ------------------------------------------------------------------------------------------ */

/* The calling thread's last failure: copies its message into buf (len bytes, may be NULL), clears
 * it, returns its hipError_t code (0 if none). No reference counterpart (the reference never checks
 * launches, stbl/kernels.cu:545-640). */
int stbl_amd_last_error(char *buf, int len);

/* ABI version of this library. */
int stbl_amd_version(void);

#ifdef __cplusplus
}
#endif

#endif /* STBL_AMD_H */
