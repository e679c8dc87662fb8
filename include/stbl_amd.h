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
 * [rows]. Scale bytes decode as the engine's (stbl/kernels.cu:32): 0 -> 0.0, 255 -> +Inf times the
 * 32-block's sum. k % 32 == 0 (any k), w and x 16-byte aligned. */
void stbl_gemv_fp8(float *y, const void *w, const void *scale, const float *x, int rows, int k, int round_out,
                   hipStream_t st);

/* stbl/kernels.h:16 -- MXFP4 rows of GGUF 17-byte blocks ([E8M0][16 bytes: element i low nibble,
 * 16+i high nibble]); y = bf16(W x) stored as fp32. Scale bytes decode as the engine's
 * (stbl/kernels.cu:32, :185): 0 -> 0.0, 255 -> +Inf times the block's sum. k % 256 == 0 (any k), w
 * 8-byte aligned. */
void stbl_gemv_mxfp4(float *y, const void *w, const float *x, int rows, int k, hipStream_t st);

/* y[r] = sum_i x_r[i] * w[r][i] in fp32 (bf16-rounded when round_out), bf16 weights [rows][k]; x_r = x
 * + (r / group_rows) * k when group_rows > 0, else x. Replaces stbl_gemv_bf16 (stbl/kernels.h:21-22,
 * stbl/kernels.cu:193-204): the attention output projection (grouped) and the head. */
void stbl_gemv_bf16(float *y, const void *w, const float *x, int rows, int k, int round_out, int group_rows,
                    hipStream_t st);

/* y[r] = sum_k x[k] * w[r][k] in fp32 (bf16-rounded when round_out), fp32 weights [rows][k]: the
 * router's logits. Replaces stbl_gemv_f32 (stbl/kernels.h:23, stbl/kernels.cu:206-214). */
void stbl_gemv_f32(float *y, const float *w, const float *x, int rows, int k, int round_out, hipStream_t st);

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

/* stbl/kernels.h:34 (stbl/kernels.cu:436-442): s[i] = sqrt(softplus(s[i])) in place, softplus with
 * torch's threshold of 20 -- the engine's router scores after stbl_gemv_f32. The same scores
 * stbl_amd_route computes with score_fn = 1. */
void stbl_sqrt_softplus(float *s, int n, hipStream_t st);

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

/* n <= 64 same-shape v2 GEMVs in one launch, each as stbl_amd_gemv_fp4 / _fp8: the batching of
 * stbl_gemv_mxfp4_batch (stbl/kernels.h:18-20, which stops at 16) in the v2 formats. y, codes, scales
 * and x are HOST arrays of n device pointers. */
int stbl_amd_gemv_fp4_batch(void *const *y, const void *const *codes, const void *const *scales, const void *const *x,
                            int n, int m, int rows, int k, int y_f32, hipStream_t st);
int stbl_amd_gemv_fp8_batch(void *const *y, const void *const *codes, const void *const *scales, const void *const *x,
                            int n, int m, int rows, int k, int y_f32, hipStream_t st);

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

/* FP8 weight quantization in the reference engine's layout, one E8M0 scale byte per 32x32 block
 * (stbl/kernels.cu:98-103; the reference's own weights arrive quantized, tools/convert_official.py:
 * 53-54): s = pow2_ceil(max(amax, 1e-4) * (1/448)) as act_quant's power-of-two rule
 * (ref/kernel.py:38-40), codes = e4m3_rne(clamp(w/s, +-448)). scales [ceil(rows/32)][k/32] bytes;
 * k % 32 == 0. */
int stbl_amd_quant_fp8_e8m0(void *codes, void *scales, const float *w, int rows, int k, hipStream_t st);

/* out fp32 [rows][k] = e2m1(code) * 2^(s-127), one fp32 product per element (ref/kernel.py:98-101). */
int stbl_amd_dequant_fp4(float *out, const void *codes, const void *scales, int rows, int k, hipStream_t st);

/* out fp32 [rows][k] from GGUF MXFP4 17-byte blocks (tools/convert_official.py:187-201 layout). */
int stbl_amd_dequant_gguf17(float *out, const void *w, int rows, int k, hipStream_t st);

/* out fp32 [rows][k] = e4m3(code) * scale (ref/kernel.py:89-90): fp32 128x128 scales, or with
 * scale_e8m0 the reference engine's E8M0 bytes per 32x32 block [(rows+31)/32][k/32]. */
int stbl_amd_dequant_fp8(float *out, const void *codes, const void *scales, int rows, int k, int scale_e8m0,
                         hipStream_t st);

/* ---- v2: expert FFN and routed MoE (stbl/model.cu:426-594 composition) ------------------------------ */

/* Weight formats of an expert slot. */
enum { STBL_AMD_FP4 = 0, STBL_AMD_FP8 = 1, STBL_AMD_FP8_E8M0 = 2 };

/* Byte layout of one expert slot: gate [inter x dim], up [inter x dim], down [dim x inter], each as
 * codes then scales (FP4: codes [rows][k/2] + E8M0 [rows][k/32]; FP8: codes [rows][k] + fp32
 * [ceil(rows/128)][ceil(k/128)]; FP8_E8M0: codes [rows][k] + E8M0 [ceil(rows/32)][k/32]), every
 * part 256-byte aligned. Writes the six part offsets (may be
 * NULL) and returns the slot size. Replaces the gate|up|down slot of stbl/model.cu:374-381. */
uint64_t stbl_amd_expert_layout(int fmt, int dim, int inter, uint64_t *offsets);

/* One expert FFN on m <= 4 tokens (stbl/model.cu:516-547 for one expert):
 * y[t] = bf16(down . act(swiglu(bf16(gate . act(x_t)), bf16(up . act(x_t)), weight, limit)))
 * where act is act_quant(., 32, ue8m0, inplace) when `official`, else the identity, and swiglu is
 * stbl_swiglu's arithmetic. slot 256-byte aligned in the layout above; x bf16 [m][dim]; y bf16
 * [m][dim] (fp32 holding the unrounded down product when y_f32); work >= m * inter * 2 bytes of
 * device scratch. FP4 and FP8_E8M0 need dim, inter % 32 == 0; FP8 % 128; K <= 16384 (FP4) / 8192
 * (FP8). */
int stbl_amd_expert_ffn(int fmt, void *y, const void *slot, const void *x, int m, int dim, int inter, float weight,
                        float limit, int official, int y_f32, void *work, hipStream_t st);

/* A routed MoE layer's expert part over cached slots (stbl/model.cu:505-592): for every token t,
 * y[t] = bf16(sum_p o(slot[pick[t][p]], weights[t][p]) + o(slot[shared], 1)) with the fp32 sum taken
 * in top-k order from 0, each o an expert FFN output rounded to bf16 with the route weight applied
 * inside SwiGLU. slots: HOST array of n_slots device pointers; pick [t][topk] (HOST) indexes it;
 * weights [t][topk] (HOST); shared = slot index of the always-on expert or -1; shared_fmt = that
 * slot's format, or -1 for fmt (the reference pairs FP4 routed experts with an FP8 E8M0 shared
 * expert, stbl/model.cu:544-547). t <= 16, topk <= 16. work: device scratch of
 * stbl_amd_moe_work_bytes() bytes. */
int stbl_amd_moe_experts(int fmt, void *y, const void *x, int t, int dim, int inter, const void *const *slots,
                         int n_slots, const int *pick, const float *weights, int topk, int shared, int shared_fmt,
                         float limit, int official, int y_f32, void *work, hipStream_t st);

/* stbl_amd_moe_experts split in two calls around an expert cache's refill wait, as the reference
 * queues its cached experts and the shared expert before reading the misses and runs the missed
 * experts after (stbl/model.cu:541-549, 588). slot_ready: HOST array of n_slots flags (the `ready`
 * output of stbl_amd_cache_lookup_begin; 1 for a resident shared slot). phase 1 runs the experts of
 * ready slots, phase 2 the others and the ordered combine; both calls take the same arguments and
 * work, and their result is bit-identical to stbl_amd_moe_experts. phase 0 = stbl_amd_moe_experts. */
int stbl_amd_moe_experts_phase(int fmt, void *y, const void *x, int t, int dim, int inter, const void *const *slots,
                               int n_slots, const int *pick, const float *weights, int topk, int shared,
                               int shared_fmt, float limit, int official, int y_f32, const int *slot_ready, int phase,
                               void *work, hipStream_t st);

/* stbl_amd_moe_experts without the work argument: it allocates nothing (no hipMalloc, no library
 * allocation) and uses a static device array of the library's, 8 MiB per GPU, held until the
 * process ends. No counterpart in the reference; it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops). Refuses (negative hipError_t) a step
 * whose stbl_amd_moe_work_bytes(t, topk, dim, inter) exceeds 8 MiB (every step of the C4 and V4.1
 * shapes up to 16 tokens x top-16 fits). Nothing in the scratch must start at zero. Calls that
 * overlap in time on one GPU share that GPU's scratch and race; serialize them (one stream). */
int stbl_amd_moe_experts_noalloc(int fmt, void *y, const void *x, int t, int dim, int inter, const void *const *slots,
                                 int n_slots, const int *pick, const float *weights, int topk, int shared,
                                 int shared_fmt, float limit, int official, int y_f32, hipStream_t st);

/* Scratch bytes for stbl_amd_moe_experts on t tokens. */
uint64_t stbl_amd_moe_work_bytes(int t, int topk, int dim, int inter);

/* Router on the device (stbl/model.cu:430-452): score_fn 0: score = 1 / (1 + exp(-logit)) (the
 * configuration's sigmoid router); score_fn 1: score = sqrt(softplus(logit)), softplus(l) = l above
 * 20 else log1p(exp(l)) (the reference engine's, stbl/kernels.cu:436-442). ids = top-k of score +
 * bias (bias may be NULL), ties to the lower id, in descending order; weights = score / (sum of the
 * top-k scores in order + 1e-20) * route_scale. logits fp32 [t][n_exp], ids int32 [t][topk],
 * weights fp32 [t][topk], scores fp32 [t][n_exp] (optional). n_exp <= 1024, topk <= 32.
 * Replaces stbl_sqrt_softplus + the host partial_sort of stbl/model.cu:431-451. */
int stbl_amd_route(const float *logits, const float *bias, int t, int n_exp, int topk, float route_scale, int score_fn,
                   int *ids, float *weights, float *scores, hipStream_t st);

/* ---- v2: multi-token expert GEMM (ref/kernel.py:85-102 with M > 4, scaled f8f6f4 MFMA) ------------ */

/* Y[m][n] = sum_k Aq[m][k] Wdeq[n][k], m <= 64, where Aq = act_quant(X, act_block, "ue8m0")
 * (act_block 32 or 128: e4m3 codes with power-of-two scales) and W is FP4 (fmt 0: codes [n][k/2] +
 * E8M0 [n][k/32]) or FP8 (fmt 1: codes [n][k] + fp32 [ceil(n/128)][k/128]). X bf16 [m][k], Y bf16
 * [m][n] (fp32 when y_f32). k % 128 == 0, n <= 2^20. work: device scratch of
 * stbl_amd_gemm_work_bytes() bytes (no initial contents needed); calls sharing one work buffer must
 * not overlap in time.
 * Replaces fp8_gemm / fp4_gemm(A = act_quant(X)) of ref/kernel.py:85-102. */
int stbl_amd_gemm(int fmt, void *y, const void *codes, const void *scales, const void *x, int m, int n, int k,
                  int act_block, int y_f32, void *work, hipStream_t st);

/* The same GEMM on activations already quantized by stbl_amd_act_quant_e4m3: aq e4m3 codes [m][k]
 * (16-byte aligned), as E8M0 scale bytes [m][k/act_block]. One launch.
 * Replaces fp8_gemm(a, a_s, b, b_s) / fp4_gemm(a, a_s, b, b_s) of ref/kernel.py:85-102, which take
 * the quantized activation and its scales as arguments. */
int stbl_amd_gemm_q(int fmt, void *y, const void *codes, const void *scales, const void *aq, const void *as, int m,
                    int n, int k, int act_block, int y_f32, void *work, hipStream_t st);

/* Scratch bytes for stbl_amd_gemm and stbl_amd_gemm_q with m activation rows (n, k as in the call);
 * a workspace of that size also serves every call with fewer rows. The same bytes serve the packed
 * variants below. */
uint64_t stbl_amd_gemm_work_bytes(int m, int n, int k);

/* No counterpart in the reference: for callers whose GEMM weights are static (an expert's matrices
 * loaded once), the weight codes rearranged once into MFMA operand order, so each wave load of the
 * GEMM reads one contiguous kilobyte instead of 16 columns x 64 bytes. packed receives as many bytes
 * as codes holds (FP4 n * k / 2, FP8 n * k); n % 16 == 0, k % 128 == 0, both 16-byte aligned and
 * distinct. The scales keep their layout. */
int stbl_amd_gemm_pack(int fmt, void *packed, const void *codes, int n, int k, hipStream_t st);

/* stbl_amd_gemm_q / stbl_amd_gemm with the weight codes from stbl_amd_gemm_pack (n % 16 == 0; every
 * other argument and result as there, bit for bit). No counterpart in the reference. */
int stbl_amd_gemm_q_packed(int fmt, void *y, const void *packed, const void *scales, const void *aq, const void *as,
                           int m, int n, int k, int act_block, int y_f32, void *work, hipStream_t st);
int stbl_amd_gemm_packed(int fmt, void *y, const void *packed, const void *scales, const void *x, int m, int n, int k,
                         int act_block, int y_f32, void *work, hipStream_t st);

/* act_quant(x, block, "ue8m0") (ref/kernel.py:35-45) as the GEMM consumes it: x bf16 [rows][k] ->
 * e4m3 codes [rows][k] and E8M0 scale bytes [rows][k/block]; block 32 or 128. Non-finite values as
 * the engine's act_quant treats them (stbl/kernels.cu:56-63): a NaN is left out of its block's
 * maximum and clamps to -448; a block holding an infinity gets scale byte 255 (+Inf) and codes
 * x / Inf (0, and -448 for the infinity). stbl_amd_act_quant follows the same rules. */
int stbl_amd_act_quant_e4m3(const void *x, int rows, int k, int block, void *codes, void *scales, hipStream_t st);

/* ---- v2: HBM expert cache (stbl/model.cu:99-106, 347-422 ExpertCache / expert() / take_slot) -------- */

/* Creates an LRU cache of `slots` expert slots of slot_bytes on the current device (allocates the
 * slots, a copy stream and events; with stbl_amd_cache_create_gguf and stbl_amd_gguf_open the only
 * allocating calls of this library). host_pool: pinned
 * host memory holding n_layers * n_experts experts host_stride bytes apart, alive as long as the
 * cache. Returns NULL on failure. */
void *stbl_amd_cache_create(int slots, uint64_t slot_bytes, const void *host_pool, uint64_t host_stride, int n_experts,
                            int n_layers);

/* File-backed cache over a GGUF file (stbl/model.cu:283-308 read_range / read_pieces, :383-422 the
 * demand read of an expert): the routed experts of GGUF blocks first_layer .. first_layer+n_layers-1
 * (blk.N.ffn_{gate,up,down}_exps.weight, MXFP4 [dim, inter, experts] / [inter, dim, experts], the
 * reference converter's tensors) are read on misses in 2 MiB pieces by `readers` threads (1..16),
 * with O_DIRECT when direct = 1 and the file system allows it, and repacked on the device into FP4
 * (OCP) slots of stbl_amd_expert_layout(STBL_AMD_FP4, dim, inter) bytes; lookup then blocks the
 * host until its misses are read. Cache layer l is GGUF block first_layer + l. NULL on failure. */
void *stbl_amd_cache_create_gguf(int slots, const char *path, int first_layer, int n_layers, int readers, int direct);

/* File-backed caches only: out[0..7] = dim, inter, experts, slot bytes, 1 if O_DIRECT, bytes read
 * from the file, nanoseconds spent reading, experts read. No reference counterpart (the reference
 * prints its read time per token, stbl/model.cu:250-258). */
int stbl_amd_cache_file_info(void *cache, uint64_t *out);

/* File-backed caches: starts `readers` (1..16) background prefetch readers (the reference's
 * STBL_PREFETCH readers, stbl/model.cu:310-345, 1007-1015), with device staging for 16 experts in
 * flight. Once per cache. */
int stbl_amd_cache_enable_prefetch(void *cache, int readers);

/* Queues background reads of experts of `layer` (HOST ids, best guess first; the stale-router guess
 * of stbl/model.cu:432-475, 555-586) that are not cached. Each is mapped to a slot at once (never a
 * slot of the last lookup); prefetch readers wait while a lookup reads on demand. A lookup that
 * routes a prefetched expert waits for it if it is being read and reads it itself if it had not
 * started; the lookup of its layer cancels it if not routed and not started (stbl/model.cu:478-496).
 * Returns the number queued (at most 16 in flight) or a negative hipError_t. */
int stbl_amd_cache_prefetch(void *cache, const int *ids, int n, int layer);

/* out[0..5] = issued, routed after landing, routed while still reading, cancelled, taken over by a
 * demand read, bytes read by prefetch readers (stbl_prefetch, stbl/model.cu:1103-1105). */
int stbl_amd_cache_prefetch_stats(void *cache, uint64_t *out);

/* Test hook: paused != 0 stops prefetch readers from starting queued jobs. */
int stbl_amd_cache_prefetch_pause(void *cache, int paused);

/* Frees the cache after its copies finished. */
void stbl_amd_cache_destroy(void *cache);

/* Looks up n expert ids (HOST array) of `layer` in order; cached experts of the lookup are touched
 * first so that a miss never evicts one of them. slot_ptrs (HOST, n) receives each expert's slot,
 * hit (HOST, optional) 1 for hits. Misses are copied from the host pool on the cache's copy stream
 * and `compute` is made to wait for them (no host blocking). Returns the number of misses or a
 * negative hipError_t; a failed refill leaves its slot unmapped. */
int stbl_amd_cache_lookup(void *cache, const int *ids, int n, int layer, void **slot_ptrs, int *hit,
                          hipStream_t compute);

/* stbl_amd_cache_lookup in two calls (stbl/model.cu:497-553, the reference's expert() lookups, then
 * read_pieces after the cached experts' kernels are queued). _begin maps every id as the lookup
 * does and queues pool refills on the copy stream; ready (HOST, optional, n flags) is 1 where
 * `compute` may read the slot at once and 0 where it must wait for _end (a refill, a file read, a
 * prefetch landed or still being read). _end reads the file misses (blocking the host), waits for
 * routed prefetches still being read, and makes `compute` wait for every copy and repack. Every
 * _begin must be followed by _end before the next lookup or prefetch on the cache. _begin returns
 * the number of misses or a negative hipError_t; _end returns 0 or a negative hipError_t (then the
 * experts not read stay unmapped and their slots must not be read). */
int stbl_amd_cache_lookup_begin(void *cache, const int *ids, int n, int layer, void **slot_ptrs, int *hit, int *ready,
                                hipStream_t compute);
int stbl_amd_cache_lookup_end(void *cache, hipStream_t compute);

/* Notes the guesses for `layer` (HOST ids, best first: the next layer's router scored on this
 * layer's input, the reference's STBL_LOOKAHEAD, stbl/model.cu:432-435, 461-474) and whether each is
 * uncached now; the lookup of `layer` then updates the lookahead counters. */
int stbl_amd_cache_note_guesses(void *cache, const int *ids, int n, int layer);

/* out[0..3] = guesses uncached when noted, of which routed; routed experts not mapped at their
 * lookup, of which guessed (stbl_lookahead, stbl/model.cu:452-460, 1107-1109). */
int stbl_amd_cache_lookahead(void *cache, uint64_t *out);

/* Marks the slots of the last lookup as used by the work queued so far on `compute`; a later refill
 * of one of them waits for that work. */
int stbl_amd_cache_mark_used(void *cache, hipStream_t compute);

/* out[0..5] = hits, misses, refill bytes, lookups, slots in use, slots (stbl_stats, stbl/stbl.h:20). */
int stbl_amd_cache_stats(void *cache, uint64_t *out);

/* Slot of a cached expert without touching the LRU order, or NULL. */
void *stbl_amd_cache_peek(void *cache, int layer, int expert);

/* Test hook: the refill after n more refills fails on the host without copying (n = -1 disables). */
int stbl_amd_cache_fail_refill_after(void *cache, int n);

/* ---- v2: GGUF reader (stbl/gguf.h:9-31, stbl/gguf.cpp) ------------------------------------------------- */

/* Parses a GGUF (version >= 2) file's header with pread: metadata and the tensor table; tensor
 * offsets become absolute file offsets (data start aligned to general.alignment, 32 if absent).
 * Returns a handle or NULL (the reason in stbl_amd_last_error). */
void *stbl_amd_gguf_open(const char *path);
void stbl_amd_gguf_close(void *g);

/* A tensor's type (GGUF type id: 0 F32, 1 F16, 24 I8, 30 BF16, 39 MXFP4, 200 E4M3, 201 E8M0), dims
 * (innermost first, up to 4 written), absolute file offset and byte size (0 for other types).
 * 0, or -hipErrorNotFound without recording an error when the tensor is absent. */
int stbl_amd_gguf_tensor(void *g, const char *name, uint32_t *type, uint64_t *dims, int *ndims, uint64_t *offset,
                         uint64_t *nbytes);

/* Scalar metadata (stbl/gguf.h:28-29 u32 / f32): 0, or -hipErrorNotFound when the key is absent or
 * of another type. */
int stbl_amd_gguf_u32(void *g, const char *key, uint32_t *v);
int stbl_amd_gguf_f32(void *g, const char *key, float *v);

/* A u32 or u64 array (stbl/gguf.h:31 uints): up to cap values into out (may be NULL); returns the
 * array's length, or -hipErrorNotFound when the key is absent or holds another type. */
int64_t stbl_amd_gguf_uints(void *g, const char *key, uint64_t *out, int64_t cap);

/* ---- v2: measurement ------------------------------------------------------------------------------------ */

/* A bare streaming read of `bytes` (a multiple of 16) from 16-byte aligned device memory in one
 * launch: the floor for one-launch kernels that read as many bytes. sink: device buffer of
 * stbl_amd_read_floor_sink_words(bytes) 32-bit words (one per wave). No reference counterpart (the
 * reference calibrates with a 64 MiB device copy, stbl/bench_gemv.py:58-61). */
int stbl_amd_read_floor(const void *src, uint64_t bytes, void *sink, hipStream_t st);
uint64_t stbl_amd_read_floor_sink_words(uint64_t bytes);

/* Writes the GPU's constant-rate wall clock into t[i] (device memory, i >= 0) when this one-thread
 * launch starts on st; stbl_amd_clock_rate_khz gives its ticks per millisecond. Captured in a graph
 * between launches, two stamps bracket exactly the launches between them. No reference counterpart
 * (the reference times with events, stbl/bench_gemv.py:18-28). */
int stbl_amd_clock_stamp(uint64_t *t, int i, hipStream_t st);
int stbl_amd_clock_rate_khz(int *khz);

/* ---- library ------------------------------------------------------------------------------------------ */

/* The calling thread's last failure: copies its message into buf (len bytes, may be NULL), clears
 * it, returns its hipError_t code (0 if none). No reference counterpart (the reference never checks
 * launches, stbl/kernels.cu:545-640). */
int stbl_amd_last_error(char *buf, int len);

/* ABI version of this library, raised whenever an exported function's signature or meaning changes
 * (stblarge_amd/cmp_builds.py compares two builds only at equal versions). */
int stbl_amd_version(void);

#ifdef __cplusplus
}
#endif

#endif /* STBL_AMD_H */
