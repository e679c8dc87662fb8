/*
 * CPU oracle for the quantized expert-GEMV path. TEST INFRASTRUCTURE ONLY: tests/, the smoke check
 * and bench.py's cpu_baseline leg load this library as the checker; the product path never does.
 *
 * It restates, in plain C with IEEE fp32 arithmetic (built with -ffp-contract=off so no product is
 * fused into an add), the arithmetic of:
 *   - ref/kernel.py:12-102      codecs, act_quant, fp4 quantization, fp8_gemm / fp4_gemm dequant;
 *   - tools/convert_official.py:40-48   e4m3 closed form; :187-201 GGUF MXFP4 17-byte blocks;
 *   - stbl/kernels.cu:54-63,86-89,134-191,444-464   engine act_quant / round / GEMV / SwiGLU / axpy;
 *   - stbl/model.cu:426-594     MoE composition (router weights, order of the expert sums);
 *   - stbl/kernels.cu:436-442   router score sqrt(softplus) (threshold 20).
 * Matrix products accumulate in double: the reference's own GEMMs only fix the products, not the
 * summation order (ref/kernel.py:6-7), so a more accurate sum is the right yardstick.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---- scalar codecs --------------------------------------------------------------------------- */

/* 2^ceil(log2 t) by exponent/mantissa bits: ref/kernel.py:22-26 (stbl/kernels.cu:26-30). */
float orc_pow2_ceil(float t) {
    const uint32_t b = f2u(t);
    const int e = (int)((b >> 23) & 0xff) - 127 + ((b & 0x7fffffu) != 0);
    return u2f((uint32_t)(e + 127) << 23);
}

/* E4M3 (fn) byte -> fp32, closed form of tools/convert_official.py:40-48; 0x7f/0xff are NaN. */
float orc_e4m3_decode(uint8_t c) {
    const int e = (c >> 3) & 15, m = c & 7;
    float v;
    if (e == 15 && m == 7) v = NAN;
    else v = e == 0 ? ldexpf((float)m, -9) : ldexpf((float)(8 + m), e - 10);
    return (c & 0x80) ? -v : v;
}

/* fp32 -> E4M3 round to nearest, ties to even (the torch .to(float8_e4m3fn) cast ref/kernel.py:41
 * applies after clamping to +-448). Saturates beyond 448; NaN -> 0x7f. Sign of zero is kept. */
uint8_t orc_e4m3_encode(float x) {
    const uint8_t sign = signbit(x) ? 0x80 : 0;
    if (isnan(x)) return 0x7f;
    const float a = fabsf(x);
    if (a >= 448.0f) return sign | 0x7e;
    if (a == 0.0f) return sign;
    int e2;
    frexpf(a, &e2);
    int E = e2 - 1;            /* a in [2^E, 2^(E+1)) */
    if (E < -6) E = -6;        /* subnormal range: step 2^-9 */
    const float q = rintf(a / ldexpf(1.0f, E - 3)); /* exact quotient, RNE */
    int qi = (int)q;
    if (E == -6 && qi < 8) return sign | (uint8_t)qi;
    if (qi == 16) { E += 1; qi = 8; }
    return sign | (uint8_t)(((E + 7) << 3) | (qi - 8));
}

/* Array forms of the encoder (the Python wrapper's vectorised path). */
void orc_e4m3_encode_n(const float *x, int n, uint8_t *out) {
    for (int i = 0; i < n; i++) out[i] = orc_e4m3_encode(x[i]);
}

/* FP4_TABLE of ref/kernel.py:14-16 (stbl/kernels.cu:44). */
static const float kFp4[16] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f, -0.f, -.5f, -1.f, -1.5f, -2.f, -3.f, -4.f, -6.f};
float orc_e2m1_decode(uint8_t nib) { return kFp4[nib & 15]; }

/* E8M0 byte -> 2^(s-127) as torch's float8_e8m0fnu reads it (code 0 = 2^-127, 255 = NaN). */
float orc_e8m0_decode(uint8_t s) {
    if (s == 255) return NAN;
    if (s == 0) return u2f(0x00400000u);
    return u2f((uint32_t)s << 23);
}

/* _round_fp4, ref/kernel.py:48-52: onto the e2m1 grid, ties to even; v already within [-6, 6]. */
float orc_round_fp4(float v) {
    const float a = fabsf(v);
    const float step = a < 2.f ? .5f : (a < 4.f ? 1.f : 2.f);
    return copysignf(rintf(a / step) * step, v);
}

/* _fp4_codes, ref/kernel.py:75-77: magnitude index on the grid | sign bit << 3 (so -0.0 -> 8). */
uint8_t orc_fp4_code(float q) {
    const float a = fabsf(q);
    int i = 0;
    while (i < 7 && kFp4[i] < a) i++;  /* searchsorted(left) over the 8 magnitudes */
    return (uint8_t)(i | (signbit(q) ? 8 : 0));
}

/* fp32 -> bf16 bits, round to nearest even (torch .to(bfloat16)). */
uint16_t orc_f2bf(float f) {
    uint32_t u = f2u(f);
    if (isnan(f)) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float orc_bf2f(uint16_t h) { return u2f((uint32_t)h << 16); }
static inline float bf16r(float f) { return orc_bf2f(orc_f2bf(f)); }

/* ---- activation quantization (ref/kernel.py:35-45; stbl/kernels.cu:54-63) --------------------- */

/* x [rows][n] fp32 (bf16 values). Per `block` values: amax >= 1e-4, t = amax * fp32(1/448),
 * s = pow2_ceil(t) if pow2 else t; q = e4m3(clamp(x / s, +-448)). Writes codes [rows][n] and
 * scales [rows][n/block]; if deq != NULL also the in-place form bf16(e4m3(q) * s) as fp32. */
void orc_act_quant(const float *x, int rows, int n, int block, int pow2, uint8_t *codes, float *scales,
                   float *deq) {
    const float inv = (float)(1.0 / 448.0);
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < n / block; b++) {
            const float *xb = x + (size_t)r * n + (size_t)b * block;
            float amax = 0.f;
            for (int i = 0; i < block; i++) amax = fmaxf(amax, fabsf(xb[i]));
            amax = fmaxf(amax, 1e-4f);
            const float t = amax * inv;
            const float s = pow2 ? orc_pow2_ceil(t) : t;
            if (scales) scales[(size_t)r * (n / block) + b] = s;
            for (int i = 0; i < block; i++) {
                float v = xb[i] / s;
                v = fminf(fmaxf(v, -448.f), 448.f);
                const uint8_t c = orc_e4m3_encode(v);
                const size_t at = (size_t)r * n + (size_t)b * block + i;
                if (codes) codes[at] = c;
                if (deq) deq[at] = bf16r(orc_e4m3_decode(c) * s);
            }
        }
}

/* ---- weight quantizers (synthetic data of the BASELINE configs) -------------------------------- */

/* FP4 e2m1 with E8M0 scales per 32 along K: fp4_act_quant(x, 32) of ref/kernel.py:55-72 applied to
 * a weight [rows][k]. codes [rows][k/2] (element 2i low nibble, 2i+1 high), scales [rows][k/32]. */
void orc_quant_fp4(const float *w, int rows, int k, uint8_t *codes, uint8_t *scales) {
    const float inv6 = (float)(1.0 / 6.0);
    const float floor_amax = 6.0f * ldexpf(1.0f, -126);
    for (int r = 0; r < rows; r++)
        for (int g = 0; g < k / 32; g++) {
            const float *wb = w + (size_t)r * k + (size_t)g * 32;
            float amax = 0.f;
            for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(wb[i]));
            amax = fmaxf(amax, floor_amax);
            const float s = orc_pow2_ceil(amax * inv6);
            scales[(size_t)r * (k / 32) + g] = (uint8_t)((f2u(s) >> 23) & 0xff);
            for (int i = 0; i < 32; i += 2) {
                const float q0 = orc_round_fp4(fminf(fmaxf(wb[i] / s, -6.f), 6.f));
                const float q1 = orc_round_fp4(fminf(fmaxf(wb[i + 1] / s, -6.f), 6.f));
                codes[(size_t)r * (k / 2) + (size_t)g * 16 + i / 2] =
                    (uint8_t)(orc_fp4_code(q0) | (orc_fp4_code(q1) << 4));
            }
        }
}

/* FP8 e4m3 with one fp32 scale per 128x128 block: s = max(amax, 1e-4) / 448 (a true division),
 * q = e4m3(clamp(w / s, +-448)). scales [ceil(rows/128)][ceil(k/128)]; edge blocks are partial. */
void orc_quant_fp8_b128(const float *w, int rows, int k, uint8_t *codes, float *scales) {
    const int nb = (rows + 127) / 128, kb = (k + 127) / 128;
    for (int bi = 0; bi < nb; bi++)
        for (int bj = 0; bj < kb; bj++) {
            const int r0 = bi * 128, r1 = r0 + 128 < rows ? r0 + 128 : rows;
            const int c0 = bj * 128, c1 = c0 + 128 < k ? c0 + 128 : k;
            float amax = 0.f;
            for (int r = r0; r < r1; r++)
                for (int c = c0; c < c1; c++) amax = fmaxf(amax, fabsf(w[(size_t)r * k + c]));
            amax = fmaxf(amax, 1e-4f);
            const float s = amax / 448.0f;
            scales[(size_t)bi * kb + bj] = s;
            for (int r = r0; r < r1; r++)
                for (int c = c0; c < c1; c++) {
                    const float v = fminf(fmaxf(w[(size_t)r * k + c] / s, -448.f), 448.f);
                    codes[(size_t)r * k + c] = orc_e4m3_encode(v);
                }
        }
}

/* FP8 e4m3 with one E8M0 scale byte per 32x32 block, the reference engine's FP8 layout
 * (stbl/kernels.cu:98-103; its weights arrive quantized, tools/convert_official.py:53-54). Synthetic
 * weights use act_quant's power-of-two rule (ref/kernel.py:38-40) per block:
 * s = pow2_ceil(max(amax, 1e-4) * fp32(1/448)), q = e4m3(clamp(w / s, +-448)).
 * scales [(rows+31)/32][k/32]; k % 32 == 0; the last row block may be partial. */
void orc_quant_fp8_e8m0_b32(const float *w, int rows, int k, uint8_t *codes, uint8_t *scales) {
    const float inv = (float)(1.0 / 448.0);
    const int nb = (rows + 31) / 32, kb = k / 32;
    for (int bi = 0; bi < nb; bi++)
        for (int bj = 0; bj < kb; bj++) {
            const int r0 = bi * 32, r1 = r0 + 32 < rows ? r0 + 32 : rows, c0 = bj * 32;
            float amax = 0.f;
            for (int r = r0; r < r1; r++)
                for (int c = c0; c < c0 + 32; c++) amax = fmaxf(amax, fabsf(w[(size_t)r * k + c]));
            const float sc = orc_pow2_ceil(fmaxf(amax, 1e-4f) * inv);
            scales[(size_t)bi * kb + bj] = (uint8_t)((f2u(sc) >> 23) & 0xff);
            for (int r = r0; r < r1; r++)
                for (int c = c0; c < c0 + 32; c++) {
                    const float v = fminf(fmaxf(w[(size_t)r * k + c] / sc, -448.f), 448.f);
                    codes[(size_t)r * k + c] = orc_e4m3_encode(v);
                }
        }
}

/* ---- dequantization (ref/kernel.py:89-90, :98-101): one fp32 product per element ---------------- */

void orc_dequant_fp8_b128(const uint8_t *codes, const float *scales, int rows, int k, float *out) {
    const int kb = (k + 127) / 128;
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < k; c++)
            out[(size_t)r * k + c] = orc_e4m3_decode(codes[(size_t)r * k + c]) * scales[(size_t)(r / 128) * kb + c / 128];
}

/* The reference engine's FP8 layout: E8M0 scale bytes per 32x32 block, [(rows+31)/32][k/32]
 * (stbl/kernels.cu:98-103). */
void orc_dequant_fp8_e8m0_b32(const uint8_t *codes, const uint8_t *scales, int rows, int k, float *out) {
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < k; c++)
            out[(size_t)r * k + c] =
                orc_e4m3_decode(codes[(size_t)r * k + c]) * orc_e8m0_decode(scales[(size_t)(r / 32) * (k / 32) + c / 32]);
}

void orc_dequant_fp4(const uint8_t *codes, const uint8_t *scales, int rows, int k, float *out) {
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < k; c++) {
            const uint8_t b = codes[(size_t)r * (k / 2) + c / 2];
            out[(size_t)r * k + c] = kFp4[(c & 1) ? (b >> 4) : (b & 15)] * orc_e8m0_decode(scales[(size_t)r * (k / 32) + c / 32]);
        }
}

/* GGUF MXFP4 rows of 17-byte blocks: [E8M0][16 B: low nibble = elements 0..15, high = 16..31]
 * (tools/convert_official.py:187-201, stbl/kernels.cu:134-141). */
void orc_dequant_gguf17(const uint8_t *w, int rows, int k, float *out) {
    for (int r = 0; r < rows; r++)
        for (int g = 0; g < k / 32; g++) {
            const uint8_t *blk = w + ((size_t)r * (k / 32) + g) * 17;
            const float s = orc_e8m0_decode(blk[0]);
            for (int i = 0; i < 16; i++) {
                out[(size_t)r * k + g * 32 + i] = kFp4[blk[1 + i] & 15] * s;
                out[(size_t)r * k + g * 32 + 16 + i] = kFp4[blk[1 + i] >> 4] * s;
            }
        }
}

/* OCP packed codes + separate scales -> GGUF 17-byte blocks (the repack of
 * tools/convert_official.py:187-201 / stbl/test_kernels.py:109-112). */
void orc_ocp_to_gguf17(const uint8_t *codes, const uint8_t *scales, int rows, int k, uint8_t *out) {
    for (int r = 0; r < rows; r++)
        for (int g = 0; g < k / 32; g++) {
            const uint8_t *cb = codes + (size_t)r * (k / 2) + (size_t)g * 16;
            uint8_t *blk = out + ((size_t)r * (k / 32) + g) * 17;
            uint8_t v[32];
            for (int i = 0; i < 16; i++) v[2 * i] = cb[i] & 15, v[2 * i + 1] = cb[i] >> 4;
            blk[0] = scales[(size_t)r * (k / 32) + g];
            for (int i = 0; i < 16; i++) blk[1 + i] = (uint8_t)(v[i] | (v[16 + i] << 4));
        }
}

/* ---- products ------------------------------------------------------------------------------------ */

/* out[m][n] = sum_k a[m][k] * w[n][k] in double (C = A @ B^T of ref/kernel.py:91,102). */
void orc_gemm(const float *a, const float *w, int m, int n, int k, double *out) {
    for (int i = 0; i < m; i++)
        for (int j = 0; j < n; j++) {
            const float *ar = a + (size_t)i * k, *wr = w + (size_t)j * k;
            double s0 = 0, s1 = 0, s2 = 0, s3 = 0;
            int c = 0;
            for (; c + 4 <= k; c += 4) {
                s0 += (double)ar[c] * wr[c];
                s1 += (double)ar[c + 1] * wr[c + 1];
                s2 += (double)ar[c + 2] * wr[c + 2];
                s3 += (double)ar[c + 3] * wr[c + 3];
            }
            for (; c < k; c++) s0 += (double)ar[c] * wr[c];
            out[(size_t)i * n + j] = (s0 + s1) + (s2 + s3);
        }
}

/* GEMV straight from FP4 OCP codes (no dequantized copy): used at full shapes and for the timed
 * CPU baseline. y[m][n] in double. */
void orc_gemv_fp4(const uint8_t *codes, const uint8_t *scales, const float *x, int m, int n, int k, double *y) {
    for (int j = 0; j < n; j++) {
        const uint8_t *cr = codes + (size_t)j * (k / 2), *sr = scales + (size_t)j * (k / 32);
        for (int i = 0; i < m; i++) {
            const float *xr = x + (size_t)i * k;
            double acc = 0;
            for (int g = 0; g < k / 32; g++) {
                const float s = orc_e8m0_decode(sr[g]);
                double part = 0;
                for (int b = 0; b < 16; b++) {
                    const uint8_t c = cr[g * 16 + b];
                    part += (double)xr[g * 32 + 2 * b] * (kFp4[c & 15] * s);
                    part += (double)xr[g * 32 + 2 * b + 1] * (kFp4[c >> 4] * s);
                }
                acc += part;
            }
            y[(size_t)i * n + j] = acc;
        }
    }
}

void orc_gemv_fp8_b128(const uint8_t *codes, const float *scales, const float *x, int m, int n, int k, double *y) {
    const int kb = (k + 127) / 128;
    for (int j = 0; j < n; j++) {
        const uint8_t *cr = codes + (size_t)j * k;
        const float *sr = scales + (size_t)(j / 128) * kb;
        for (int i = 0; i < m; i++) {
            const float *xr = x + (size_t)i * k;
            double acc = 0;
            for (int c = 0; c < k; c++) acc += (double)xr[c] * (orc_e4m3_decode(cr[c]) * sr[c / 128]);
            y[(size_t)i * n + j] = acc;
        }
    }
}

/* ---- the reference engine's GEMVs with its own E8M0 decode --------------------------------------
 * stbl/kernels.cu:32 decodes a scale byte as the float with that exponent field, so byte 0 is 0.0
 * and byte 255 +Inf (E8M0 itself, orc_e8m0_decode, reads 2^-127 and NaN), and its GEMVs scale each
 * 32-element block's sum of products (stbl/kernels.cu:127 FP8, :185 GGUF FP4). These restate that:
 * block sums in double, times the engine's scale, added over the row in double. */
double orc_e8m0_engine(uint8_t s) { return (double)u2f((uint32_t)s << 23); }

/* GGUF MXFP4 rows of 17-byte blocks (stbl/kernels.cu:134-191), one token: y[n] in double. */
void orc_gemv_gguf_engine(const uint8_t *w, const float *x, int n, int k, double *y) {
    for (int j = 0; j < n; j++) {
        double acc = 0;
        for (int g = 0; g < k / 32; g++) {
            const uint8_t *blk = w + ((size_t)j * (k / 32) + g) * 17;
            double part = 0;
            for (int i = 0; i < 16; i++) {
                part += (double)x[g * 32 + i] * kFp4[blk[1 + i] & 15];
                part += (double)x[g * 32 + 16 + i] * kFp4[blk[1 + i] >> 4];
            }
            acc += part * orc_e8m0_engine(blk[0]);
        }
        y[j] = acc;
    }
}

/* FP8 e4m3 rows with E8M0 scale bytes per 32x32 block, [(n+31)/32][k/32] (stbl/kernels.cu:98-132),
 * one token: y[n] in double. */
void orc_gemv_fp8_e8m0_engine(const uint8_t *codes, const uint8_t *scales, const float *x, int n, int k, double *y) {
    for (int j = 0; j < n; j++) {
        double acc = 0;
        for (int g = 0; g < k / 32; g++) {
            double part = 0;
            for (int i = 0; i < 32; i++) part += (double)x[g * 32 + i] * orc_e4m3_decode(codes[(size_t)j * k + g * 32 + i]);
            acc += part * orc_e8m0_engine(scales[(size_t)(j / 32) * (k / 32) + g]);
        }
        y[j] = acc;
    }
}

/* ---- elementwise epilogues (stbl/kernels.cu:86-89, 444-464) ------------------------------------ */

/* out = bf16(silu(min(g, lim)) * clamp(u, -lim, lim) * w); no clamp when lim <= 0. */
float orc_swiglu1(float g, float u, float w, float lim) {
    if (lim > 0) { u = fminf(fmaxf(u, -lim), lim); g = fminf(g, lim); }
    return bf16r(g / (1.f + expf(-g)) * u * w);
}

void orc_swiglu(const float *g, const float *u, float w, float lim, int n, float *out) {
    for (int i = 0; i < n; i++) out[i] = orc_swiglu1(g[i], u[i], w, lim);
}

void orc_round_bf16(float *x, int n) {
    for (int i = 0; i < n; i++) x[i] = bf16r(x[i]);
}

/* ---- router (scores, top-k, renormalised weights) ------------------------------------------------ */

/* Router score of one logit: score_fn 0 = sigmoid 1/(1+exp(-l)) (the configuration's router);
 * 1 = sqrt(softplus(l)) with softplus(l) = l above 20, else log1p(exp(l)) (stbl/kernels.cu:436-442,
 * torch's threshold). */
float orc_route_score(float l, int score_fn) {
    if (score_fn == 1) return sqrtf(l > 20.f ? l : log1pf(expf(l)));
    return 1.f / (1.f + expf(-l));
}

/* logits [t][e]. score = orc_route_score(l); top-k by score + bias (bias may be NULL), ties to the
 * lower id; weight_i = score_i / (sum of the top-k scores in top-k order + 1e-20) * route_scale
 * (stbl/model.cu:444-451, 528-530). A NaN key ranks below every number (the reference's host sort
 * leaves NaN undefined; this is the rule the device router follows). */
void orc_route(const float *logits, const float *bias, int t, int e, int topk, float route_scale, int score_fn,
               float *scores, int *ids, float *weights) {
    for (int i = 0; i < t; i++) {
        float *sc = scores + (size_t)i * e;
        for (int j = 0; j < e; j++) sc[j] = orc_route_score(logits[(size_t)i * e + j], score_fn);
        int *id = ids + (size_t)i * topk;
        for (int p = 0; p < topk; p++) {
            int best = -1;
            float bv = 0.f;
            for (int j = 0; j < e; j++) {
                int used = 0;
                for (int q = 0; q < p; q++) used |= id[q] == j;
                if (used) continue;
                float v = sc[j] + (bias ? bias[j] : 0.f);
                if (v != v) v = -INFINITY; /* a NaN key ranks last (then the lower id wins) */
                if (best < 0 || v > bv) best = j, bv = v;
            }
            id[p] = best;
        }
        float sum = 0.f;
        for (int p = 0; p < topk; p++) sum += sc[id[p]];
        for (int p = 0; p < topk; p++) {
            float wt = sc[id[p]];
            wt /= sum + 1e-20f;
            wt *= route_scale;
            weights[(size_t)i * topk + p] = wt;
        }
    }
}

/* ---- expert FFN (stbl/model.cu:516-547 run_experts / shared expert) ----------------------------- */

/* One FP4 expert on one token. slot = gate codes | gate scales | up codes | up scales | down codes |
 * down scales (OCP), gate/up [inter][dim], down [dim][inter]. x [dim] (bf16 values).
 * g = bf16(W1 x), u = bf16(W3 x), h = swiglu(g, u, w), h -> act_quant per 32 (pow2) when `official`,
 * o = bf16(W2 h). If act_in, x is act-quantized first (official linear()). o [dim]. */
static void ffn_fp4_one(const uint8_t *slot, int dim, int inter, const float *x, float w, float lim, int official,
                        float *o, float *xbuf, float *h, double *acc, double *raw) {
    const size_t gc = (size_t)inter * dim / 2, gs = (size_t)inter * dim / 32;
    const uint8_t *gcodes = slot, *gsc = slot + gc, *ucodes = gsc + gs, *usc = ucodes + gc, *dcodes = usc + gs,
                  *dsc = dcodes + gc;
    if (official) orc_act_quant(x, 1, dim, 32, 1, NULL, NULL, xbuf);
    else memcpy(xbuf, x, sizeof(float) * dim);
    orc_gemv_fp4(gcodes, gsc, xbuf, 1, inter, dim, acc);
    for (int i = 0; i < inter; i++) h[i] = bf16r((float)acc[i]);
    orc_gemv_fp4(ucodes, usc, xbuf, 1, inter, dim, acc);
    for (int i = 0; i < inter; i++) h[i] = orc_swiglu1(h[i], bf16r((float)acc[i]), w, lim);
    if (official) orc_act_quant(h, 1, inter, 32, 1, NULL, NULL, h);
    orc_gemv_fp4(dcodes, dsc, h, 1, dim, inter, acc);
    for (int i = 0; i < dim; i++) o[i] = bf16r((float)acc[i]);
    if (raw) memcpy(raw, acc, sizeof(double) * dim);
}

/* raw (may be NULL) receives the down product before its bf16 rounding. */
void orc_expert_ffn_fp4(const uint8_t *slot, int dim, int inter, const float *x, float w, float lim, int official,
                        float *o, double *raw) {
    float *xbuf = malloc(sizeof(float) * dim), *h = malloc(sizeof(float) * inter);
    double *acc = malloc(sizeof(double) * (dim > inter ? dim : inter));
    ffn_fp4_one(slot, dim, inter, x, w, lim, official, o, xbuf, h, acc, raw);
    free(xbuf), free(h), free(acc);
}

/* FP8 expert, 128x128 fp32 block scales. slot = gate codes | up codes | down codes, scales given
 * separately per matrix. */
void orc_expert_ffn_fp8(const uint8_t *gcodes, const float *gsc, const uint8_t *ucodes, const float *usc,
                        const uint8_t *dcodes, const float *dsc, int dim, int inter, const float *x, float w,
                        float lim, int official, float *o, double *raw) {
    float *xbuf = malloc(sizeof(float) * dim), *h = malloc(sizeof(float) * inter);
    double *acc = malloc(sizeof(double) * (dim > inter ? dim : inter));
    if (official) orc_act_quant(x, 1, dim, 32, 1, NULL, NULL, xbuf);
    else memcpy(xbuf, x, sizeof(float) * dim);
    orc_gemv_fp8_b128(gcodes, gsc, xbuf, 1, inter, dim, acc);
    for (int i = 0; i < inter; i++) h[i] = bf16r((float)acc[i]);
    orc_gemv_fp8_b128(ucodes, usc, xbuf, 1, inter, dim, acc);
    for (int i = 0; i < inter; i++) h[i] = orc_swiglu1(h[i], bf16r((float)acc[i]), w, lim);
    if (official) orc_act_quant(h, 1, inter, 32, 1, NULL, NULL, h);
    orc_gemv_fp8_b128(dcodes, dsc, h, 1, dim, inter, acc);
    for (int i = 0; i < dim; i++) o[i] = bf16r((float)acc[i]);
    if (raw) memcpy(raw, acc, sizeof(double) * dim);
    free(xbuf), free(h), free(acc);
}

/* Routed MoE layer on t tokens: for token i, y = bf16( sum over its top-k experts in top-k order of
 * o_e + o_shared ), each o from ffn_fp4_one with the route weight folded into the SwiGLU; the sum is
 * fp32, starting at zero (stbl/model.cu:589-592). slots[i*topk + p] is the expert slot of token i's
 * p-th pick; shared is the shared expert's slot (weight 1). x, y [t][dim]. */
void orc_moe_fp4(const uint8_t *const *slots, const float *weights, const uint8_t *shared, int t, int topk, int dim,
                 int inter, const float *x, float lim, int official, float *y) {
    float *xbuf = malloc(sizeof(float) * dim), *h = malloc(sizeof(float) * inter), *o = malloc(sizeof(float) * dim);
    float *sum = malloc(sizeof(float) * dim);
    double *acc = malloc(sizeof(double) * (dim > inter ? dim : inter));
    for (int i = 0; i < t; i++) {
        for (int c = 0; c < dim; c++) sum[c] = 0.f;
        for (int p = 0; p <= topk; p++) {
            const uint8_t *slot = p < topk ? slots[(size_t)i * topk + p] : shared;
            const float w = p < topk ? weights[(size_t)i * topk + p] : 1.f;
            if (!slot) continue;
            ffn_fp4_one(slot, dim, inter, x + (size_t)i * dim, w, lim, official, o, xbuf, h, acc, NULL);
            for (int c = 0; c < dim; c++) sum[c] += 1.f * o[c];
        }
        for (int c = 0; c < dim; c++) y[(size_t)i * dim + c] = bf16r(sum[c]);
    }
    free(xbuf), free(h), free(o), free(sum), free(acc);
}

/* ---- expert FFN / MoE on dequantized weights (any weight format) -------------------------------- */

/* One expert with dequantized fp32 matrices gw, uw [inter][dim], dw [dim][inter]: the composition of
 * ffn_fp4_one (every format dequantizes exactly, so the products are the same). raw may be NULL. */
void orc_expert_ffn_deq(const float *gw, const float *uw, const float *dw, int dim, int inter, const float *x,
                        float w, float lim, int official, float *o, double *raw) {
    float *xbuf = malloc(sizeof(float) * dim), *h = malloc(sizeof(float) * inter);
    double *acc = malloc(sizeof(double) * (dim > inter ? dim : inter));
    if (official) orc_act_quant(x, 1, dim, 32, 1, NULL, NULL, xbuf);
    else memcpy(xbuf, x, sizeof(float) * dim);
    orc_gemm(xbuf, gw, 1, inter, dim, acc);
    for (int i = 0; i < inter; i++) h[i] = bf16r((float)acc[i]);
    orc_gemm(xbuf, uw, 1, inter, dim, acc);
    for (int i = 0; i < inter; i++) h[i] = orc_swiglu1(h[i], bf16r((float)acc[i]), w, lim);
    if (official) orc_act_quant(h, 1, inter, 32, 1, NULL, NULL, h);
    orc_gemm(h, dw, 1, dim, inter, acc);
    for (int i = 0; i < dim; i++) o[i] = bf16r((float)acc[i]);
    if (raw) memcpy(raw, acc, sizeof(double) * dim);
    free(xbuf), free(h), free(acc);
}

/* The MoE of orc_moe_fp4 on dequantized experts: mats[(i*topk + p)*3 + {0,1,2}] are token i's p-th
 * pick's gate, up and down; shared[0..2] the shared expert's (or NULL). y [t][dim]. */
void orc_moe_deq(const float *const *mats, const float *weights, const float *const *shared, int t, int topk,
                 int dim, int inter, const float *x, float lim, int official, float *y) {
    float *o = malloc(sizeof(float) * dim), *sum = malloc(sizeof(float) * dim);
    for (int i = 0; i < t; i++) {
        for (int c = 0; c < dim; c++) sum[c] = 0.f;
        for (int p = 0; p <= topk; p++) {
            const float *const *m = p < topk ? mats + ((size_t)i * topk + p) * 3 : shared;
            if (!m) continue;
            const float w = p < topk ? weights[(size_t)i * topk + p] : 1.f;
            orc_expert_ffn_deq(m[0], m[1], m[2], dim, inter, x + (size_t)i * dim, w, lim, official, o, NULL);
            for (int c = 0; c < dim; c++) sum[c] += 1.f * o[c];
        }
        for (int c = 0; c < dim; c++) y[(size_t)i * dim + c] = bf16r(sum[c]);
    }
    free(o), free(sum);
}
