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
#include <atomic>

#include "abi_util.hpp"
#include "gemv_core.hpp"

namespace stbl {

// DW: OCP FP4 scales fetched as dwords and handed to the lanes by ds_bpermute (tiles of 4 rows and
// 2-4 tokens whose scale rows are dword-aligned: k % 128 == 0 and 4-byte aligned scales).
template <WFmt F, bool XF32, int M, int R, bool DW>
__global__ __launch_bounds__(512) void k_gemv(GemvJobs jobs, int rows, int k, int out_mode) {
    using T = WTraits<F>;
    constexpr int CH = T::CH;
    static_assert(F == WFmt::FP4_GGUF || 32 % R == 0, "a row tile must sit inside one scale block");
    static_assert(F != WFmt::FP4_GGUF || (XF32 && M == 1), "GGUF rows: the reference ABI's one fp32 token");
    const GemvJob J = jobs.j[blockIdx.y];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const int nch = k / CH, c = wave * 64 + lane;
    const bool active = c < nch;
    const int cc = active ? c : 0;
    const int row0 = blockIdx.x * R;

    // 0. OCP FP4 scales. A wave's 64 chunks of one row have 64 consecutive scale bytes. When they
    //    are dword-aligned (DW), lane j < 16 R loads dword j % 16 of row j / 16 (one instruction for
    //    up to 4 rows) and each lane takes its byte from lane 16 r + lane / 4 with ds_bpermute.
    //    Otherwise tiles of 4 or more rows stage them: the tile's rows hold one contiguous
    //    block of R * nch scale bytes, fetched with one 16-byte load per thread (from the block's
    //    16-byte units; such a load never crosses a page, so the bytes around the block are safe to
    //    read) and handed out through LDS, instead of one byte load per row per lane. With 8 rows,
    //    and with 4 rows of one token, the block is loaded before the weights, so each row's
    //    products start as soon as that row arrives; with 4 rows of 2-4 tokens (scale rows that are
    //    not dword-aligned) it is loaded after them and the tile waits for all its loads at once;
    //    tiles of 1-2 rows load each lane's scale bytes directly.
    //    (Measured: dwords beat the LDS block by 5% at 4 rows x 4 tokens (4096x4096: 13%), but with
    //    one token the early LDS block is 2-4% faster at 4 rows (7168x2048 3.46 -> 3.38 us, 4096x4096
    //    3.74 -> 3.62, 3072x3072 3.26 -> 3.15; loaded after the weights it gained 0-3%); at 2 rows
    //    dwords are up to 1.6% slower than bytes; the early LDS block is the fastest at 8 rows.)
    static_assert(!DW || (F == WFmt::FP4_OCP && R <= 4), "dword scale loads: FP4 tiles of at most 4 rows");
    constexpr bool kStageScales = F == WFmt::FP4_OCP && R >= 4 && !DW;
    constexpr bool kScalesEarly = R >= 8 || (R >= 4 && M == 1);
    static_assert(!kStageScales || R <= kMaxStageRows, "the staged scale block holds at most kMaxStageRows rows");
    constexpr int kScaleLoads = R > 8 ? 2 : 1;  // units <= R nch / 16 + 2 <= kScaleLoads * threads
    // One slot past the block takes the writes of threads without a unit, so the LDS write is
    // unconditional: a conditional one lets the compiler sink the load into the branch.
    constexpr int kScaleUnits = R * kMaxWaves * 64 / 16 + 2;  // 16-byte units of the staged block, at most
    __shared__ u32x4 lds_sc[kStageScales ? kScaleUnits + 1 : 1];
    u32x4 scv[kScaleLoads] = {};
    size_t sc_len = 0;
    int sc_units = 0;
    auto load_scale_block = [&]() {
        // pointer arithmetic (no integer round trip), so these stay global loads
        const uint8_t *blk = (const uint8_t *)J.s + (size_t)row0 * nch;
        sc_len = (size_t)(min(row0 + R, rows) - row0) * nch;
        const uint8_t *p0 = blk - ((uintptr_t)blk & 15);
        sc_units = (int)((((uintptr_t)blk & 15) + sc_len - 1) >> 4) + 1;
#pragma unroll
        for (int i = 0; i < kScaleLoads; i++)
            scv[i] = ld_stream(p0 + 16 * (size_t)min((int)threadIdx.x + i * (int)blockDim.x, sc_units - 1));
    };
    if constexpr (kStageScales && kScalesEarly) load_scale_block();
    // 1. loads: x first (it is needed by every row), then every row of the tile. fp32 activations
    //    (the reference ABI) are widened once and use exact FMAs; bf16 activations stay packed for
    //    the dot2 path (gemv_core.hpp).
    float xf[XF32 ? M : 1][XF32 ? CH : 1];
    uint32_t xw[XF32 ? 1 : M][XF32 ? 1 : CH / 2];
    if constexpr (XF32) load_x<true, M, CH>(xf, J.x, k, cc * CH);
    else load_x_packed<M, CH>(xw, (const uint16_t *)J.x, k, cc * CH);
    u32x4 w[R];
    uint32_t sb[R];
    GgufRaw graw[F == WFmt::FP4_GGUF ? R : 1];  // GGUF rows: raw dwords, realigned after every load is out
    uint32_t sdw = 0;
    if constexpr (DW) {  // rows and dwords clamped into the matrix; lanes j >= 16 R repeat the last row
        const int rr = min(lane >> 4, R - 1);
        const int dwi = min(wave * 16 + (lane & 15), (nch >> 2) - 1);
        sdw = __builtin_nontemporal_load((const uint32_t *)((const uint8_t *)J.s + (size_t)min(row0 + rr, rows - 1) * nch) + dwi);
    } else if constexpr (F == WFmt::FP4_OCP && !kStageScales) {  // tiles of 1-2 rows: each lane's bytes
#pragma unroll
        for (int r = 0; r < R; r++) sb[r] = ld_stream_u8((const uint8_t *)J.s + (size_t)min(row0 + r, rows - 1) * nch + cc);
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const size_t row = (size_t)min(row0 + r, rows - 1);
        if constexpr (F == WFmt::FP4_OCP) {
            w[r] = ld_stream(J.w + row * (k >> 1) + (size_t)cc * 16);
        } else if constexpr (F == WFmt::FP4_GGUF) {
            load_gguf_raw_at(J.w + row * (size_t)(nch * 17), (uint32_t)cc * 17u, graw[r]);
        } else {
            w[r] = ld_stream(J.w + row * k + (size_t)cc * 16);
        }
    }
    if constexpr (kStageScales && !kScalesEarly) load_scale_block();
    // With 2-4 tokens every load above is issued before anything below runs: without this fence the
    // scheduler trades registers for issue order and holds x loads of later tokens back behind the
    // first waits (4 tokens: 6.7 instead of 6.0 us at 2048x7168). One bf16 token gains nothing from
    // it; with fp32 x (the GGUF blocks' five dword loads per row) or dword scales the compiler
    // otherwise puts waits between the rows' loads (a row's registers reused for the last row).
    if constexpr (M >= 2 || XF32 || DW) __builtin_amdgcn_sched_barrier(0);
    // GGUF rows with fp32 x (the reference ABI): when every active lane's x chunk is bf16-exact, as the
    // reference engine's x is (stbl_act_quant_fp8 writes e4m3 codes times powers of two,
    // stbl/kernels.cu:54-63), the products take the packed-bf16 path (one conversion and one
    // v_dot2_f32_bf16 per two weights instead of one conversion and two FMAs; the products are exact
    // either way). xg[j] packs elements j and j + 16, the two nibbles of GGUF code byte j. Only the
    // batched launches' 8- and 16-row tiles take it: with the one-round tiles of single GEMVs, whose
    // time is load latency, the check and the second code path cost more than they save (2304x5120:
    // 4.59 -> 4.87 us with random fp32 x).
    constexpr bool kGgufX = F == WFmt::FP4_GGUF && XF32 && M == 1 && (R == 8 || R == 16);
    bool gguf_bf16 = false;  // wave-uniform
    [[maybe_unused]] uint32_t xg[kGgufX ? 16 : 1];
    if constexpr (kGgufX) {
        uint32_t low = 0;
#pragma unroll
        for (int i = 0; i < 32; i++) low |= __float_as_uint(xf[0][i]);
        gguf_bf16 = __builtin_amdgcn_ballot_w64(active && (low & 0xffffu) != 0) == 0;
#pragma unroll
        for (int j = 0; j < 16; j++) xg[j] = (__float_as_uint(xf[0][j]) >> 16) | (__float_as_uint(xf[0][j + 16]) & 0xffff0000u);
    }
    if constexpr (F == WFmt::FP4_GGUF) {
#pragma unroll
        for (int r = 0; r < R; r++) realign_gguf(graw[r], sb[r], w[r]);
    }
    float lscale = 1.f;  // FP8: one block scale per lane for the whole tile
    if constexpr (F == WFmt::FP8_B128)
        lscale = ((const float *)J.s)[(size_t)(row0 >> 7) * ((k + 127) >> 7) + ((cc * 16) >> 7)];
    uint32_t lsb = 0;
    if constexpr (F == WFmt::FP8_E8M0) lsb = ((const uint8_t *)J.s)[(size_t)(row0 >> 5) * (k >> 5) + ((cc * 16) >> 5)];
    if constexpr (kStageScales) {
#pragma unroll
        for (int i = 0; i < kScaleLoads; i++) {
            const int u = threadIdx.x + i * blockDim.x;
            lds_sc[u < sc_units ? u : kScaleUnits] = scv[i];
        }
        __syncthreads();
        const uint8_t *sl = (const uint8_t *)lds_sc + (((uintptr_t)J.s + (size_t)row0 * nch) & 15);
#pragma unroll
        for (int r = 0; r < R; r++) sb[r] = sl[r * nch + cc];  // < R nch + 15: inside lds_sc
    }

    if constexpr (DW) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t d = (uint32_t)__builtin_amdgcn_ds_bpermute((r * 16 + (lane >> 2)) << 2, (int)sdw);
            sb[r] = (d >> (8 * (lane & 3))) & 255u;
        }
    }
    // 2. products, scales, masking; 3. lane reduction of all M * R values together (wave_sum_rows:
    //    lane L ends with value L >> (6 - log2 NV), padded with zeros to a power of two)
    constexpr int NV = pow2_at_least(M * R), kShift = 6 - log2_exact(NV);
    __shared__ float red[kMaxWaves][M * R];
    float vals[NV];
#pragma unroll
    for (int i = M * R; i < NV; i++) vals[i] = 0.f;
    // GGUF rows (the reference ABI) take each block's sum at scale 1 times the engine's decode of the
    // block's scale byte, the float with that exponent field (stbl/kernels.cu:32, :185): byte 0 gives
    // 0.0 and 255 +Inf (the block's sum times +Inf: +-Inf, or NaN for a zero sum), where E8M0 (and the
    // scaled conversions) read 2^-127 and NaN. For bytes 1..254 this is the same product as a scale
    // inside the conversions (a power of two), and measured no slower on the GGUF tiles (2304x5120
    // 4.48 -> 4.35 us; a ballot-guarded fix-up for 0 and 255 instead cost 4-6%).
    if constexpr (kGgufX) {
        if (gguf_bf16) {
#pragma unroll
            for (int r = 0; r < R; r++) vals[r] = active ? gguf_dot_bf16(w[r], xg, 1.0f) * __uint_as_float(sb[r] << 23) : 0.f;
        }
    }
#pragma unroll
    for (int r = 0; r < R && !gguf_bf16; r++) {
        // E8M0 scales (OCP FP4; FP8 E8M0 with bf16 x) go into the conversions; the GGUF blocks, the
        // FP8 fp32 block scale and the fp32-x FP8 path multiply the chunk sum
        float s[M];
        if constexpr (F == WFmt::FP4_GGUF) chunk_dot<F, M, CH>(s, w[r], xf, 1.0f);
        else if constexpr (XF32 && T::fp4) chunk_dot<F, M, CH>(s, w[r], xf, e8m0_cvt_scale(sb[r]));
        else if constexpr (XF32) chunk_dot<F, M, CH>(s, w[r], xf);
        else if constexpr (T::fp4) chunk_dot_packed<F, M, CH>(s, w[r], xw, e8m0_cvt_scale(sb[r]));
        else if constexpr (F == WFmt::FP8_E8M0) chunk_dot_packed<F, M, CH>(s, w[r], xw, e8m0_cvt_scale(lsb));
        else chunk_dot_packed<F, M, CH>(s, w[r], xw);
        float scale = 1.f;
        if constexpr (F == WFmt::FP4_GGUF) scale = __uint_as_float(sb[r] << 23);
        else if constexpr (F == WFmt::FP8_B128) scale = lscale;
        else if constexpr (F == WFmt::FP8_E8M0 && XF32) scale = lsb == 255 ? 1.f : __uint_as_float(lsb << 23);  // 0: 0.0
#pragma unroll
        for (int t = 0; t < M; t++) vals[t * R + r] = active ? s[t] * scale : 0.f;
    }
    if constexpr (F == WFmt::FP8_E8M0 && XF32) {
        // The reference engine decodes an E8M0 byte as the float with that exponent field
        // (stbl/kernels.cu:32, :127): 0 is 0.0 (the scale above) and 255 +Inf, where E8M0 itself
        // reads 2^-127 and NaN. It multiplies each 32-wide block's sum by it; a block is two lanes
        // (2i, 2i + 1) here, so a block with byte 255 (scale 1 above) takes the pair's sum times
        // +Inf (rare: the engine's converter rejects 255, tools/convert_official.py:167-168).
        const bool sp = active && lsb == 255;
        if (__builtin_amdgcn_ballot_w64(sp)) {
#pragma unroll
            for (int i = 0; i < M * R; i++) {
                const float pair = vals[i] + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(
                                                 __builtin_bit_cast(int, vals[i]), 0xb1, 0xf, 0xf, false));
                vals[i] = sp ? ((lane & 1) ? 0.f : pair * __builtin_inff()) : vals[i];
            }
        }
    }
    const float mine = wave_sum_rows<NV>(vals);
    const int vi = lane >> kShift;
    const bool holder = (lane & ((1 << kShift) - 1)) == 0 && vi < M * R;
    auto store = [&](int i, float v) {
        const int t = i / R, r = i % R;
        if (row0 + r >= rows) return;
        const size_t at = (size_t)t * rows + row0 + r;
        if (out_mode == OUT_BF16) ((uint16_t *)J.y)[at] = f32_to_bf16_bits(v);
        else if (out_mode == OUT_F32) ((float *)J.y)[at] = v;
        else ((float *)J.y)[at] = bf16_round(v);
    };
    if (waves == 1) {
        if (holder) store(vi, mine);
        return;
    }
    if (holder) red[wave][vi] = mine;
    __syncthreads();
    if ((int)threadIdx.x < M * R) {
        const int i = threadIdx.x;
        float acc = red[0][i];
        for (int v = 1; v < waves; v++) acc += red[v][i];
        store(i, acc);
    }
}

// fp32 GEMV (the router's logits, stbl/kernels.cu:206-214): y[r] = sum_k x[k] w[r][k], optionally
// rounded to bf16. One 256-thread workgroup per row; with VEC (k % 4 == 0, 16-byte aligned w and x)
// every thread issues up to 8 16-byte loads of the row at once, else it strides the row one float at
// a time. Lanes reduce with DPP and the 4 waves through LDS in wave order.
template <bool VEC>
__global__ __launch_bounds__(256) void k_gemv_f32(float *__restrict__ y, const float *__restrict__ w,
                                                  const float *__restrict__ x, int k, int round_out) {
    __shared__ float red[4];
    const float *wr = w + (size_t)blockIdx.x * k;
    float acc = 0.f;
    if constexpr (VEC) {
        const int n4 = k >> 2;
        for (int base = threadIdx.x; base < n4; base += 256 * 8) {
            f32x4 wv[8], xv[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = base + 256 * u, ic = i < n4 ? i : 0;
                wv[u] = __builtin_bit_cast(f32x4, ld_stream(wr + 4 * (size_t)ic));
                xv[u] = *(const f32x4 *)(x + 4 * (size_t)ic);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (base + 256 * u >= n4) continue;
#pragma unroll
                for (int e = 0; e < 4; e++) acc = fmaf(xv[u][e], wv[u][e], acc);
            }
        }
    } else {
        for (int i = threadIdx.x; i < k; i += 256) acc = fmaf(x[i], wr[i], acc);
    }
    acc = dpp_sum(acc);
    if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        const float v = ((red[0] + red[1]) + red[2]) + red[3];
        y[blockIdx.x] = round_out ? bf16_round(v) : v;
    }
}

// bf16-weight GEMV (stbl/kernels.cu:193-204, the attention output and the head): y[r] = sum_i
// x_r[i] * w[r][i] with x_r = x + (r / group_rows) * k when group_rows > 0 (the block-diagonal wo_a
// product), fp32 accumulation, bf16-rounded when round_out. A wave owns R rows (which share one x
// row: group_rows % R == 0); with VEC (k % 8 == 0, 16-byte aligned w rows and x) every lane streams
// 16-byte units of 8 weights, U units of each row in flight, else one element at a time.
template <int R, bool VEC>
__global__ __launch_bounds__(256) void k_gemv_bf16(float *__restrict__ y, const uint16_t *__restrict__ w,
                                                   const float *__restrict__ x, int rows, int k, int round_out,
                                                   int group_rows) {
    constexpr int U = 4;
    const int lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (row0 >= rows) return;  // a whole wave
    const float *xr = x + (group_rows > 0 ? (size_t)(row0 / group_rows) * k : 0);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    if constexpr (VEC) {
        const int n8 = k >> 3;
        for (int base = lane; base < n8; base += 64 * U) {
            u32x4 wv[R][U];
            f32x4 xv[U][2];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = base + 64 * u, ic = i < n8 ? i : 0;
                xv[u][0] = *(const f32x4 *)(xr + 8 * (size_t)ic);
                xv[u][1] = *(const f32x4 *)(xr + 8 * (size_t)ic + 4);
#pragma unroll
                for (int r = 0; r < R; r++)
                    wv[r][u] = ld_stream(w + (size_t)min(row0 + r, rows - 1) * k + 8 * (size_t)ic);
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                if (base + 64 * u >= n8) continue;
#pragma unroll
                for (int r = 0; r < R; r++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        acc[r] = fmaf(xv[u][j >> 1][2 * (j & 1)], bf16_lo(wv[r][u][j]), acc[r]);
                        acc[r] = fmaf(xv[u][j >> 1][2 * (j & 1) + 1], bf16_hi(wv[r][u][j]), acc[r]);
                    }
            }
        }
    } else {
        for (int i = lane; i < k; i += 64)
#pragma unroll
            for (int r = 0; r < R; r++)
                acc[r] = fmaf(xr[i], bf16_bits_to_f32(w[(size_t)min(row0 + r, rows - 1) * k + i]), acc[r]);
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float tot = dpp_sum(acc[r]);
        if (lane == 63 && row0 + r < rows) y[row0 + r] = round_out ? bf16_round(tot) : tot;
    }
}

// Reference-ABI GEMVs over any K (stbl/kernels.cu:104-131 and :159-189 loop over K in 32-block
// slices): the one-pass tiles above hold at most kMaxWaves * 64 chunks per row, so longer rows
// (FP8 K > 8192, GGUF FP4 K > 16384; no call site of the reference engine has them) take this
// kernel. A 256-thread workgroup owns R rows; thread j sums the 32-element blocks j, j + 256, ... of
// each row: the block's products at scale 1 (the same conversions as the tiles), times the engine's
// decode of the block's scale byte (the float with that exponent field: 0 gives 0.0, 255 +Inf,
// stbl/kernels.cu:32), added to the row's running sum. Lanes reduce with DPP, the 4 waves through
// LDS in wave order. GGUF: w [rows][k/32][17]; FP8: w [rows][k] e4m3 with E8M0 bytes
// [(rows+31)/32][k/32] in the job's s. x fp32 [k].
template <bool GGUF, int R>
__global__ __launch_bounds__(256) void k_gemv_abi_longk(GemvJobs jobs, int rows, int k, int out_mode) {
    const GemvJob J = jobs.j[blockIdx.y];
    const int nblk = k >> 5, row0 = blockIdx.x * R;
    const float *x = (const float *)J.x;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    for (int b = threadIdx.x; b < nblk; b += 256) {
        float xf[1][32];
        load_x<true, 1, 32>(xf, x, k, b * 32);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const size_t row = (size_t)min(row0 + r, rows - 1);
            float bsum;
            uint32_t sbyte;
            if constexpr (GGUF) {
                u32x4 codes;
                load_gguf_block(J.w + row * (size_t)nblk * 17 + (size_t)b * 17, sbyte, codes);
                float s[1];
                chunk_dot<WFmt::FP4_GGUF, 1, 32>(s, codes, xf, 1.0f);
                bsum = s[0];
            } else {
                const uint8_t *p = J.w + row * (size_t)k + (size_t)b * 32;
                const u32x4 w0 = ld_stream(p), w1 = ld_stream(p + 16);
                sbyte = ((const uint8_t *)J.s)[(row >> 5) * (size_t)nblk + b];
                float lo[1][16], hi[1][16], s0[1], s1[1];
#pragma unroll
                for (int i = 0; i < 16; i++) lo[0][i] = xf[0][i], hi[0][i] = xf[0][16 + i];
                chunk_dot<WFmt::FP8_E8M0, 1, 16>(s0, w0, lo);
                chunk_dot<WFmt::FP8_E8M0, 1, 16>(s1, w1, hi);
                bsum = s0[0] + s1[0];
            }
            acc[r] += bsum * __uint_as_float((sbyte & 0xffu) << 23);
        }
    }
    __shared__ float red[4][R];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int r = 0; r < R; r++) {
        const float t = dpp_sum(acc[r]);
        if (lane == 63) red[wave][r] = t;
    }
    __syncthreads();
    if ((int)threadIdx.x < R && row0 + (int)threadIdx.x < rows) {
        const int r = threadIdx.x;
        const float v = ((red[0][r] + red[1][r]) + red[2][r]) + red[3][r];
        ((float *)J.y)[row0 + r] = out_mode == OUT_F32 ? v : bf16_round(v);
    }
}

static inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// The reference ABI's rows beyond the one-pass tiles' K (see k_gemv_abi_longk).
template <bool GGUF>
static hipError_t launch_longk(const GemvJobs &jobs, int njobs, int rows, int k, int out_mode, hipStream_t st) {
    hipLaunchKernelGGL((k_gemv_abi_longk<GGUF, 4>), dim3(ceil_div(rows, 4), njobs), dim3(256), 0, st, jobs, rows, k,
                       out_mode);
    return hipGetLastError();
}

template <WFmt F, bool XF32, int M, int R>
static hipError_t launch_r(const GemvJobs &jobs, int njobs, int rows, int k, int out_mode, hipStream_t st) {
    const int nch = k / WTraits<F>::CH, waves = ceil_div(nch, 64);
    const dim3 grid(ceil_div(rows, R), njobs), block(64 * waves);
    if constexpr (F == WFmt::FP4_OCP && R == 4 && M >= 2) {
        bool dw = nch % 4 == 0;
        for (int j = 0; j < njobs; j++) dw = dw && ((uintptr_t)jobs.j[j].s & 3) == 0;
        if (dw) {
            hipLaunchKernelGGL((k_gemv<F, XF32, M, R, true>), grid, block, 0, st, jobs, rows, k, out_mode);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((k_gemv<F, XF32, M, R, false>), grid, block, 0, st, jobs, rows, k, out_mode);
    return hipGetLastError();
}

// Compute units of the current device (256 on MI355X), read once per device.
static int device_cus() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Rows per workgroup for 2-4 tokens of bf16 x (FP4 and FP8 with 128x128 scales). A lane's x chunk
// is M times one token's and every row of the tile reuses it, so taller tiles cut the x bytes the
// vector L1 takes in per weight byte (4 M / R for FP4, 2 M / R for FP8), while shorter ones keep
// more waves in flight per CU. Chosen from a sweep that forced each height in turn (rows 512-16384,
// K 1024-7168, M = 2-4): the tallest tile that still gives each CU a number of tiles depending on
// the format and the waves per row (us at M = 4 for 2 / 4 / 8 rows):
//   FP4, rows of 4+ waves, and FP8 of 5+: 8 or 4 rows while every CU gets one (FP4 2048x7168 6.70 /
//     5.54 / 5.21, 512x7168 3.37 / 3.73 / 4.63; FP8 2048x7168 7.09 / 6.14 / 6.08);
//   FP4, rows of 1-3 waves: while every CU gets four (7168x2048 5.75 / 4.74 / 4.82, 16384x2048
//     10.31 / 7.98 / 7.73, 16384x1024 8.88 / 7.05 / 6.32, 4096x4096 6.44 / 5.33 / 6.16);
//   FP8, rows of 3-4 waves, 3-4 tokens: 8 rows while every CU gets two, 4 while it gets one
//     (2048x4096 4.77 / 4.29 / 4.65, 4096x4096 7.31 / 6.34 / 6.22; with 2 tokens 8 rows win at
//     2048x4096: 3.91 / 3.89 / 3.76);
//   FP8, rows of 1-2 waves: never 8 rows; 4 while every CU gets four, or six for rows of one wave
//     or 2 tokens (7168x2048 6.18 / 5.67 / 6.05, 2048x2048 3.27 / 3.62 / 3.88; 4096x1024 3.19 /
//     3.21, 2 tokens 4096x2048 3.59 / 3.66).
// A height of 16 was slower everywhere at M = 2 (no gain for FP8, 2-4x slower for FP4).
template <WFmt F, int M>
static int multi_token_rows(int rows, int njobs, int k) {
    static_assert(F == WFmt::FP4_OCP || F == WFmt::FP8_B128, "bf16-x formats only");
    const long cus = device_cus();
    const int waves = ceil_div(k / WTraits<F>::CH, 64);
    const long tiles8 = (long)ceil_div(rows, 8) * njobs, tiles4 = (long)ceil_div(rows, 4) * njobs;
    long per_cu8 = 1, per_cu4 = 1;  // tiles each CU must get for the height (0: never)
    if constexpr (F == WFmt::FP4_OCP) {
        if (waves < 4) per_cu8 = per_cu4 = 4;
    } else if (waves < 3) {
        per_cu8 = 0;
        per_cu4 = waves == 1 || M == 2 ? 6 : 4;
    } else if (waves < 5 && M > 2) {
        per_cu8 = 2;
    }
    if (per_cu8 > 0 && tiles8 >= per_cu8 * cus) return 8;
    if (tiles4 >= per_cu4 * cus) return 4;
    return 2;
}

// Rows per workgroup for one token. A launch with much more work (batched matrices) takes 8 rows per
// workgroup, so the fixed per-workgroup cost (x chunk, prologue, reduction) is spread over 4x the
// weight bytes while still leaving thousands of workgroups. Otherwise 4 rows halve the x loads per
// weight byte, unless that leaves the busiest CU more rows than 2-row tiles would (workgroups come
// in whole rounds over the CUs: 2304 rows are 2.25 rounds of 4-row tiles but 4.5 of 2-row ones)
// or a row takes too few waves: one wave (FP4 K <= 2048) or, for FP8, whose x chunk per weight
// byte is half FP4's, two. Measured (M = 1, us, 2 -> 4 rows): FP4 2048x7168 4.01 -> 3.84,
// 5120x2304 3.98 -> 3.84, 7168x2048 3.71 -> 3.99, 2304x5120 3.64 -> 3.84; FP8 2048x7168 4.73 ->
// 4.66, 7168x2048 4.52 -> 4.58.
template <WFmt F, bool XF32, int M>
static hipError_t launch(const GemvJobs &jobs, int njobs, int rows, int k, int out_mode, hipStream_t st) {
    if constexpr (M > 2 && XF32) {
        return launch_r<F, XF32, M, 1>(jobs, njobs, rows, k, out_mode, st);
    } else if constexpr (M >= 2 && !XF32) {
        switch (multi_token_rows<F, M>(rows, njobs, k)) {
            case 8: return launch_r<F, XF32, M, 8>(jobs, njobs, rows, k, out_mode, st);
            case 4: return launch_r<F, XF32, M, 4>(jobs, njobs, rows, k, out_mode, st);
            default: return launch_r<F, XF32, M, 2>(jobs, njobs, rows, k, out_mode, st);
        }
    }
    else if constexpr (XF32) {
        // fp32 activations (the reference ABI): a lane's x chunk is 4-8x its weight bytes per row, so
        // 4 rows share it (measured 2-8% faster than 2 at 2304x5120 and 5120x2304; 8 gains nothing
        // there), and 8 in launches with much more work: the engine's expert batches (12 x 2304x5120
        // 32.7 -> 24.8 us, 6 x 5120x2304 17.0 -> 14.3, 16 x 2048x7168 52.2 -> 37.0). The largest GGUF
        // FP4 launches take 16 (12 x 2304x5120 25.3 -> 23.3 us, 16 x 2048x7168 38.1 -> 31.5); FP8
        // E8M0 at 32768x1280 was 5% slower with 16, so it keeps 8.
        const long wgs8 = (long)ceil_div(rows, 8) * njobs * ceil_div(k / WTraits<F>::CH, 64);
        if constexpr (F == WFmt::FP4_GGUF) {
            // 9-10 rows per CU: tiles of exactly that many rows make the launch one round over the CUs,
            // so each CU reads the fp32 x chunk (twice the weight bytes of a 4-row tile) once, not 3
            // times (2304x5120: 5.99 -> 5.06 us; 9-10 rows are 53-58 loads per lane, within the
            // limit of loads in flight; 20 rows per CU, as at 5120x2304, are not: 5.47 -> 7.9 us)
            const long per_cu = ((long)rows * njobs + device_cus() - 1) / device_cus();
            if (per_cu == 9) return launch_r<F, XF32, M, 9>(jobs, njobs, rows, k, out_mode, st);
            if (per_cu == 10) return launch_r<F, XF32, M, 10>(jobs, njobs, rows, k, out_mode, st);
        }
        if constexpr (F == WFmt::FP4_GGUF)
            if (wgs8 >= 8192) return launch_r<F, XF32, M, 16>(jobs, njobs, rows, k, out_mode, st);
        if (wgs8 >= 4096) return launch_r<F, XF32, M, 8>(jobs, njobs, rows, k, out_mode, st);
        // small matrices, whose 4-row tiles would leave CUs idle, take 2 or 1 rows (FP8 512x5120
        // 3.23 -> 2.89 us, 1000x1280 2.80 -> 2.59; GGUF FP4 512x2560 3.32 -> 3.03)
        const int cus = device_cus();
        if ((long)ceil_div(rows, 4) * njobs < cus) {
            if ((long)ceil_div(rows, 2) * njobs < cus) return launch_r<F, XF32, M, 1>(jobs, njobs, rows, k, out_mode, st);
            return launch_r<F, XF32, M, 2>(jobs, njobs, rows, k, out_mode, st);
        }
        return launch_r<F, XF32, M, 4>(jobs, njobs, rows, k, out_mode, st);
    } else {
        const long wgs8 = (long)ceil_div(rows, 8) * njobs * ceil_div(k / WTraits<F>::CH, 64);
        if (wgs8 >= 8192) {
            // FP4 rows of 2+ waves: 16 rows (16 x 2048x7168: 21.4 -> 21.0 us, 64 x 76.4 -> 73.6; 64 x
            // 5120x2304, whose second wave has 8 chunks, 93.7 -> 82.8; 2304x5120 within the spread
            // between runs); rows of one wave lose (16 x 7168x2048 20.3 -> 21.1). FP8 rows of 1-2
            // waves take 4 rows (16 x 7168x2048 36.1 -> 35.3 us, 64 x 140.8 -> 137.1), longer ones 8
            // (64 x 2048x7168 137.0, 140.6 with 4).
            if constexpr (F == WFmt::FP4_OCP)
                if (k / WTraits<F>::CH > 64) return launch_r<F, XF32, M, 16>(jobs, njobs, rows, k, out_mode, st);
            if constexpr (F == WFmt::FP8_B128)
                if (k / WTraits<F>::CH <= 128) return launch_r<F, XF32, M, 4>(jobs, njobs, rows, k, out_mode, st);
            return launch_r<F, XF32, M, 8>(jobs, njobs, rows, k, out_mode, st);
        }
        const int cus = device_cus();
        // FP4 rows of one wave: rows of at most 32 chunks (K <= 1024) use half the lanes of their
        // workgroup, so a 2-row tile has little in flight: 8-row tiles wherever each CU still gets two
        // (us, 2 -> 8 rows: 32768x1024 7.12 -> 5.49, 16384x1024 4.69 -> 3.87, 7168x1024 3.27 -> 3.03,
        // 4096x1024 2.83 -> 2.75; at 3072x1024, 1.5 tiles per CU, 2.63 -> 2.67). Rows of 33-64 chunks
        // take 8 rows wherever each CU gets eight tiles (16384x2048 5.22 -> 4.70), else 4 wherever it
        // gets four (7168x2048 3.55 -> 3.46, 7168x1536 3.43 -> 3.30, 9216x2048 with 8 rows 3.86 ->
        // 3.80; 5120x2048 and 4096x2048 within 0.01 us)
        if constexpr (F == WFmt::FP4_OCP) {
            const long tiles8 = (long)ceil_div(rows, 8) * njobs, tiles4 = (long)ceil_div(rows, 4) * njobs;
            const int nch = k / WTraits<F>::CH;
            if ((nch <= 32 && tiles8 >= 2L * cus) || (nch <= 64 && tiles8 >= 8L * cus))
                return launch_r<F, XF32, M, 8>(jobs, njobs, rows, k, out_mode, st);
            if (nch > 32 && nch <= 64 && tiles4 >= 4L * cus)
                return launch_r<F, XF32, M, 4>(jobs, njobs, rows, k, out_mode, st);
        }
        // one token of FP4 over rows of 4+ waves: 8-row tiles when they still fill every CU, halving the
        // x reads per weight byte again (2048x7168 3.85 -> 3.80 us; rows of one wave lose: 7168x2048
        // 3.73 -> 4.62 us)
        if constexpr (F == WFmt::FP4_OCP)
            if (k / WTraits<F>::CH > 3 * 64 && (long)ceil_div(rows, 8) * njobs >= cus)
                return launch_r<F, XF32, M, 8>(jobs, njobs, rows, k, out_mode, st);
        const long busiest2 = ceil_div(ceil_div(rows, 2) * njobs, cus) * 2L;
        const long busiest4 = ceil_div(ceil_div(rows, 4) * njobs, cus) * 4L;
        // FP4 rows of 2-3 waves: 8-row tiles when they leave the busiest CU no more rows than 4-row
        // ones and come in one round over the CUs or in four or more, never in between (4096x4096,
        // two rounds: 3.74 -> 3.91 us; 3072x3072 3.28 -> 3.58). Against 4- or 2-row tiles at K 3072-
        // 6144: 2048 rows (one round) 3.13-3.56 -> 2.93-3.25 us, 16384 rows 3-8% faster, 8192 rows -5%
        // to +0.6%, 1536 rows -5% to +3%
        if constexpr (F == WFmt::FP4_OCP) {
            const int nch = k / WTraits<F>::CH;
            const long tiles8 = (long)ceil_div(rows, 8) * njobs;
            const long busiest8 = (tiles8 + cus - 1) / cus * 8L;
            if (nch > 64 && nch <= 3 * 64 && busiest8 <= busiest4 && (tiles8 <= cus || tiles8 >= 4L * cus))
                return launch_r<F, XF32, M, 8>(jobs, njobs, rows, k, out_mode, st);
        }
        const int min_waves = F == WFmt::FP4_OCP ? 2 : 3;
        if (ceil_div(k / WTraits<F>::CH, 64) >= min_waves && busiest4 <= busiest2)
            return launch_r<F, XF32, M, 4>(jobs, njobs, rows, k, out_mode, st);
        return launch_r<F, XF32, M, 2>(jobs, njobs, rows, k, out_mode, st);
    }
}

// v2 dispatch over the token count: n <= 16 same-shape matrices (host arrays of device pointers).
template <WFmt F>
static int gemv_v2(const char *name, void *const *y, const void *const *w, const void *const *s,
                   const void *const *x, int n, int m, int rows, int k, int y_f32, hipStream_t st) {
    constexpr int CH = WTraits<F>::CH;
    if (!y || !w || !s || !x || n < 1 || n > kMaxJobs)
        return abi_fail(hipErrorInvalidValue, "%s: need 1..%d matrices (n=%d)", name, kMaxJobs, n);
    if (rows <= 0 || k <= 0 || k % CH != 0 || k / CH > kMaxWaves * 64)
        return abi_fail(hipErrorInvalidValue, "%s: need k %% %d == 0 and 0 < k <= %d (k=%d)", name, CH,
                        kMaxWaves * 64 * CH, k);
    if (m < 1 || m > 4) return abi_fail(hipErrorInvalidValue, "%s: m must be 1..4 (m=%d); use the GEMM for more", name, m);
    GemvJobs jobs = {};
    for (int j = 0; j < n; j++) {
        if (!y[j] || !w[j] || !s[j] || !x[j]) return abi_fail(hipErrorInvalidValue, "%s: matrix %d: null pointer", name, j);
        if (!aligned16(w[j]) || !aligned16(x[j]))
            return abi_fail(hipErrorInvalidValue, "%s: matrix %d: weights and x must be 16-byte aligned", name, j);
        jobs.j[j] = GemvJob{(const uint8_t *)w[j], s[j], x[j], y[j]};
    }
    const int mode = y_f32 ? OUT_F32 : OUT_BF16;
    hipError_t e;
    switch (m) {
        case 1: e = launch<F, false, 1>(jobs, n, rows, k, mode, st); break;
        case 2: e = launch<F, false, 2>(jobs, n, rows, k, mode, st); break;
        case 3: e = launch<F, false, 3>(jobs, n, rows, k, mode, st); break;
        default: e = launch<F, false, 4>(jobs, n, rows, k, mode, st); break;
    }
    return abi_status(e, name);
}

}  // namespace stbl

using namespace stbl;

extern "C" {

int stbl_amd_gemv_fp4(void *y, const void *codes, const void *scales, const void *x, int m, int rows, int k,
                      int y_f32, hipStream_t st) {
    const void *sc = scales;
    return gemv_v2<WFmt::FP4_OCP>("gemv_fp4", &y, &codes, &sc, &x, 1, m, rows, k, y_f32, st);
}

int stbl_amd_gemv_fp8(void *y, const void *codes, const float *scales, const void *x, int m, int rows, int k,
                      int y_f32, hipStream_t st) {
    const void *sc = scales;
    return gemv_v2<WFmt::FP8_B128>("gemv_fp8", &y, &codes, &sc, &x, 1, m, rows, k, y_f32, st);
}

// n <= 16 same-shape GEMVs in one launch (the batching of stbl_gemv_mxfp4_batch, stbl/kernels.h:18-20,
// in the v2 formats). All pointer arguments are HOST arrays of n device pointers.
int stbl_amd_gemv_fp4_batch(void *const *y, const void *const *codes, const void *const *scales, const void *const *x,
                            int n, int m, int rows, int k, int y_f32, hipStream_t st) {
    return gemv_v2<WFmt::FP4_OCP>("gemv_fp4_batch", y, codes, scales, x, n, m, rows, k, y_f32, st);
}

int stbl_amd_gemv_fp8_batch(void *const *y, const void *const *codes, const void *const *scales, const void *const *x,
                            int n, int m, int rows, int k, int y_f32, hipStream_t st) {
    return gemv_v2<WFmt::FP8_B128>("gemv_fp8_batch", y, codes, scales, x, n, m, rows, k, y_f32, st);
}

// stbl/kernels.h:14-15. Requires k % 32 == 0 and 16-byte aligned rows, as the reference does.
void stbl_gemv_fp8(float *y, const void *w, const void *scale, const float *x, int rows, int k, int round_out,
                   hipStream_t st) {
    if (!y || !w || !scale || !x || rows <= 0 || k <= 0 || k % 32 != 0 || !aligned16(w) || !aligned16(x)) {
        abi_fail(hipErrorInvalidValue, "stbl_gemv_fp8: bad arguments (rows=%d k=%d)", rows, k);
        return;
    }
    GemvJobs jobs = {};
    jobs.j[0] = GemvJob{(const uint8_t *)w, scale, x, y};
    const int mode = round_out ? OUT_F32_ROUNDED : OUT_F32;
    if (k / 16 > kMaxWaves * 64) abi_status(launch_longk<false>(jobs, 1, rows, k, mode, st), "stbl_gemv_fp8 launch");
    else abi_status(launch<WFmt::FP8_E8M0, true, 1>(jobs, 1, rows, k, mode, st), "stbl_gemv_fp8 launch");
}

// stbl/kernels.h:19-20. n <= 16 same-shape matrices in one launch; needs k % 256 == 0 and w 8-byte
// aligned (the reference's preconditions, stbl/kernels.cu:138-139). y, w, x are host arrays.
void stbl_gemv_mxfp4_batch(float *const *y, const void *const *w, const float *const *x, int n, int rows, int k,
                           hipStream_t st) {
    if (!y || !w || !x || n <= 0 || n > kMxBatch || rows <= 0 || k <= 0 || k % 256 != 0) {
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
    if (k / 32 > kMaxWaves * 64)
        abi_status(launch_longk<true>(jobs, n, rows, k, OUT_F32_ROUNDED, st), "stbl_gemv_mxfp4_batch launch");
    else
        abi_status(launch<WFmt::FP4_GGUF, true, 1>(jobs, n, rows, k, OUT_F32_ROUNDED, st), "stbl_gemv_mxfp4_batch launch");
}

// stbl/kernels.h:16.
void stbl_gemv_mxfp4(float *y, const void *w, const float *x, int rows, int k, hipStream_t st) {
    stbl_gemv_mxfp4_batch(&y, &w, &x, 1, rows, k, st);
}

// stbl/kernels.h:21-22 (bf16 weights; group_rows > 0: row r reads x + (r / group_rows) * k). Any k;
// the 16-byte path when k % 8 == 0 and w, x are 16-byte aligned.
void stbl_gemv_bf16(float *y, const void *w, const float *x, int rows, int k, int round_out, int group_rows,
                    hipStream_t st) {
    if (!y || !w || !x || rows <= 0 || k <= 0 || group_rows < 0) {
        abi_fail(hipErrorInvalidValue, "stbl_gemv_bf16: bad arguments (rows=%d k=%d group_rows=%d)", rows, k, group_rows);
        return;
    }
    const bool vec = k % 8 == 0 && aligned16(w) && aligned16(x);
    const bool two = group_rows == 0 || group_rows % 2 == 0;  // two rows per wave must share an x row
    const dim3 grid(ceil_div(rows, 4 * (two ? 2 : 1)));
    const uint16_t *wb = (const uint16_t *)w;
    if (vec && two) hipLaunchKernelGGL((k_gemv_bf16<2, true>), grid, dim3(256), 0, st, y, wb, x, rows, k, round_out, group_rows);
    else if (vec) hipLaunchKernelGGL((k_gemv_bf16<1, true>), grid, dim3(256), 0, st, y, wb, x, rows, k, round_out, group_rows);
    else if (two) hipLaunchKernelGGL((k_gemv_bf16<2, false>), grid, dim3(256), 0, st, y, wb, x, rows, k, round_out, group_rows);
    else hipLaunchKernelGGL((k_gemv_bf16<1, false>), grid, dim3(256), 0, st, y, wb, x, rows, k, round_out, group_rows);
    abi_status(hipGetLastError(), "stbl_gemv_bf16 launch");
}

// stbl/kernels.h:23 (the router's logits, stbl/model.cu:430). Any k; the 16-byte path when k % 4 == 0
// and w, x are 16-byte aligned.
void stbl_gemv_f32(float *y, const float *w, const float *x, int rows, int k, int round_out, hipStream_t st) {
    if (!y || !w || !x || rows <= 0 || k <= 0) {
        abi_fail(hipErrorInvalidValue, "stbl_gemv_f32: bad arguments (rows=%d k=%d)", rows, k);
        return;
    }
    if (k % 4 == 0 && aligned16(w) && aligned16(x))
        hipLaunchKernelGGL(k_gemv_f32<true>, dim3(rows), dim3(256), 0, st, y, w, x, k, round_out);
    else
        hipLaunchKernelGGL(k_gemv_f32<false>, dim3(rows), dim3(256), 0, st, y, w, x, k, round_out);
    abi_status(hipGetLastError(), "stbl_gemv_f32 launch");
}

}  // extern "C"
