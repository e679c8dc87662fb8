// Expert FFN and routed-MoE kernels over quantized expert slots (layout: expert_layout.hpp).
//
// The reference engine runs one MoE layer as (stbl/model.cu:426-594):
//   router scores -> host top-k -> for the cached and then the refilled experts:
//   gemv_mxfp4_batch(gate, up) -> swiglu_batch(route weights) -> act_quant_fp8(mid) ->
//   gemv_mxfp4_batch(down) -> shared expert -> axpy of every expert output in top-k order, then the
//   shared one -> round_bf16.
// Here the same arithmetic runs as three launches over a job table (one job = one expert slot and
// the <= 4 tokens routed to it, each token with its own route weight):
//   k_moe_gateup  gate and up rows of a job in the same workgroup; the epilogue rounds both to bf16
//                 and applies SwiGLU with the token's route weight (stbl/kernels.cu:444-459), so
//                 the gate/up outputs never leave the chip;
//   k_moe_down    down rows of a job; output rounded to bf16 as the reference's GEMV does;
//   k_moe_combine per token, the fp32 sum of its experts' outputs in top-k order plus the shared
//                 expert's, rounded to bf16 (stbl/model.cu:589-592).
// Jobs are compiled per token class (1, 2 or 3-4 tokens). A step whose jobs of one format span
// several classes runs them all in one gate/up and one down launch (k_moe_gateup_any /
// k_moe_down_any); otherwise each class has its launches, one launch holding both formats where a
// class has FP4 and FP8 E8M0 jobs (k_moe_gateup_mix / k_moe_down_mix).
// In the reference's "official" numerics the expert input and the SwiGLU output are quantized to FP8
// per 32 first (stbl/model.cu:510, :538); both kernels do that quantization in registers on the
// lane's own chunk of the activation, so it costs no launch and no memory traffic.
// The router is k_route: sigmoid scores, top-k by score + bias with ties to the lower id, weights
// renormalized in top-k order (stbl/model.cu:444-451, :528-530 with sigmoid for sqrt-softplus).
#include <algorithm>
#include <mutex>

#include "abi_util.hpp"
#include "expert_layout.hpp"
#include "gemv_core.hpp"

namespace stbl {

constexpr int kMoeMaxTok = 4;    // tokens per job
constexpr int kMoeMaxJobs = 40;  // jobs per launch
constexpr int kMoeMaxT = 16;     // tokens per MoE call
constexpr int kMoeMaxPick = 17;  // top-k + shared

struct MoeJob {
    const uint8_t *slot;
    int fmt;                   // the slot's format (ExpertFmt); read by the mixed-format kernels
    int m;                     // tokens of this job, 1..4
    int tok[kMoeMaxTok];       // token rows of x
    int pair[kMoeMaxTok];      // rows of the intermediate / output buffers
    float w[kMoeMaxTok];       // route weight of each token
};
struct MoeJobs {
    MoeJob j[kMoeMaxJobs];
};

// Weights of matrix `mat` (0 gate, 1 up, 2 down) of a slot.
template <WFmt F>
struct SlotMat {
    const uint8_t *codes;
    const uint8_t *scales;
    int rows, k;
    __device__ SlotMat(const uint8_t *slot, const ExpertLayout &L, int mat, int dim, int inter)
        : codes(slot + L.off[2 * mat]), scales(slot + L.off[2 * mat + 1]), rows(mat == 2 ? dim : inter),
          k(mat == 2 ? inter : dim) {}
    // 16 bytes of codes of row `row`, chunk cc, and the chunk's E8M0 scale byte (FP4 only)
    __device__ __forceinline__ void load(size_t row, int cc, u32x4 &w, uint32_t &sb) const {
        if constexpr (WTraits<F>::fp4) {
            w = ld_stream(codes + row * (size_t)(k >> 1) + (size_t)cc * 16);
            sb = ld_stream_u8(scales + row * (size_t)(k >> 5) + cc);
        } else {
            w = ld_stream(codes + row * (size_t)k + (size_t)cc * 16);
            sb = 0;
        }
    }
    __device__ __forceinline__ u32x4 load_codes(size_t row, int cc) const {
        return ld_stream(codes + row * (size_t)(WTraits<F>::fp4 ? k >> 1 : k) + (size_t)cc * 16);
    }
    // FP4, DW: dword `dwi` of row `row`'s scale bytes (rows are k/32 bytes, a multiple of 4)
    __device__ __forceinline__ uint32_t load_scale_dword(size_t row, int dwi) const {
        return __builtin_nontemporal_load((const uint32_t *)(scales + row * (size_t)(k >> 5)) + dwi);
    }
    // FP8: the lane's block scale for a tile whose rows share row0's 128-row (fp32 scales) or
    // 32-row (E8M0 scales, returned as the conversion scale of e8m0_cvt_scale) block
    __device__ __forceinline__ float block_scale(int row0, int cc) const {
        if constexpr (F == WFmt::FP8_E8M0)
            return e8m0_cvt_scale(scales[(size_t)(row0 >> 5) * (k >> 5) + ((cc * 16) >> 5)]);
        else return ((const float *)scales)[(size_t)(row0 >> 7) * ((k + 127) >> 7) + ((cc * 16) >> 7)];
    }
};

// Scale byte of virtual row vr for this lane, from the dwords lane j of the wave loaded (dword j % 16
// of virtual row 4 q + j / 16 in sdw[q]).
__device__ __forceinline__ uint32_t dw_scale_byte(const uint32_t *sdw, int vr, int lane) {
    const uint32_t d = (uint32_t)__builtin_amdgcn_ds_bpermute(((vr & 3) * 16 + (lane >> 2)) << 2, (int)sdw[vr >> 2]);
    return (d >> (8 * (lane & 3))) & 255u;
}

// A chunk's scale: E8M0 scales (FP4 bytes; FP8 E8M0 blocks, already a conversion scale) go into the
// conversions (conv_scale), the fp32 128x128 block scale multiplies the chunk sum (post_scale).
template <WFmt F>
__device__ __forceinline__ float conv_scale(uint32_t sb, float lscale) {
    if constexpr (WTraits<F>::fp4) return e8m0_cvt_scale(sb);
    else if constexpr (F == WFmt::FP8_E8M0) return lscale;
    else return 1.f;
}
template <WFmt F>
__device__ __forceinline__ float post_scale(float lscale) {
    if constexpr (F == WFmt::FP8_B128) return lscale;
    else return 1.f;
}

// Sums N per-lane values over the wave (wave_sum_rows, padded with zeros to a power of two) and over
// the waves: the first lane holding each value's wave total writes red[wave][i]; after the barrier
// thread i < N holds the total of value i in *out.
template <int N>
__device__ __forceinline__ bool wave_total(float (&vals)[N], float (*red)[N], float *out) {
    constexpr int NV = pow2_at_least(N), kShift = 6 - log2_exact(NV);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    float p[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) p[i] = i < N ? vals[i] : 0.f;
    const float mine = wave_sum_rows<NV>(p);
    const int vi = lane >> kShift;
    if ((lane & ((1 << kShift) - 1)) == 0 && vi < N) red[wave][vi] = mine;
    __syncthreads();
    const int i = threadIdx.x;
    if (i >= N) return false;
    float acc = red[0][i];
    for (int v = 1; v < waves; v++) acc += red[v][i];
    *out = acc;
    return true;
}

// The lane's products over its CPL chunks of 16 bytes (x words of chunk i: i * CH / 2 on), chunk by
// chunk.
template <WFmt F, int M, int CPL>
__device__ __forceinline__ void chunk_dot_lane(float (&s)[M], const u32x4 (&w)[CPL],
                                               const uint32_t (&xw)[M][WTraits<F>::CH * CPL / 2], float cs) {
    constexpr int CH = WTraits<F>::CH;
    if constexpr (CPL == 1) {
        chunk_dot_packed<F, M, CH>(s, w[0], xw, cs);
    } else {
#pragma unroll
        for (int t = 0; t < M; t++) s[t] = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; i++) {
            uint32_t part[M][CH / 2];
#pragma unroll
            for (int t = 0; t < M; t++)
#pragma unroll
                for (int j = 0; j < CH / 2; j++) part[t][j] = xw[t][i * CH / 2 + j];
            float si[M];
            chunk_dot_packed<F, M, CH>(si, w[i], part, cs);
#pragma unroll
            for (int t = 0; t < M; t++) s[t] += si[t];
        }
    }
}

// ---- gate/up + SwiGLU ----------------------------------------------------------------------------

// Job blockIdx.y, rows [row0, row0 + R) of gate and of up. x bf16 [T][dim] -> h bf16 [P][inter].
// DW (FP4, scale rows a multiple of 4 bytes): the scale bytes of the 2R rows come as dwords, lane j
// loading dword j % 16 of the wave's segment of row j / 16 (gate rows, then up rows), and each lane
// takes its byte with ds_bpermute; otherwise one byte load per row per lane.
// The body runs in any workgroup of at least ceil(dim / CH / 64) waves: waves past the job's K (in
// the mixed-format launches, whose workgroups are sized for the format with the most waves) load
// nothing and add zeros.
template <WFmt F, int M, int R, bool DW, int CPL = 1>
__device__ __forceinline__ void gateup_job(const MoeJob &J, const ExpertLayout &L, const uint16_t *__restrict__ x,
                                           uint16_t *__restrict__ h, int dim, int inter, float limit, int official,
                                           int tile0 = -1) {
    static_assert(CPL == 1 || !WTraits<F>::fp4, "two chunks per lane: FP8 rows");
    constexpr int CH = WTraits<F>::CH * CPL;  // elements per lane
    const SlotMat<F> G(J.slot, L, 0, dim, inter), U(J.slot, L, 1, dim, inter);
    const int lane = threadIdx.x & 63, c = (threadIdx.x >> 6) * 64 + lane, nch = dim / CH;
    const bool active = c < nch;
    const int cc = active ? c : 0;
    const int row0 = tile0 < 0 ? (int)blockIdx.x * R : tile0;  // the tile's first row
    const int m = J.m;
    // the output row and route weight of the (token, row) this thread may finish, read now: indexed
    // by thread they are memory loads, which at the end would add a round trip to every workgroup
    const int t_out = min((int)(threadIdx.x >> 1) / R, M - 1);
    const int pair_out = J.pair[t_out];
    const float w_out = J.w[t_out];
    __shared__ float red[kMaxWaves][2 * M * R];
    float tot[2 * M * R];
#pragma unroll
    for (int i = 0; i < 2 * M * R; i++) tot[i] = 0.f;
    if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * 64 < nch) {
        uint32_t xw[M][CH / 2];
#pragma unroll
        for (int t = 0; t < M; t++) {
            uint32_t tmp[1][CH / 2];
            load_x_packed<1, CH>(tmp, x + (size_t)J.tok[t < m ? t : 0] * dim, dim, cc * CH);
#pragma unroll
            for (int i = 0; i < CH / 2; i++) xw[t][i] = tmp[0][i];
        }
        u32x4 wg[R][CPL], wu[R][CPL];
        uint32_t sg[R], su[R];
        uint32_t sdw[(2 * R + 3) / 4];
        if constexpr (DW) {
            // virtual rows 0..R-1 gate, R..2R-1 up; rows and dwords clamped into the matrices
            const int wave = threadIdx.x >> 6, dwi = min(wave * 16 + (lane & 15), (nch >> 2) - 1);
#pragma unroll
            for (int q = 0; q < (2 * R + 3) / 4; q++) {
                const int vr = min(4 * q + (lane >> 4), 2 * R - 1);
                const size_t row = (size_t)min(row0 + (vr < R ? vr : vr - R), inter - 1);
                sdw[q] = vr < R ? G.load_scale_dword(row, dwi) : U.load_scale_dword(row, dwi);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const size_t row = (size_t)min(row0 + r, inter - 1);
                wg[r][0] = G.load_codes(row, cc);
                wu[r][0] = U.load_codes(row, cc);
            }
        } else {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const size_t row = (size_t)min(row0 + r, inter - 1);
#pragma unroll
                for (int i = 0; i < CPL; i++) {
                    G.load(row, cc * CPL + i, wg[r][i], sg[r]);
                    U.load(row, cc * CPL + i, wu[r][i], su[r]);
                }
            }
        }
        float lg = 1.f, lu = 1.f;
        if constexpr (!WTraits<F>::fp4) lg = G.block_scale(row0, cc * CPL), lu = U.block_scale(row0, cc * CPL);
        if (official) act_quant_packed<M, CH>(xw);
        if constexpr (DW) {
#pragma unroll
            for (int r = 0; r < R; r++) sg[r] = dw_scale_byte(sdw, r, lane), su[r] = dw_scale_byte(sdw, R + r, lane);
        }

#pragma unroll
        for (int r = 0; r < R; r++) {
            float sgv[M], suv[M];
            chunk_dot_lane<F, M, CPL>(sgv, wg[r], xw, conv_scale<F>(sg[r], lg));
            chunk_dot_lane<F, M, CPL>(suv, wu[r], xw, conv_scale<F>(su[r], lu));
            const float a = post_scale<F>(lg), b = post_scale<F>(lu);
#pragma unroll
            for (int t = 0; t < M; t++) {
                tot[(t * R + r) * 2] = active ? sgv[t] * a : 0.f;
                tot[(t * R + r) * 2 + 1] = active ? suv[t] * b : 0.f;
            }
        }
    }
    // thread q = (t * R + r) * 2 + {0 gate, 1 up}; the even thread finishes the pair
    float v = 0.f;
    const bool mine = wave_total<2 * M * R>(tot, red, &v);
    const float u = __shfl_down(v, 1, kWave);
    if (!mine || (threadIdx.x & 1)) return;
    const int q = threadIdx.x >> 1, t = q / R, r = q % R;
    if (t >= m || row0 + r >= inter) return;
    float gv = bf16_round(v), uv = bf16_round(u);
    if (limit > 0) {
        uv = fminf(fmaxf(uv, -limit), limit);
        gv = fminf(gv, limit);
    }
    h[(size_t)pair_out * inter + row0 + r] = f32_to_bf16_bits(__fdiv_rn(gv, 1.f + expf(-gv)) * uv * w_out);
}

template <WFmt F, int M, int R, bool DW>
__global__ __launch_bounds__(512) void k_moe_gateup(MoeJobs jobs, ExpertLayout L, const uint16_t *__restrict__ x,
                                                    uint16_t *__restrict__ h, int dim, int inter, float limit,
                                                    int official) {
    gateup_job<F, M, R, DW>(jobs.j[blockIdx.y], L, x, h, dim, inter, limit, official);
}

// Jobs of two formats in one launch (the reference's FP4 routed experts next to its FP8 E8M0 shared
// expert, stbl/model.cu:536-547): each workgroup takes its job's format (wave-uniform), so the
// shared expert costs no launches of its own. FP8 rows next to FP4 ones take two 16-byte chunks per
// lane (mix_cpl), so both formats' rows span the same lanes and no wave of a workgroup idles.
template <WFmt FA, WFmt FB>
constexpr int mix_cpl() {
    return WTraits<FB>::fp4 ? 1 : WTraits<FA>::CH / WTraits<FB>::CH;
}

template <WFmt FA, WFmt FB, int M, int R, bool DWA, bool DWB>
__global__ __launch_bounds__(512) void k_moe_gateup_mix(MoeJobs jobs, ExpertLayout LA, ExpertLayout LB,
                                                        const uint16_t *__restrict__ x, uint16_t *__restrict__ h,
                                                        int dim, int inter, float limit, int official, int fmt_a) {
    const MoeJob &J = jobs.j[blockIdx.y];
    if (J.fmt == fmt_a) gateup_job<FA, M, R, DWA>(J, LA, x, h, dim, inter, limit, official);
    else gateup_job<FB, M, R, DWB, mix_cpl<FA, FB>()>(J, LB, x, h, dim, inter, limit, official);
}

// ---- down ------------------------------------------------------------------------------------------

// Job blockIdx.y, rows [row0, row0 + R) of down. h bf16 [P][inter] -> o [P][dim] (bf16, or fp32
// holding the unrounded sum when out_f32). DW as in k_moe_gateup.
template <WFmt F, int M, int R, bool DW, int CPL = 1>
__device__ __forceinline__ void down_job(const MoeJob &J, const ExpertLayout &L, const uint16_t *__restrict__ h,
                                         void *__restrict__ o, int dim, int inter, int official, int out_f32,
                                         int tile0 = -1) {
    static_assert(CPL == 1 || !WTraits<F>::fp4, "two chunks per lane: FP8 rows");
    constexpr int CH = WTraits<F>::CH * CPL;  // elements per lane
    const SlotMat<F> D(J.slot, L, 2, dim, inter);
    const int lane = threadIdx.x & 63, c = (threadIdx.x >> 6) * 64 + lane, nch = inter / CH;
    const bool active = c < nch;
    const int cc = active ? c : 0;
    const int row0 = tile0 < 0 ? (int)blockIdx.x * R : tile0;  // the tile's first row
    const int m = J.m;
    const int pair_out = J.pair[min((int)threadIdx.x / R, M - 1)];  // read early, as in gateup_job
    __shared__ float red[kMaxWaves][M * R];
    float tot[M * R];
#pragma unroll
    for (int i = 0; i < M * R; i++) tot[i] = 0.f;
    if (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * 64 < nch) {
        uint32_t xw[M][CH / 2];
#pragma unroll
        for (int t = 0; t < M; t++) {
            uint32_t tmp[1][CH / 2];
            load_x_packed<1, CH>(tmp, h + (size_t)J.pair[t < m ? t : 0] * inter, inter, cc * CH);
#pragma unroll
            for (int i = 0; i < CH / 2; i++) xw[t][i] = tmp[0][i];
        }
        u32x4 wd[R][CPL];
        uint32_t sd[R];
        uint32_t sdw[(R + 3) / 4];
        if constexpr (DW) {
            const int wave = threadIdx.x >> 6, dwi = min(wave * 16 + (lane & 15), (nch >> 2) - 1);
#pragma unroll
            for (int q = 0; q < (R + 3) / 4; q++)
                sdw[q] = D.load_scale_dword((size_t)min(row0 + min(4 * q + (lane >> 4), R - 1), dim - 1), dwi);
#pragma unroll
            for (int r = 0; r < R; r++) wd[r][0] = D.load_codes((size_t)min(row0 + r, dim - 1), cc);
        } else {
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int i = 0; i < CPL; i++) D.load((size_t)min(row0 + r, dim - 1), cc * CPL + i, wd[r][i], sd[r]);
        }
        float ld = 1.f;
        if constexpr (!WTraits<F>::fp4) ld = D.block_scale(row0, cc * CPL);
        if (official) act_quant_packed<M, CH>(xw);
        if constexpr (DW) {
#pragma unroll
            for (int r = 0; r < R; r++) sd[r] = dw_scale_byte(sdw, r, lane);
        }

#pragma unroll
        for (int r = 0; r < R; r++) {
            float s[M];
            chunk_dot_lane<F, M, CPL>(s, wd[r], xw, conv_scale<F>(sd[r], ld));
            const float a = post_scale<F>(ld);
#pragma unroll
            for (int t = 0; t < M; t++) tot[t * R + r] = active ? s[t] * a : 0.f;
        }
    }
    float v = 0.f;
    if (!wave_total<M * R>(tot, red, &v)) return;
    const int t = threadIdx.x / R, r = threadIdx.x % R;
    if (t >= m || row0 + r >= dim) return;
    const size_t at = (size_t)pair_out * dim + row0 + r;
    if (out_f32) ((float *)o)[at] = v;
    else ((uint16_t *)o)[at] = f32_to_bf16_bits(v);
}

template <WFmt F, int M, int R, bool DW>
__global__ __launch_bounds__(512) void k_moe_down(MoeJobs jobs, ExpertLayout L, const uint16_t *__restrict__ h,
                                                  void *__restrict__ o, int dim, int inter, int official, int out_f32) {
    down_job<F, M, R, DW>(jobs.j[blockIdx.y], L, h, o, dim, inter, official, out_f32);
}

// Down rows of jobs of two formats in one launch, as k_moe_gateup_mix.
template <WFmt FA, WFmt FB, int M, int R, bool DWA, bool DWB>
__global__ __launch_bounds__(512) void k_moe_down_mix(MoeJobs jobs, ExpertLayout LA, ExpertLayout LB,
                                                      const uint16_t *__restrict__ h, void *__restrict__ o, int dim,
                                                      int inter, int official, int out_f32, int fmt_a) {
    const MoeJob &J = jobs.j[blockIdx.y];
    if (J.fmt == fmt_a) down_job<FA, M, R, DWA>(J, LA, h, o, dim, inter, official, out_f32);
    else down_job<FB, M, R, DWB, mix_cpl<FA, FB>()>(J, LB, h, o, dim, inter, official, out_f32);
}

// ---- jobs of every token class in one launch --------------------------------------------------------

// Jobs of 1, 2 and 3-4 tokens of one format in one gate/up and one down launch: each workgroup
// takes its job's token class (workgroup-uniform). The few multi-token jobs of a step (the shared
// expert, which every token takes; experts two tokens picked) then compute while the one-token jobs
// stream, instead of running in launches of their own at a fraction of the bandwidth. The kernel
// needs more registers than the one-token body alone, so a launch of one-token jobs only keeps
// k_moe_gateup / k_moe_down.
template <WFmt F, int R, bool DW>
__global__ __launch_bounds__(512) void k_moe_gateup_any(MoeJobs jobs, ExpertLayout L, const uint16_t *__restrict__ x,
                                                        uint16_t *__restrict__ h, int dim, int inter, float limit,
                                                        int official) {
    const MoeJob &J = jobs.j[blockIdx.y];
    if (J.m == 1) {
        gateup_job<F, 1, R, DW>(J, L, x, h, dim, inter, limit, official);
    } else if (J.m == 2) {
        gateup_job<F, 2, R, DW>(J, L, x, h, dim, inter, limit, official);
    } else {
        // the 4-token body in passes of one row (down: two rows), so that the kernel needs no more
        // registers than for the 2-token body
#pragma unroll 1
        for (int p = 0; p < R; p++) {
            if (p > 0) __syncthreads();  // the pass before has read its sums out of LDS
            gateup_job<F, 4, 1, DW>(J, L, x, h, dim, inter, limit, official, (int)blockIdx.x * R + p);
        }
    }
}

template <WFmt F, int R, bool DW>
__global__ __launch_bounds__(512) void k_moe_down_any(MoeJobs jobs, ExpertLayout L, const uint16_t *__restrict__ h,
                                                      void *__restrict__ o, int dim, int inter, int official,
                                                      int out_f32) {
    const MoeJob &J = jobs.j[blockIdx.y];
    if (J.m == 1) {
        down_job<F, 1, R, DW>(J, L, h, o, dim, inter, official, out_f32);
    } else if (J.m == 2) {
        down_job<F, 2, R, DW>(J, L, h, o, dim, inter, official, out_f32);
    } else {
#pragma unroll 1
        for (int p = 0; p < R / 2; p++) {
            if (p > 0) __syncthreads();
            down_job<F, 4, 2, DW>(J, L, h, o, dim, inter, official, out_f32, (int)blockIdx.x * R + 2 * p);
        }
    }
}

// ---- combine ------------------------------------------------------------------------------------

struct PickTable {
    int pair[kMoeMaxT][kMoeMaxPick];  // per token: output rows in top-k order, then the shared one
};

// y[t][r] = bf16(sum over token t's picks in order of o[pair][r]) with the fp32 sum starting at 0
// (stbl/model.cu:579-592: memset, axpy per expert in top-k order, axpy shared, round_bf16).
// Every pick's load is issued before the sum (a fixed trip count; unused picks read pick 0's row),
// so the thread waits for one memory latency, not one per pick.
__global__ void k_moe_combine(PickTable picks, int npick, const uint16_t *__restrict__ o, void *__restrict__ y,
                              int dim, int y_f32) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
    if (r >= dim) return;
    uint32_t v[kMoeMaxPick];
#pragma unroll
    for (int p = 0; p < kMoeMaxPick; p++) v[p] = o[(size_t)picks.pair[t][p < npick ? p : 0] * dim + r];
    float acc = 0.f;
#pragma unroll
    for (int p = 0; p < kMoeMaxPick; p++)
        if (p < npick) acc = fmaf(1.f, bf16_bits_to_f32(v[p]), acc);
    if (y_f32) ((float *)y)[(size_t)t * dim + r] = bf16_round(acc);
    else ((uint16_t *)y)[(size_t)t * dim + r] = f32_to_bf16_bits(acc);
}

// ---- router -------------------------------------------------------------------------------------

// The reference engine's router score sqrt(softplus(l)), softplus with torch's threshold of 20
// (stbl/kernels.cu:436-442); k_route and stbl_sqrt_softplus share it, so their scores are identical.
__device__ __forceinline__ float sqrt_softplus(float l) { return sqrtf(l > 20.f ? l : log1pf(expf(l))); }

__global__ __launch_bounds__(256) void k_sqrt_softplus(float *__restrict__ s, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) s[i] = sqrt_softplus(s[i]);
}

// One workgroup of 256 threads per token. score = 1 / (1 + exp(-logit)) (score_fn 0, the
// configuration's router) or sqrt(softplus(logit)) with softplus(l) = l above 20, else
// log1p(exp(l)) (score_fn 1, stbl/kernels.cu:436-442); the top-k of score + bias (ties to the lower
// expert id) by k rounds of a workgroup argmax; weight_i = score_i / (sum of the top-k scores in
// top-k order + 1e-20) * route_scale. A NaN key ranks below every number (so a token with fewer than
// k numeric keys takes the lowest unused ids next), and its weight comes out NaN.
__global__ __launch_bounds__(256) void k_route(const float *__restrict__ logits, const float *__restrict__ bias,
                                               int n_exp, int topk, float route_scale, int score_fn,
                                               int *__restrict__ ids, float *__restrict__ weights,
                                               float *__restrict__ scores) {
    __shared__ float sc[1024];
    __shared__ float bv[4];
    __shared__ int bi[4];
    __shared__ int chosen[32];
    const int t = blockIdx.x, tid = threadIdx.x;
    for (int e = tid; e < n_exp; e += 256) {
        const float l = logits[(size_t)t * n_exp + e];
        const float s = score_fn == 1 ? sqrt_softplus(l) : __fdiv_rn(1.f, 1.f + expf(-l));
        sc[e] = s;
        if (scores) scores[(size_t)t * n_exp + e] = s;
    }
    __syncthreads();
    for (int p = 0; p < topk; p++) {
        float best = -INFINITY;
        int besti = 0x7fffffff;
        for (int e = tid; e < n_exp; e += 256) {
            bool used = false;
            for (int q = 0; q < p; q++) used |= chosen[q] == e;
            if (used) continue;
            float v = sc[e] + (bias ? bias[e] : 0.f);
            v = v != v ? -INFINITY : v;  // a NaN key ranks last; among equal keys the lower id wins
            if (v > best || (v == best && e < besti)) best = v, besti = e;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(best, off, kWave);
            const int oi = __shfl_xor(besti, off, kWave);
            if (ov > best || (ov == best && oi < besti)) best = ov, besti = oi;
        }
        if ((tid & 63) == 0) bv[tid >> 6] = best, bi[tid >> 6] = besti;
        __syncthreads();
        if (tid == 0) {
            float b = bv[0];
            int i = bi[0];
            for (int w = 1; w < 4; w++)
                if (bv[w] > b || (bv[w] == b && bi[w] < i)) b = bv[w], i = bi[w];
            chosen[p] = i;
        }
        __syncthreads();
    }
    if (tid == 0) {
        float sum = 0.f;
        for (int p = 0; p < topk; p++) sum += sc[chosen[p]];
        for (int p = 0; p < topk; p++) {
            float wt = sc[chosen[p]];
            wt = __fdiv_rn(wt, sum + 1e-20f);
            wt *= route_scale;
            ids[(size_t)t * topk + p] = chosen[p];
            weights[(size_t)t * topk + p] = wt;
        }
    }
}

// ---- host side -------------------------------------------------------------------------------------

static inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Rows per workgroup. Several experts per launch: 4 gate and 4 up rows share a lane's x chunk, and
// 8 down rows (4 with 4 tokens), measured best for the MoE steps (2 rows for more than one token
// was 6-11% slower at T=4). One expert per launch (the FFN on its own): 2 down rows, which keep 4x
// more workgroups in flight (4 / 8 rows: 9.48 -> 9.48 / 9.58 us for one FP4 expert); gate/up takes
// 4 and 4 rows for FP4, whose dword scale loads need 4+ rows (9.48 -> 9.25 us; 8 and 8: 10.2 us),
// and 2 and 2 for FP8 (11.80 against 11.85 us with 4).
template <WFmt F, int M, int R>
static hipError_t launch_gateup_r(const MoeJobs &jobs, int n, const ExpertLayout &L, const uint16_t *x, uint16_t *h,
                                  int dim, int inter, float limit, int official, hipStream_t st) {
    const int waves = ceil_div(dim / WTraits<F>::CH, 64);
    // FP4 tiles of 4+ rows whose scale rows (dim / 32 bytes) are a multiple of 4 bytes fetch their
    // scales as dwords (slot parts are 256-byte aligned): the MoE steps' 4-row gate/up tiles issue 2
    // dword loads instead of 8 byte loads per lane (measured T=1 41.6 -> 40.1 us, T=4 134.9 -> 126.0
    // us); one expert's 2-row tiles keep byte loads (dwords there: 9.24 -> 9.33 us)
    if (WTraits<F>::fp4 && R >= 4 && (dim / 32) % 4 == 0)
        hipLaunchKernelGGL((k_moe_gateup<F, M, R, WTraits<F>::fp4 && R >= 4>), dim3(ceil_div(inter, R), n), dim3(64 * waves), 0,
                           st, jobs, L, x, h, dim, inter, limit, official);
    else
        hipLaunchKernelGGL((k_moe_gateup<F, M, R, false>), dim3(ceil_div(inter, R), n), dim3(64 * waves), 0, st, jobs,
                           L, x, h, dim, inter, limit, official);
    return hipGetLastError();
}

template <WFmt F, int M>
static hipError_t launch_gateup(const MoeJobs &jobs, int n, const ExpertLayout &L, const uint16_t *x, uint16_t *h,
                                int dim, int inter, float limit, int official, hipStream_t st) {
    if (n == 1) return launch_gateup_r<F, M, WTraits<F>::fp4 ? 4 : 2>(jobs, n, L, x, h, dim, inter, limit, official, st);
    return launch_gateup_r<F, M, 4>(jobs, n, L, x, h, dim, inter, limit, official, st);
}

template <WFmt F, int M, int R>
static hipError_t launch_down_r(const MoeJobs &jobs, int n, const ExpertLayout &L, const uint16_t *h, void *o, int dim,
                                int inter, int official, int out_f32, hipStream_t st) {
    const int waves = ceil_div(inter / WTraits<F>::CH, 64);
    if (WTraits<F>::fp4 && R >= 4 && (inter / 32) % 4 == 0)
        hipLaunchKernelGGL((k_moe_down<F, M, R, WTraits<F>::fp4 && R >= 4>), dim3(ceil_div(dim, R), n), dim3(64 * waves), 0, st,
                           jobs, L, h, o, dim, inter, official, out_f32);
    else
        hipLaunchKernelGGL((k_moe_down<F, M, R, false>), dim3(ceil_div(dim, R), n), dim3(64 * waves), 0, st, jobs, L,
                           h, o, dim, inter, official, out_f32);
    return hipGetLastError();
}

template <WFmt F, int M>
static hipError_t launch_down(const MoeJobs &jobs, int n, const ExpertLayout &L, const uint16_t *h, void *o, int dim,
                              int inter, int official, int out_f32, hipStream_t st) {
    if (n == 1) return launch_down_r<F, M, 2>(jobs, n, L, h, o, dim, inter, official, out_f32, st);
    return launch_down_r<F, M, M == 4 ? 4 : 8>(jobs, n, L, h, o, dim, inter, official, out_f32, st);
}

// Token class of a job: 1 (one token), 2 (two) or 3 (three or four: the M = 4 templates).
static int token_class(const MoeJob &J) { return J.m == 1 ? 1 : (J.m == 2 ? 2 : 3); }

static bool several_classes(const MoeJob *all, int njobs) {
    for (int j = 1; j < njobs; j++)
        if (token_class(all[j]) != token_class(all[0])) return true;
    return false;
}

// One gate/up (4 gate and 4 up rows per workgroup) or down (8 rows) launch over jobs of every token
// class (k_moe_gateup_any, k_moe_down_any).
template <WFmt F>
static hipError_t launch_any(bool gateup, const MoeJobs &jobs, int n, const ExpertLayout &L, const uint16_t *x,
                             uint16_t *h, void *o, int dim, int inter, float limit, int official, int out_f32,
                             hipStream_t st) {
    const int k = gateup ? dim : inter;
    const dim3 block(64 * ceil_div(k / WTraits<F>::CH, 64));
    // FP4 tiles whose scale rows are a multiple of 4 bytes fetch their scales as dwords
    const bool dw = WTraits<F>::fp4 && (k / 32) % 4 == 0;
    if (gateup) {
        const dim3 grid(ceil_div(inter, 4), n);
        if (dw)
            hipLaunchKernelGGL((k_moe_gateup_any<F, 4, WTraits<F>::fp4>), grid, block, 0, st, jobs, L, x, h, dim, inter,
                               limit, official);
        else
            hipLaunchKernelGGL((k_moe_gateup_any<F, 4, false>), grid, block, 0, st, jobs, L, x, h, dim, inter, limit,
                               official);
    } else {
        const dim3 grid(ceil_div(dim, 8), n);
        if (dw)
            hipLaunchKernelGGL((k_moe_down_any<F, 8, WTraits<F>::fp4>), grid, block, 0, st, jobs, L, h, o, dim, inter,
                               official, out_f32);
        else
            hipLaunchKernelGGL((k_moe_down_any<F, 8, false>), grid, block, 0, st, jobs, L, h, o, dim, inter, official,
                               out_f32);
    }
    return hipGetLastError();
}

// Runs jobs of one format and several token classes through one gate/up and one down launch (per
// kMoeMaxJobs jobs), in order of falling token class: the workgroups with the most arithmetic per
// byte are dispatched first, so it overlaps the one-token jobs' streaming.
template <WFmt F>
static hipError_t run_jobs_any(const MoeJob *all, int njobs, const ExpertLayout &L, const uint16_t *x, uint16_t *h,
                               void *o, int dim, int inter, float limit, int official, int out_f32, hipStream_t st) {
    for (int phase = 0; phase < 2; phase++) {
        MoeJobs batch;
        int n = 0;
        auto flush = [&]() -> hipError_t {
            if (n == 0) return hipSuccess;
            const hipError_t e = launch_any<F>(phase == 0, batch, n, L, x, h, o, dim, inter, limit, official, out_f32, st);
            n = 0;
            return e;
        };
        for (int cls = 3; cls >= 1; cls--)
            for (int j = 0; j < njobs; j++) {
                if (token_class(all[j]) != cls) continue;
                batch.j[n++] = all[j];
                if (n == kMoeMaxJobs) {
                    const hipError_t e = flush();
                    if (e != hipSuccess) return e;
                }
            }
        const hipError_t e = flush();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Runs the jobs through gate/up and down in launches of one token class each.
template <WFmt F>
static hipError_t run_jobs_by_class(const MoeJob *all, int njobs, const ExpertLayout &L, const uint16_t *x,
                                    uint16_t *h, void *o, int dim, int inter, float limit, int official, int out_f32,
                                    hipStream_t st) {
    for (int phase = 0; phase < 2; phase++) {
        for (int mclass = 1; mclass <= 3; mclass++) {  // M = 1, 2, 4 templates
            MoeJobs batch;
            int n = 0;
            auto flush = [&]() -> hipError_t {
                if (n == 0) return hipSuccess;
                hipError_t e;
                if (phase == 0) {
                    e = mclass == 1 ? launch_gateup<F, 1>(batch, n, L, x, h, dim, inter, limit, official, st)
                        : mclass == 2 ? launch_gateup<F, 2>(batch, n, L, x, h, dim, inter, limit, official, st)
                                      : launch_gateup<F, 4>(batch, n, L, x, h, dim, inter, limit, official, st);
                } else {
                    e = mclass == 1 ? launch_down<F, 1>(batch, n, L, h, o, dim, inter, official, out_f32, st)
                        : mclass == 2 ? launch_down<F, 2>(batch, n, L, h, o, dim, inter, official, out_f32, st)
                                      : launch_down<F, 4>(batch, n, L, h, o, dim, inter, official, out_f32, st);
                }
                n = 0;
                return e;
            };
            for (int j = 0; j < njobs; j++) {
                const int cls = all[j].m == 1 ? 1 : (all[j].m == 2 ? 2 : 3);
                if (cls != mclass) continue;
                batch.j[n++] = all[j];
                if (n == kMoeMaxJobs) {
                    const hipError_t e = flush();
                    if (e != hipSuccess) return e;
                }
            }
            const hipError_t e = flush();
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

// Gate/up and down launches over jobs of two formats, FA (format fmt_a) and FB (each job's fmt
// says which), with the same row tiles as the single-format launches (4 gate and 4 up rows, 8 down
// rows, 4 with 4 tokens). A workgroup has as many waves as the format with the longer rows needs.
template <WFmt FA, WFmt FB, int M>
static hipError_t launch_mix(bool gateup, const MoeJobs &jobs, int n, int fmt_a, int fmt_b, const uint16_t *x,
                             uint16_t *h, void *o, int dim, int inter, float limit, int official, int out_f32,
                             hipStream_t st) {
    const ExpertLayout LA = expert_layout(fmt_a, dim, inter), LB = expert_layout(fmt_b, dim, inter);
    const int k = gateup ? dim : inter;
    const int waves = std::max(ceil_div(k / WTraits<FA>::CH, 64), ceil_div(k / (WTraits<FB>::CH * mix_cpl<FA, FB>()), 64));
    // FP4 tiles of 4+ rows whose scale rows are a multiple of 4 bytes fetch their scales as dwords
    const bool dwa = WTraits<FA>::fp4 && (k / 32) % 4 == 0, dwb = WTraits<FB>::fp4 && (k / 32) % 4 == 0;
    if (gateup) {
        constexpr int R = 4;
        const dim3 grid(ceil_div(inter, R), n), block(64 * waves);
#define STBL_GU(DA, DB)                                                                                          \
    hipLaunchKernelGGL((k_moe_gateup_mix<FA, FB, M, R, DA, DB>), grid, block, 0, st, jobs, LA, LB, x, h, dim, inter, \
                       limit, official, fmt_a)
        if (dwa && dwb) STBL_GU(WTraits<FA>::fp4, WTraits<FB>::fp4);
        else if (dwa) STBL_GU(WTraits<FA>::fp4, false);
        else if (dwb) STBL_GU(false, WTraits<FB>::fp4);
        else STBL_GU(false, false);
#undef STBL_GU
    } else {
        constexpr int R = M == 4 ? 4 : 8;
        const dim3 grid(ceil_div(dim, R), n), block(64 * waves);
#define STBL_DN(DA, DB)                                                                                             \
    hipLaunchKernelGGL((k_moe_down_mix<FA, FB, M, R, DA, DB>), grid, block, 0, st, jobs, LA, LB, h, o, dim, inter, \
                       official, out_f32, fmt_a)
        if (dwa && dwb) STBL_DN(WTraits<FA>::fp4, WTraits<FB>::fp4);
        else if (dwa) STBL_DN(WTraits<FA>::fp4, false);
        else if (dwb) STBL_DN(false, WTraits<FB>::fp4);
        else STBL_DN(false, false);
#undef STBL_DN
    }
    return hipGetLastError();
}

// Runs jobs of formats fmt_a (FA) and fmt_b (FB) through gate/up and down in launches of one token
// class each, a launch holding both formats where its class has both (the FB jobs first: their
// workgroups carry more bytes, so they are dispatched before the others), else the single-format
// launches.
template <WFmt FA, WFmt FB>
static hipError_t run_jobs_mix_by_class(const MoeJob *all, int njobs, int fmt_a, int fmt_b, const uint16_t *x,
                                        uint16_t *h, void *o, int dim, int inter, float limit, int official,
                                        int out_f32, hipStream_t st) {
    const ExpertLayout LA = expert_layout(fmt_a, dim, inter), LB = expert_layout(fmt_b, dim, inter);
    for (int phase = 0; phase < 2; phase++) {
        for (int mclass = 1; mclass <= 3; mclass++) {
            MoeJobs batch;
            int n = 0, na = 0, nb = 0;
            auto flush = [&]() -> hipError_t {
                if (n == 0) return hipSuccess;
                hipError_t e;
                const bool gu = phase == 0;
                if (na > 0 && nb > 0) {
                    e = mclass == 1 ? launch_mix<FA, FB, 1>(gu, batch, n, fmt_a, fmt_b, x, h, o, dim, inter, limit, official, out_f32, st)
                        : mclass == 2 ? launch_mix<FA, FB, 2>(gu, batch, n, fmt_a, fmt_b, x, h, o, dim, inter, limit, official, out_f32, st)
                                      : launch_mix<FA, FB, 4>(gu, batch, n, fmt_a, fmt_b, x, h, o, dim, inter, limit, official, out_f32, st);
                } else if (na > 0) {
                    e = gu ? (mclass == 1 ? launch_gateup<FA, 1>(batch, n, LA, x, h, dim, inter, limit, official, st)
                              : mclass == 2 ? launch_gateup<FA, 2>(batch, n, LA, x, h, dim, inter, limit, official, st)
                                            : launch_gateup<FA, 4>(batch, n, LA, x, h, dim, inter, limit, official, st))
                           : (mclass == 1 ? launch_down<FA, 1>(batch, n, LA, h, o, dim, inter, official, out_f32, st)
                              : mclass == 2 ? launch_down<FA, 2>(batch, n, LA, h, o, dim, inter, official, out_f32, st)
                                            : launch_down<FA, 4>(batch, n, LA, h, o, dim, inter, official, out_f32, st));
                } else {
                    e = gu ? (mclass == 1 ? launch_gateup<FB, 1>(batch, n, LB, x, h, dim, inter, limit, official, st)
                              : mclass == 2 ? launch_gateup<FB, 2>(batch, n, LB, x, h, dim, inter, limit, official, st)
                                            : launch_gateup<FB, 4>(batch, n, LB, x, h, dim, inter, limit, official, st))
                           : (mclass == 1 ? launch_down<FB, 1>(batch, n, LB, h, o, dim, inter, official, out_f32, st)
                              : mclass == 2 ? launch_down<FB, 2>(batch, n, LB, h, o, dim, inter, official, out_f32, st)
                                            : launch_down<FB, 4>(batch, n, LB, h, o, dim, inter, official, out_f32, st));
                }
                n = na = nb = 0;
                return e;
            };
            for (int pass = 0; pass < 2; pass++) {  // the FB jobs, then the FA jobs
                for (int j = 0; j < njobs; j++) {
                    const int cls = all[j].m == 1 ? 1 : (all[j].m == 2 ? 2 : 3);
                    if (cls != mclass || (all[j].fmt == fmt_a) != (pass == 1)) continue;
                    batch.j[n++] = all[j];
                    (pass == 1 ? na : nb)++;
                    if (n == kMoeMaxJobs) {
                        const hipError_t e = flush();
                        if (e != hipSuccess) return e;
                    }
                }
            }
            const hipError_t e = flush();
            if (e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

// The launch plan of a set of jobs: when the jobs of format fmt_a (every job, with one format) span
// several token classes, they go through run_jobs_any and the others (format fmt_b) through the
// launches per class; otherwise every job goes through the launches per class. The formats stay
// apart: in one launch with both, each workgroup holds the registers of the widest of six bodies
// (measured with FP8 E8M0 jobs of two chunks per lane: C4 T=4 122 -> 137 us, V4.1 T=4 108 -> 115 us).
template <WFmt FA, WFmt FB>
static hipError_t run_jobs_split(const MoeJob *all, int njobs, int fmt_a, int fmt_b, const uint16_t *x, uint16_t *h,
                                 void *o, int dim, int inter, float limit, int official, int out_f32, hipStream_t st) {
    const ExpertLayout LA = expert_layout(fmt_a, dim, inter);
    static thread_local MoeJob lo[kMoeMaxT * kMoeMaxPick], hi[kMoeMaxT * kMoeMaxPick];
    int nlo = 0, nhi = 0;
    for (int j = 0; j < njobs; j++) {
        if (FA == FB || all[j].fmt == fmt_a) lo[nlo++] = all[j];
        else hi[nhi++] = all[j];
    }
    if (!several_classes(lo, nlo)) {
        if constexpr (FA == FB) return run_jobs_by_class<FA>(all, njobs, LA, x, h, o, dim, inter, limit, official, out_f32, st);
        else return run_jobs_mix_by_class<FA, FB>(all, njobs, fmt_a, fmt_b, x, h, o, dim, inter, limit, official, out_f32, st);
    }
    hipError_t e = run_jobs_any<FA>(lo, nlo, LA, x, h, o, dim, inter, limit, official, out_f32, st);
    if constexpr (FA != FB) {
        if (e == hipSuccess && nhi > 0)
            e = run_jobs_by_class<FB>(hi, nhi, expert_layout(fmt_b, dim, inter), x, h, o, dim, inter, limit, official,
                                      out_f32, st);
    }
    return e;
}

// Runs jobs whose slots hold format fmt.
static hipError_t run_fmt(int fmt, const MoeJob *all, int njobs, int dim, int inter, const uint16_t *x, uint16_t *h,
                          void *o, float limit, int official, int out_f32, hipStream_t st) {
    if (fmt == EXPERT_FP4)
        return run_jobs_split<WFmt::FP4_OCP, WFmt::FP4_OCP>(all, njobs, fmt, fmt, x, h, o, dim, inter, limit, official,
                                                            out_f32, st);
    if (fmt == EXPERT_FP8)
        return run_jobs_split<WFmt::FP8_B128, WFmt::FP8_B128>(all, njobs, fmt, fmt, x, h, o, dim, inter, limit, official,
                                                              out_f32, st);
    return run_jobs_split<WFmt::FP8_E8M0, WFmt::FP8_E8M0>(all, njobs, fmt, fmt, x, h, o, dim, inter, limit, official,
                                                          out_f32, st);
}

static bool fmt_ok(int fmt) { return fmt == EXPERT_FP4 || fmt == EXPERT_FP8 || fmt == EXPERT_FP8_E8M0; }

static bool dims_ok(int fmt, int dim, int inter) {
    const int CH = fmt == EXPERT_FP4 ? 32 : 16;
    // FP8: the rows of a tile must share a scale block (128 rows for fp32 scales, 32 for E8M0)
    const int align = fmt == EXPERT_FP8 ? 128 : 32;
    return dim > 0 && inter > 0 && dim % align == 0 && inter % align == 0 && dim / CH <= kMaxWaves * 64 &&
           inter / CH <= kMaxWaves * 64;
}

}  // namespace stbl

using namespace stbl;

extern "C" {

uint64_t stbl_amd_expert_layout(int fmt, int dim, int inter, uint64_t *offsets) {
    const ExpertLayout L = expert_layout(fmt, dim, inter);
    if (offsets)
        for (int i = 0; i < 6; i++) offsets[i] = L.off[i];
    return L.bytes;
}

int stbl_amd_expert_ffn(int fmt, void *y, const void *slot, const void *x, int m, int dim, int inter, float weight,
                        float limit, int official, int y_f32, void *work, hipStream_t st) {
    if (!fmt_ok(fmt)) return abi_fail(hipErrorInvalidValue, "expert_ffn: unknown format %d", fmt);
    if (!y || !slot || !x || !work) return abi_fail(hipErrorInvalidValue, "expert_ffn: null pointer");
    if (!dims_ok(fmt, dim, inter)) return abi_fail(hipErrorInvalidValue, "expert_ffn: unsupported dims %d x %d", dim, inter);
    if (m < 1 || m > kMoeMaxTok) return abi_fail(hipErrorInvalidValue, "expert_ffn: m must be 1..4 (m=%d)", m);
    if (!aligned16(slot) || ((uintptr_t)slot & 255) || !aligned16(x) || !aligned16(work))
        return abi_fail(hipErrorInvalidValue, "expert_ffn: slot must be 256-byte and x/work 16-byte aligned");
    MoeJob J = {};
    J.slot = (const uint8_t *)slot;
    J.m = m;
    for (int t = 0; t < m; t++) J.tok[t] = t, J.pair[t] = t, J.w[t] = weight;
    const hipError_t e = run_fmt(fmt, &J, 1, dim, inter, (const uint16_t *)x, (uint16_t *)work, y, limit, official,
                                 y_f32, st);
    return abi_status(e, "expert_ffn launch");
}

// Routed MoE over cached expert slots, in up to two phases. slots: HOST array of n_slots device
// pointers (one per distinct expert used by this call). pick: HOST [t][topk] indices into slots,
// weights: HOST [t][topk] route weights, shared: index into slots of the always-on expert (weight
// 1) or -1, whose slot holds format shared_fmt (-1: the routed experts' format; the reference's
// shared expert is FP8 with E8M0 32x32 scales, stbl/model.cu:544-547, next to FP4 routed experts).
// work: device scratch of at least stbl_amd_moe_work_bytes(t, topk, dim, inter) bytes.
// phase 0 runs every expert and the combine. With slot_ready (HOST, n_slots flags), phase 1 runs
// the experts whose slots are ready and phase 2 the others and then the combine, so a caller can
// queue phase 1 before an expert cache's refills are waited for and phase 2 after
// (stbl/model.cu:541-549, 588). Both phases must get the same arguments and work; every expert's
// output has its own rows of work, and the combine adds them in top-k order, so the result is the
// same bits as phase 0.
static int moe_experts_impl(int fmt, void *y, const void *x, int t, int dim, int inter, const void *const *slots,
                            int n_slots, const int *pick, const float *weights, int topk, int shared, int shared_fmt,
                            float limit, int official, int y_f32, const int *slot_ready, int phase, void *work,
                            hipStream_t st) {
    if (shared_fmt < 0) shared_fmt = fmt;
    if (!fmt_ok(fmt) || !fmt_ok(shared_fmt))
        return abi_fail(hipErrorInvalidValue, "moe_experts: unknown format %d / %d", fmt, shared_fmt);
    if (!y || !x || !slots || !pick || !weights || !work) return abi_fail(hipErrorInvalidValue, "moe_experts: null pointer");
    if (phase < 0 || phase > 2 || (phase > 0 && !slot_ready))
        return abi_fail(hipErrorInvalidValue, "moe_experts: phase must be 0, or 1 or 2 with slot_ready (phase=%d)", phase);
    if (!dims_ok(fmt, dim, inter) || !dims_ok(shared_fmt, dim, inter))
        return abi_fail(hipErrorInvalidValue, "moe_experts: unsupported dims %d x %d", dim, inter);
    if (t < 1 || t > kMoeMaxT || topk < 1 || topk + 1 > kMoeMaxPick || n_slots < 1 || shared >= n_slots)
        return abi_fail(hipErrorInvalidValue, "moe_experts: need 1 <= t <= 16, 1 <= topk <= 16 (t=%d topk=%d)", t, topk);
    if (!aligned16(x) || !aligned16(work)) return abi_fail(hipErrorInvalidValue, "moe_experts: x and work must be 16-byte aligned");
    for (int i = 0; i < n_slots; i++)
        if (!slots[i] || ((uintptr_t)slots[i] & 255)) return abi_fail(hipErrorInvalidValue, "moe_experts: slot %d null or not 256-byte aligned", i);
    const int npick = topk + (shared >= 0 ? 1 : 0);
    for (int tt = 0; tt < t; tt++)
        for (int p = 0; p < topk; p++)
            if (pick[tt * topk + p] < 0 || pick[tt * topk + p] >= n_slots)
                return abi_fail(hipErrorInvalidValue, "moe_experts: pick out of range");
    // jobs: one per (slot, group of <= 4 tokens); pair rows numbered in job order over all slots,
    // so both phases number them alike. A shared expert of another format runs in launches of its
    // own (sjobs). Each array holds every (token, pick) pair, duplicates included.
    static thread_local MoeJob jobs[kMoeMaxT * kMoeMaxPick], sjobs[kMoeMaxT * kMoeMaxPick];
    PickTable table = {};
    int njobs = 0, nsjobs = 0, npairs = 0;
    for (int s = 0; s < n_slots; s++) {
        const bool run = phase == 0 || (phase == 1) == (slot_ready[s] != 0);
        MoeJob *J = nullptr;
        for (int tt = 0; tt < t; tt++)
            for (int p = 0; p < npick; p++) {
                const int sl = p < topk ? pick[tt * topk + p] : shared;
                if (sl != s) continue;
                table.pair[tt][p] = npairs;
                if (run) {
                    if (!J || J->m == kMoeMaxTok) {
                        const bool other = s == shared && shared_fmt != fmt;
                        J = other ? &sjobs[nsjobs++] : &jobs[njobs++];
                        *J = MoeJob{};
                        J->slot = (const uint8_t *)slots[s];
                        J->fmt = other ? shared_fmt : fmt;
                    }
                    J->tok[J->m] = tt;
                    J->pair[J->m] = npairs;
                    J->w[J->m] = p < topk ? weights[tt * topk + p] : 1.f;
                    J->m++;
                }
                npairs++;
            }
    }
    uint16_t *h = (uint16_t *)work;
    uint16_t *o = h + (size_t)t * npick * inter;
    hipError_t e;
    if (nsjobs > 0 && fmt == EXPERT_FP4 && shared_fmt == EXPERT_FP8_E8M0) {
        // the reference's pairing (FP4 routed, FP8 E8M0 shared): both formats in the same launches
        for (int i = 0; i < nsjobs; i++) jobs[njobs + i] = sjobs[i];
        e = run_jobs_split<WFmt::FP4_OCP, WFmt::FP8_E8M0>(jobs, njobs + nsjobs, EXPERT_FP4, EXPERT_FP8_E8M0,
                                                          (const uint16_t *)x, h, o, dim, inter, limit, official, 0, st);
    } else {
        e = run_fmt(fmt, jobs, njobs, dim, inter, (const uint16_t *)x, h, o, limit, official, 0, st);
        if (e == hipSuccess && nsjobs > 0)
            e = run_fmt(shared_fmt, sjobs, nsjobs, dim, inter, (const uint16_t *)x, h, o, limit, official, 0, st);
    }
    if (e == hipSuccess && phase != 1) {
        hipLaunchKernelGGL(k_moe_combine, dim3(ceil_div(dim, 256), t), dim3(256), 0, st, table, npick, o, y, dim, y_f32);
        e = hipGetLastError();
    }
    return abi_status(e, "moe_experts launch");
}

int stbl_amd_moe_experts(int fmt, void *y, const void *x, int t, int dim, int inter, const void *const *slots,
                         int n_slots, const int *pick, const float *weights, int topk, int shared, int shared_fmt,
                         float limit, int official, int y_f32, void *work, hipStream_t st) {
    return moe_experts_impl(fmt, y, x, t, dim, inter, slots, n_slots, pick, weights, topk, shared, shared_fmt, limit,
                            official, y_f32, nullptr, 0, work, st);
}

int stbl_amd_moe_experts_phase(int fmt, void *y, const void *x, int t, int dim, int inter, const void *const *slots,
                               int n_slots, const int *pick, const float *weights, int topk, int shared,
                               int shared_fmt, float limit, int official, int y_f32, const int *slot_ready, int phase,
                               void *work, hipStream_t st) {
    return moe_experts_impl(fmt, y, x, t, dim, inter, slots, n_slots, pick, weights, topk, shared, shared_fmt, limit,
                            official, y_f32, slot_ready, phase, work, st);
}

// ---- the MoE step without a caller workspace --------------------------------------------------------

// Device scratch of stbl_amd_moe_experts_noalloc: the SwiGLU intermediates and expert outputs of one
// call (what `work` holds for stbl_amd_moe_experts), at most kMoeScratchBytes. Each GPU the library
// runs on holds its own copy until the process ends; every call on a GPU uses that GPU's copy.
constexpr uint64_t kMoeScratchBytes = 8ull << 20;
static __device__ __align__(256) uint8_t scratch[kMoeScratchBytes];

// The current device's address of `scratch`, looked up once per device (the array's name in host
// code is not a device address). nullptr on failure, recorded for stbl_amd_last_error.
static void *scratch_address() {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void *addr[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        abi_status(e, "moe_experts_noalloc: hipGetDevice");
        return nullptr;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        abi_fail(hipErrorInvalidDevice, "moe_experts_noalloc: device %d beyond %d", dev, kMaxDevices);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(mu);
    if (!addr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            abi_status(e != hipSuccess ? e : hipErrorInvalidSymbol, "moe_experts_noalloc: hipGetSymbolAddress(scratch)");
            return nullptr;
        }
        addr[dev] = p;
    }
    return addr[dev];
}

// Scratch bytes stbl_amd_moe_experts needs for t tokens.
uint64_t stbl_amd_moe_work_bytes(int t, int topk, int dim, int inter) {
    const uint64_t pairs = (uint64_t)t * (topk + 1);
    return align256(pairs * inter * 2) + align256(pairs * dim * 2);
}

// stbl_amd_moe_experts with the library's static device scratch instead of `work`: no allocation
// of any kind, for callers that cannot allocate. Refuses steps whose scratch would exceed
// kMoeScratchBytes. Every scratch byte a step reads is written earlier in the same step (gate/up
// writes each pair's SwiGLU output before down reads it, down each pair's output before the
// combine), so nothing left by an earlier call is read and nothing is cleared. Calls that overlap on
// one GPU share its scratch and race.
int stbl_amd_moe_experts_noalloc(int fmt, void *y, const void *x, int t, int dim, int inter, const void *const *slots,
                                 int n_slots, const int *pick, const float *weights, int topk, int shared,
                                 int shared_fmt, float limit, int official, int y_f32, hipStream_t st) {
    if (t < 1 || t > kMoeMaxT || topk < 1 || topk + 1 > kMoeMaxPick || dim < 1 || inter < 1)
        return abi_fail(hipErrorInvalidValue, "moe_experts_noalloc: need 1 <= t <= 16, 1 <= topk <= 16, dims > 0");
    const uint64_t need = stbl_amd_moe_work_bytes(t, topk, dim, inter);
    if (need > kMoeScratchBytes)
        return abi_fail(hipErrorInvalidValue, "moe_experts_noalloc: the step needs %llu bytes of scratch, more than the %llu it has",
                        (unsigned long long)need, (unsigned long long)kMoeScratchBytes);
    void *work = scratch_address();
    if (!work) return -(int)hipErrorInvalidSymbol;
    return moe_experts_impl(fmt, y, x, t, dim, inter, slots, n_slots, pick, weights, topk, shared, shared_fmt, limit,
                            official, y_f32, nullptr, 0, work, st);
}

// stbl/kernels.h:34: s[i] = sqrt(softplus(s[i])) in place, the engine's router scores.
void stbl_sqrt_softplus(float *s, int n, hipStream_t st) {
    if (!s || n <= 0) {
        abi_fail(hipErrorInvalidValue, "stbl_sqrt_softplus: bad arguments (n=%d)", n);
        return;
    }
    hipLaunchKernelGGL(k_sqrt_softplus, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, s, n);
    abi_status(hipGetLastError(), "stbl_sqrt_softplus launch");
}

int stbl_amd_route(const float *logits, const float *bias, int t, int n_exp, int topk, float route_scale, int score_fn,
                   int *ids, float *weights, float *scores, hipStream_t st) {
    if (!logits || !ids || !weights || t < 1 || n_exp < 1 || n_exp > 1024 || topk < 1 || topk > 32 || topk > n_exp)
        return abi_fail(hipErrorInvalidValue, "route: need 1 <= topk <= min(32, n_exp), n_exp <= 1024");
    if (score_fn != 0 && score_fn != 1) return abi_fail(hipErrorInvalidValue, "route: score_fn must be 0 (sigmoid) or 1 (sqrt-softplus)");
    hipLaunchKernelGGL(k_route, dim3(t), dim3(256), 0, st, logits, bias, n_exp, topk, route_scale, score_fn, ids,
                       weights, scores);
    return abi_status(hipGetLastError(), "route launch");
}

}  // extern "C"
