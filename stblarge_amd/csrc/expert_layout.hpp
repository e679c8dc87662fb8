// Byte layout of one expert's weights in an HBM cache slot (and in the host pool it is refilled
// from): gate [inter x dim], up [inter x dim], down [dim x inter], each as codes then scales.
//
//   FP4 (OCP e2m1 + E8M0 per 32 along K): codes [rows][k/2], scales [rows][k/32] bytes.
//   FP8 (e4m3 + fp32 per 128x128 block):  codes [rows][k],   scales [ceil(rows/128)][ceil(k/128)] fp32.
//   FP8_E8M0 (e4m3 + E8M0 per 32x32, the reference engine's FP8 layout, stbl/kernels.cu:98-103):
//                                          codes [rows][k],   scales [ceil(rows/32)][k/32] bytes.
//
// Every part starts on a 256-byte boundary, so 128-bit loads of codes are aligned and the fp32
// scales are naturally aligned. The reference keeps gate | up | down contiguous in its slot the same
// way (stbl/model.cu:374-381, :511), with GGUF blocks instead of separate scale arrays.
#pragma once

#include <stdint.h>

namespace stbl {

enum ExpertFmt { EXPERT_FP4 = 0, EXPERT_FP8 = 1, EXPERT_FP8_E8M0 = 2 };

struct ExpertLayout {
    uint64_t off[6];  // gate codes, gate scales, up codes, up scales, down codes, down scales
    uint64_t bytes;   // slot size
};

__host__ __device__ inline uint64_t align256(uint64_t v) { return (v + 255) & ~(uint64_t)255; }

__host__ __device__ inline uint64_t codes_bytes(int fmt, int rows, int k) {
    return fmt == EXPERT_FP4 ? (uint64_t)rows * k / 2 : (uint64_t)rows * k;
}

__host__ __device__ inline uint64_t scales_bytes(int fmt, int rows, int k) {
    if (fmt == EXPERT_FP4) return (uint64_t)rows * (k / 32);
    if (fmt == EXPERT_FP8_E8M0) return (uint64_t)((rows + 31) / 32) * (k / 32);
    return (uint64_t)((rows + 127) / 128) * ((k + 127) / 128) * 4;
}

__host__ __device__ inline ExpertLayout expert_layout(int fmt, int dim, int inter) {
    ExpertLayout L;
    uint64_t at = 0;
    const int rows[3] = {inter, inter, dim}, ks[3] = {dim, dim, inter};
    for (int m = 0; m < 3; m++) {
        L.off[2 * m] = at;
        at = align256(at + codes_bytes(fmt, rows[m], ks[m]));
        L.off[2 * m + 1] = at;
        at = align256(at + scales_bytes(fmt, rows[m], ks[m]));
    }
    L.bytes = at;
    return L;
}

}  // namespace stbl
