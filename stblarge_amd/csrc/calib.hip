// Calibration kernel for the measurements: a bare streaming read of a byte range in one launch, the
// floor any one-launch kernel that reads the same bytes from HBM stays above. It has no reference
// counterpart (the reference times a device-to-device copy for the same purpose,
// stbl/bench_gemv.py:58-61).
//
// Every thread issues kReadLoads 16-byte non-temporal loads, one per pass over the workgroup's span, all
// before its first use (2 loads x 512 threads was the fastest of the shapes measured: 1-16 loads per
// thread, 64-1024 threads, row-contiguous waves; 3.06 us for 7.8 MB, 19.7 us for 125 MB) (the loads of a wave cover consecutive kilobytes, as the GEMV weight loads
// do), folds them with XOR, the wave folds its lanes' words, and lane 0 writes one word per wave, so
// no load can be dropped. Bytes past the range are not read (the last unit clamps its address and
// drops its value).
#include "abi_util.hpp"
#include "common.hpp"

namespace stbl {

constexpr int kReadLoads = 2;
constexpr int kReadThreads = 512;

__global__ __launch_bounds__(kReadThreads) void k_read_floor(const u32x4 *__restrict__ src, uint64_t units,
                                                             uint32_t *__restrict__ sink) {
    const uint64_t base = (uint64_t)blockIdx.x * kReadThreads * kReadLoads + threadIdx.x;
    u32x4 v[kReadLoads];
#pragma unroll
    for (int i = 0; i < kReadLoads; i++) {
        const uint64_t u = base + (uint64_t)i * kReadThreads;
        v[i] = __builtin_nontemporal_load(src + (u < units ? u : units - 1));
    }
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < kReadLoads; i++) {
        const uint64_t u = base + (uint64_t)i * kReadThreads;
        if (u < units) acc ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o, kWave);
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * (kReadThreads / 64) + (threadIdx.x >> 6)] = acc;
}

// Clock stamps for the measurements: one thread writes the GPU's constant-rate wall clock
// (s_memrealtime, hipDeviceAttributeWallClockRate kHz) into t[i] as the kernel starts. Captured in
// a graph between launches, consecutive stamps bracket exactly the launches between them.
__global__ void k_clock_stamp(uint64_t *t, int i) {
    const uint64_t now = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) t[i] = now;
}

}  // namespace stbl

using namespace stbl;

extern "C" {

// Reads `bytes` (a multiple of 16, 16-byte aligned src) in one launch; sink receives one word per
// wave and must hold stbl_amd_read_floor_sink_words(bytes) words.
uint64_t stbl_amd_read_floor_sink_words(uint64_t bytes) {
    const uint64_t per_wg = (uint64_t)kReadThreads * kReadLoads * 16;
    return (bytes + per_wg - 1) / per_wg * (kReadThreads / 64);
}

int stbl_amd_read_floor(const void *src, uint64_t bytes, void *sink, hipStream_t st) {
    if (!src || !sink || bytes == 0 || bytes % 16 || !aligned16(src))
        return abi_fail(hipErrorInvalidValue, "read_floor: need a 16-byte aligned src and bytes %% 16 == 0");
    const uint64_t per_wg = (uint64_t)kReadThreads * kReadLoads * 16;
    const uint64_t wgs = (bytes + per_wg - 1) / per_wg;
    if (wgs > 0x7fffffffull) return abi_fail(hipErrorInvalidValue, "read_floor: too many bytes");
    hipLaunchKernelGGL(k_read_floor, dim3((unsigned)wgs), dim3(kReadThreads), 0, st, (const u32x4 *)src, bytes / 16,
                       (uint32_t *)sink);
    return abi_status(hipGetLastError(), "read_floor launch");
}

// Writes the wall clock into t[i] (device memory) when the launch starts on st.
int stbl_amd_clock_stamp(uint64_t *t, int i, hipStream_t st) {
    if (!t || i < 0) return abi_fail(hipErrorInvalidValue, "clock_stamp: need a buffer and i >= 0");
    hipLaunchKernelGGL(k_clock_stamp, dim3(1), dim3(64), 0, st, t, i);
    return abi_status(hipGetLastError(), "clock_stamp launch");
}

// The stamps' clock rate in kHz (ticks per millisecond) of the current device.
int stbl_amd_clock_rate_khz(int *khz) {
    if (!khz) return abi_fail(hipErrorInvalidValue, "clock_rate_khz: null output");
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(khz, hipDeviceAttributeWallClockRate, dev);
    return abi_status(e, "clock_rate_khz");
}

}  // extern "C"
