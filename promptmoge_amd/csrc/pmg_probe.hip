// Peak probes: the practical HBM bandwidth and int8 MFMA rate of the device this runs on, measured with the same
// instruction forms the kernels use (16-byte vector loads/stores; v_mfma_i32_16x16x64_i8). The benchmark reports
// each kernel against the published peaks and against these.
#include <climits>

#include "pmg_common.h"

namespace pmg {

// Streaming copy: each thread moves 4 independent 16-byte vectors (all loads issued before the first store).
__global__ __launch_bounds__(256) void probe_copy_k(const v4i* __restrict__ src, v4i* __restrict__ dst, int64_t n) {
    const int64_t base = (int64_t)blockIdx.x * 1024 + threadIdx.x;
    v4i v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t i = base + k * 256;
        v[k] = i < n ? src[i] : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t i = base + k * 256;
        if (i < n) dst[i] = v[k];
    }
}

// Register-only MFMA loop: `iters` rounds of 16 independent 16x16x64 int8 MFMAs per wave. The sum of the
// accumulators is compared with a value it cannot take, so the work is kept without storing anything.
__global__ __launch_bounds__(256) void probe_mfma_k(int iters, int32_t* sink) {
    const v4i a = {(int)threadIdx.x, 1, 2, 3}, b = {3, 2, 1, (int)blockIdx.x};
    v4i acc[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) acc[k] = v4i{k, 0, 0, 0};
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int k = 0; k < 16; ++k) acc[k] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[k], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) s += acc[k][0] + acc[k][1] + acc[k][2] + acc[k][3];
    if (s == 0x7fffffff && threadIdx.x == 0) sink[0] = s;
}

}  // namespace pmg

using namespace pmg;

extern "C" {

int pmg_probe_copy(const void* src, void* dst, int64_t bytes, void* stream) {
    PMG_REQUIRE(src && dst, "null buffer");
    PMG_REQUIRE(bytes > 0 && bytes % 16 == 0, "bytes must be a positive multiple of 16");
    PMG_REQUIRE(aligned16(src) && aligned16(dst), "buffers must be 16-byte aligned");
    const int64_t n = bytes / 16;
    PMG_REQUIRE((n + 1023) / 1024 <= INT_MAX, "too large");
    hipLaunchKernelGGL(probe_copy_k, dim3((unsigned)((n + 1023) / 1024)), dim3(256), 0, (hipStream_t)stream,
                       (const v4i*)src, (v4i*)dst, n);
    return check_launch("probe_copy_k");
}

int pmg_probe_mfma_i8(int iters, int waves_per_cu, int32_t* sink, void* stream) {
    PMG_REQUIRE(sink, "null sink");
    PMG_REQUIRE(iters > 0 && waves_per_cu >= 4 && waves_per_cu % 4 == 0 && waves_per_cu <= 32, "bad probe shape");
    const int blocks = num_cus() * waves_per_cu / 4;
    hipLaunchKernelGGL(probe_mfma_k, dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, sink);
    return check_launch("probe_mfma_k");
}

}  // extern "C"
