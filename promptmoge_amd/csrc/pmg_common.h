// Internal helpers shared by the HIP translation units of libpmg.so.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/pmg.h"
#include "pmg_math.h"

namespace pmg {

// ---------------------------------------------------------------------------------------------------------------
// Errors: every entry point returns a status and leaves a thread-local message.
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

#define PMG_CHECK_HIP(expr)                                                                       \
    do {                                                                                          \
        hipError_t e_ = (expr);                                                                   \
        if (e_ != hipSuccess)                                                                     \
            return ::pmg::fail(PMG_E_HIP, std::string(#expr) + ": " + hipGetErrorString(e_));    \
    } while (0)

#define PMG_REQUIRE(cond, msg)                                                     \
    do {                                                                           \
        if (!(cond)) return ::pmg::fail(PMG_E_INVALID, std::string(__func__) + ": " + (msg)); \
    } while (0)

// Checks the launch that was just issued (invalid configuration, missing code object, ...).
int check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Number of compute units of the current device (cached per device).
int num_cus();

// ---------------------------------------------------------------------------------------------------------------
// Vector types for MFMA operands (16 bytes per lane).
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------------------------------------------------------
// Wave-level reductions (64 lanes), deterministic butterfly order.
__device__ inline int wave_min_i32(int v) {
    for (int o = 32; o > 0; o >>= 1) { int t = __shfl_xor(v, o, 64); v = t < v ? t : v; }
    return v;
}
__device__ inline int wave_max_i32(int v) {
    for (int o = 32; o > 0; o >>= 1) { int t = __shfl_xor(v, o, 64); v = t > v ? t : v; }
    return v;
}

// ---------------------------------------------------------------------------------------------------------------
// Device-wide barrier for persistent kernels whose whole grid is resident (grid <= CUs x resident blocks/CU, one
// kernel on the stream at a time). `counter` starts at 0 for the launch; barrier number `index` (0, 1, 2, ...)
// waits until counter == (index + 1) * nblocks. The wait is bounded: on expiry the block raises `err` and every
// later barrier of the launch returns at once, so the kernel always terminates.
// Release/acquire at agent scope make the writes of every block visible across the XCDs' L2 caches.
__device__ inline void grid_barrier(unsigned* counter, unsigned index, unsigned nblocks, int* err) {
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned target = (index + 1u) * nblocks;
        if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
            unsigned spins = 0;
            while (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
                __builtin_amdgcn_s_sleep(2);
                if (++spins > (1u << 22)) {
                    __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
}

// Fill kernels (used instead of hipMemsetAsync so that the step can be captured into a HIP graph).
void fill_u32(void* p, uint32_t value, int64_t n, hipStream_t s);

}  // namespace pmg
