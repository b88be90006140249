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
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

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
// Wave-level inclusive scans with DPP (gfx9 encodings): Hillis-Steele over each 16-lane row with row_shr 1, 2, 4, 8,
// then row 0's total into row 1 and row 2's into row 3 (row_bcast:15 on rows 1 and 3), then the total of rows 0-1
// into rows 2-3 (row_bcast:31 on rows 2 and 3). Lanes whose source is outside the row read 0. Lane 63 ends with
// the wave total. The additions happen in a fixed order, so floating-point results are reproducible; each step
// is a VALU op, far cheaper than a cross-lane permute through the LDS crossbar.
template <int CTRL, int ROW_MASK>
__device__ inline uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, false);
}
template <int CTRL, int ROW_MASK>
__device__ inline double dpp_f64(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = dpp_u32<CTRL, ROW_MASK>((uint32_t)u);
    const uint32_t hi = dpp_u32<CTRL, ROW_MASK>((uint32_t)(u >> 32));
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ inline uint32_t wave_incl_scan_u32(uint32_t v) {
    v += dpp_u32<0x111, 0xf>(v);
    v += dpp_u32<0x112, 0xf>(v);
    v += dpp_u32<0x114, 0xf>(v);
    v += dpp_u32<0x118, 0xf>(v);
    v += dpp_u32<0x142, 0xa>(v);
    v += dpp_u32<0x143, 0xc>(v);
    return v;
}
__device__ inline double wave_incl_scan_f64(double v) {
    v += dpp_f64<0x111, 0xf>(v);
    v += dpp_f64<0x112, 0xf>(v);
    v += dpp_f64<0x114, 0xf>(v);
    v += dpp_f64<0x118, 0xf>(v);
    v += dpp_f64<0x142, 0xa>(v);
    v += dpp_f64<0x143, 0xc>(v);
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

// The LiDAR depth and confidence/2 clamped to [0, 1] seen by pixel (b, i, j) of an H x W map: F.interpolate
// mode='nearest' from dh x dw, source row floor(i * (dh / H)) (the scale in fp32), clamped to the last row
// (v3.py:374-375, 389-390).
__device__ inline void lidar_at(const float* lidar, const float* conf, int b, int i, int j, int H, int W, int dh,
                                int dw, float& d, float& c) {
    const float scy = (float)dh / (float)H, scx = (float)dw / (float)W;
    int sy = (int)__builtin_floorf((float)i * scy);
    int sx = (int)__builtin_floorf((float)j * scx);
    sy = sy < dh - 1 ? sy : dh - 1;
    sx = sx < dw - 1 ? sx : dw - 1;
    const int64_t p = ((int64_t)b * dh + sy) * dw + sx;
    d = lidar[p];
    c = fmin_(fmax_(conf[p] / 2.0f, 0.0f), 1.0f);
}

// _lidar_uncertainty (v3.py:386-393) with range_uncertainty (prompt_stem.py:41-42, falloff 3 m -> 5 m):
// u = 1 - c * (1 - clamp((d - 3) / 2, 0, 1)) where the LiDAR has a value, else 1.
__device__ inline float lidar_uncertainty(float d, float c) {
    const bool valid = __builtin_isfinite(d) && d > 0.0f;
    const float ru = fmin_(fmax_((d - 3.0f) / 2.0f, 0.0f), 1.0f);
    return valid ? 1.0f - c * (1.0f - ru) : 1.0f;
}

// One channel of the level-0 residual stream h = input_proj(x/z, y/z, logz) (+ prompt_proj(residual, gate))
// (sparse_unet.py:189-192), in the one operation order every kernel that forms it uses, so a kernel that recomputes
// h instead of reading it gets the same bits. w: the channel's input_proj row (3), b its bias; pw, pb: prompt_proj's.
__device__ inline float x0_channel(float w0, float w1, float w2, float b, float f0, float f1, float f2, bool prompt,
                                   float pw0, float pw1, float pb, float res, float gate) {
    float t = b + w0 * f0;
    t = t + w1 * f1;
    t = t + w2 * f2;
    if (prompt) {
        float pp = pb + pw0 * res;
        pp = pp + pw1 * gate;
        t = t + pp;
    }
    return t;
}

// Row layout shared by the fused epilogues and the row kernels: a wave covers 16 rows; lane l holds row l % 16
// and, of its C channels, n = 16j + 4g + i with g = l / 16 (j < C/16, i < 4). Row reductions run in the "quad"
// order: each lane sums its channels (j outer, i inner) from 0, then the four lane groups combine as
// ((s0 + s1) + (s2 + s3)) -- identical in every lane.
__device__ inline float quad_sum(float s) {
    const float a = s + __shfl_xor(s, 16, 64);
    return a + __shfl_xor(a, 32, 64);
}

// SiLU of a value that is stored as fp16: the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32, within 1 ulp
// each) give silu(y) with a relative error below |y| * 7.4e-8 + 4.2e-7, far under fp16's half-ulp (2^-12
// relative), so the rounded half is the correctly rounded silu_f32 or its neighbour (the two differ only when a
// rounding tie of fp16 falls between them). About 6 instructions instead of silu_f32's ~50. Every int8 code keeps
// the exact form (a code flips at a .5 tie).
__device__ inline float silu_fast(float y) {
    const float e = __builtin_amdgcn_exp2f(y * -PMG_LOG2E);
    return y * __builtin_amdgcn_rcpf(1.0f + e);
}

// LayerNorm (two-pass, quad order) + affine + SiLU of the lane's NB x 4 channels of one row, in place. SILU is set
// only where the result is stored as fp16 (int8 outputs apply SiLU inside their requantisation), so it uses
// silu_fast.
template <int NB, bool SILU = true, class P = const float*>
__device__ inline void ln_silu_quad(float (&y)[NB][4], P gamma, P beta, float eps, int g) {
    constexpr int C = 16 * NB;
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) s = s + y[j][i];
    const float mean = quad_sum(s) / (float)C;
    float vs = 0.0f;
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float d = y[j][i] - mean;
            vs = vs + d * d;
        }
    const float var = quad_sum(vs) / (float)C;
    const float rstd = 1.0f / __builtin_sqrtf(var + eps);
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = 16 * j + 4 * g + i;
            float t = (y[j][i] - mean) * rstd;
            t = t * gamma[n];
            t = t + beta[n];
            y[j][i] = SILU ? silu_fast(t) : t;
        }
}

// q = quant_i8(silu_f32(y), mult), bit for bit, at a fraction of the cost. The hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32: within 1 ulp; 0.77 and 0.88 ulp measured on gfx950) give v = silu(y) * mult with a relative
// error below |y| * 7.4e-8 + 4.2e-7 (exponent argument rounding, 1 ulp each for exp2 and rcp, 4 roundings); the
// exact evaluation is within 4.5e-7 of the true value. So unless v lies within twice the sum of both bounds of a
// rounding tie (k + 1/2, including the saturation edge 127.5), both round to the same integer, and only those rare
// elements (a few per 10^4) take the exact path. NaN and infinities fall through to the same clamp as the exact form.
__device__ inline float silu_quant_fast(float y, float mult, bool& unsure) {
    const float e = __builtin_amdgcn_exp2f(y * -PMG_LOG2E);
    const float v = (y * __builtin_amdgcn_rcpf(1.0f + e)) * mult;
    const float q0 = rne(v);
    const float tol = __builtin_fabsf(v) * (__builtin_fabsf(y) * 1.5e-7f + 1.8e-6f);
    unsure = 0.5f - __builtin_fabsf(v - q0) <= tol;
    return fmin_(fmax_(q0, -127.0f), 127.0f);
}
__device__ inline int8_t silu_quant_i8(float y, float mult) {
    bool unsure;
    float q = silu_quant_fast(y, mult, unsure);
    if (unsure) q = quant_f32(silu_f32(y), mult);
    return (int8_t)(int)q;
}

// The int8 codes (quant by mult) of 4 channels, packed into a word (channel i in byte i).
__device__ inline uint32_t pack_codes4(const float (&h)[4], float mult) {
    uint32_t pk = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) pk |= (uint32_t)(uint8_t)quant_i8(h[i], mult) << (8 * i);
    return pk;
}
// Stores the lane's 4 channels of block j of row m as int8 codes (quant by mult) or fp16.
__device__ inline void store_codes4(const float (&h)[4], float mult, int8_t* q) { *(uint32_t*)q = pack_codes4(h, mult); }
// As pack_codes4 for silu(t): the codes of silu of the 4 pre-activations t (silu_quant_i8 with one branch to the
// exact evaluation per 4 values).
__device__ inline uint32_t pack_silu_codes4(const float (&t)[4], float mult) {
    float c[4];
    bool u[4], any = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        c[i] = silu_quant_fast(t[i], mult, u[i]);
        any = any || u[i];
    }
    if (any) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (u[i]) c[i] = quant_f32(silu_f32(t[i]), mult);
    }
    uint32_t pk = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) pk |= (uint32_t)(uint8_t)(int)c[i] << (8 * i);
    return pk;
}
__device__ inline void store_silu_codes4(const float (&t)[4], float mult, int8_t* q) {
    *(uint32_t*)q = pack_silu_codes4(t, mult);
}

// A 4 x 4 transpose of words between the four 16-lane groups of a wave: on entry word k of lane group g is
// element (k, g), on exit it holds element (g, k) (two v_permlane32_swap, two v_permlane16_swap; lanes keep their
// position within the group). With word k of lane (r, g) holding the 4 codes of channels 16k + 4g .. +3 of row r
// (the MFMA output layout of a 64-channel block), lane (r, g) then holds channels 16g .. 16g + 15 in words 0..3:
// 16 contiguous bytes, so a row of the block is stored by four 16-byte lanes instead of sixteen 4-byte ones.
__device__ inline void lane_groups_transpose4(uint32_t (&w)[4]) {
    const auto a = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    w[0] = c[0];
    w[1] = c[1];
    w[2] = d[0];
    w[3] = d[1];
}
// silu_quant_i8 of NB x 4 values, packed four codes to a word, with one branch to the exact evaluation for all of
// them (so the fast evaluations of the NB x 4 values can interleave).
template <int NB>
__device__ inline void silu_codes_packed(const float (&t)[NB][4], float mult, uint32_t (&pk)[NB]) {
    float c[NB][4];
    bool u[NB][4], any = false;
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            c[j][i] = silu_quant_fast(t[j][i], mult, u[j][i]);
            any = any || u[j][i];
        }
    if (any) {
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (u[j][i]) c[j][i] = quant_f32(silu_f32(t[j][i]), mult);
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        pk[j] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) pk[j] |= (uint32_t)(uint8_t)(int)c[j][i] << (8 * i);
    }
}
__device__ inline void store_half4(const float (&h)[4], _Float16* o) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    h4 hv;
#pragma unroll
    for (int i = 0; i < 4; ++i) hv[i] = (_Float16)h[i];
    *(h4*)o = hv;
}

// Fill kernels (used instead of hipMemsetAsync so that the step can be captured into a HIP graph).
void fill_u32(void* p, uint32_t value, int64_t n, hipStream_t s);

}  // namespace pmg
