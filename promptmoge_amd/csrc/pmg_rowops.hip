// Per-voxel row operations of the refiner: the fused input stage (voxel keys, prompt residual, input/prompt
// projections, the first block's LayerNorm/SiLU/quantise) and the standalone LayerNorm/SiLU/quantise. One thread per
// voxel row, channel loops unrolled at compile time (C is a template parameter), every sum in a fixed order so that
// the NumPy restatement reproduces the bits.
#include <cstring>

#include "pmg_common.h"
#include "pmg_internal.h"

namespace pmg {

__global__ void fill_u32_k(uint32_t* p, uint32_t v, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = v;
}

void fill_u32(void* p, uint32_t value, int64_t n, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(fill_u32_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (uint32_t*)p, value, n);
}

// Sum of a row in the "quad" order shared with the convolution epilogues (pmg_conv_col.hip): group g accumulates
// channels 16j + 4g + i (j outer, i inner), then ((s0 + s1) + (s2 + s3)).
template <int C>
__device__ inline float quad_row_sum(const float (&v)[C]) {
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < C / 16; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) s[g] = s[g] + v[16 * j + 4 * g + i];
    return (s[0] + s[1]) + (s[2] + s[3]);
}

// LayerNorm (two-pass), affine, SiLU. flex_sparse_blocks.py:230 (norm1, eps 1e-6, then SiLU).
template <int C>
__device__ inline void ln_silu_row(float (&h)[C], const float* gamma, const float* beta, float eps) {
    const float mean = quad_row_sum<C>(h) / (float)C;
    float d2[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const float d = h[c] - mean;
        d2[c] = d * d;
    }
    const float var = quad_row_sum<C>(d2) / (float)C;
    const float rstd = 1.0f / __builtin_sqrtf(var + eps);
#pragma unroll
    for (int c = 0; c < C; ++c) {
        float y = (h[c] - mean) * rstd;
        y = y * gamma[c];
        y = y + beta[c];
        h[c] = silu_f32(y);
    }
}

template <int C>
__device__ inline void store_q_row(const float (&h)[C], float out_scale, int8_t* q) {
#pragma unroll
    for (int c0 = 0; c0 < C; c0 += 16) {
        int32_t pk[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t b = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) b |= (uint32_t)(uint8_t)quant_i8(h[c0 + 4 * k + e], out_scale) << (8 * e);
            pk[k] = (int32_t)b;
        }
        *(int4*)(q + c0) = make_int4(pk[0], pk[1], pk[2], pk[3]);
    }
}

template <int C>
__device__ inline void store_h_row(const float (&h)[C], _Float16* o) {
#pragma unroll
    for (int c0 = 0; c0 < C; c0 += 8) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        h8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (_Float16)h[c0 + e];
        *(h8*)(o + c0) = v;
    }
}

template <int C>
__device__ inline void load_row(const float* x, float (&h)[C]) {
#pragma unroll
    for (int c = 0; c < C; c += 4) {
        const float4 v = *(const float4*)(x + c);
        h[c] = v.x;
        h[c + 1] = v.y;
        h[c + 2] = v.z;
        h[c + 3] = v.w;
    }
}

template <int C>
__device__ inline void store_row(float* x, const float (&h)[C]) {
#pragma unroll
    for (int c = 0; c < C; c += 4) *(float4*)(x + c) = make_float4(h[c], h[c + 1], h[c + 2], h[c + 3]);
}

template <int C, bool F16>
__global__ __launch_bounds__(256) void ln_silu_k(const float* __restrict__ x, int64_t M,
                                                 const float* __restrict__ gamma, const float* __restrict__ beta,
                                                 float eps, float out_scale, void* __restrict__ out) {
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (m >= M) return;
    float h[C];
    load_row<C>(x + m * C, h);
    ln_silu_row<C>(h, gamma, beta, eps);
    if constexpr (F16)
        store_h_row<C>(h, (_Float16*)out + m * C);
    else
        store_q_row<C>(h, out_scale, (int8_t*)out + m * C);
}

// ------------------------------------------------------------------------------------------------------------
// Fused input stage of one refiner step (single level):
//   prompt residual and gate          MoGeModel._lidar_in_affine_frame, v3.py:373-383, and v3.py:552-555
//   h = input_proj(x/z, y/z, logz) (+ prompt_proj(residual, gate))   sparse_unet.py:189-192
//   x_out = h (the residual stream), then the first block's LayerNorm/SiLU and quantise (or fp16).
// Nearest resizing of the LiDAR map uses F.interpolate's index rule src = min(floor(dst * (in/out)), in-1).
struct InputArgs {
    const float* points;  // [M][3]
    int B, H, W;
    const float* lidar;  // [B][dh][dw]
    const float* conf;
    int dh, dw;
    const float* st;  // [B][2] prompt-fit (s, t)
    int use_prompt, soft_gate;
    const float* in_w;  // [C][3]
    const float* in_b;
    const float* pr_w;  // [C][2]
    const float* pr_b;
    float* x_out;  // [M][C]
    const float* gamma;
    const float* beta;
    float eps;
    float out_scale;
    void* q_out;        // int8 or fp16 [M][C]
    float resolution;   // voxel keys: zq = rint(logz * resolution) (v3.py:332)
    int32_t* zq_out;    // [M] or NULL
};

__device__ inline void prompt_feats(const InputArgs& a, int b, int i, int j, float logz, float& res, float& gate) {
    const float scy = (float)a.dh / (float)a.H, scx = (float)a.dw / (float)a.W;
    int sy = (int)__builtin_floorf((float)i * scy);
    int sx = (int)__builtin_floorf((float)j * scx);
    sy = sy < a.dh - 1 ? sy : a.dh - 1;
    sx = sx < a.dw - 1 ? sx : a.dw - 1;
    const int64_t p = ((int64_t)b * a.dh + sy) * a.dw + sx;
    const float d = a.lidar[p];
    const float c = fmin_(fmax_(a.conf[p] / 2.0f, 0.0f), 1.0f);
    const bool valid = __builtin_isfinite(d) && d > 0.0f;
    const float s = a.st[2 * b], t = a.st[2 * b + 1];
    const float daff = (d - t) / fmax_(s, 1e-6f);
    const bool ok = valid && daff > 1e-4f;
    const float lda = ok ? log_f32(fmax_(daff, 1e-4f)) : logz;
    const float okf = ok ? 1.0f : 0.0f;
    gate = a.soft_gate ? (0.15f + 0.85f * c) * okf : c * okf;
    res = (lda - logz) * gate;
}

template <int C, bool F16>
__global__ __launch_bounds__(256) void input_stage_k(InputArgs a) {
    const int64_t M = (int64_t)a.B * a.H * a.W;
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (m >= M) return;
    const float f0 = a.points[m * 3 + 0], f1 = a.points[m * 3 + 1], f2 = a.points[m * 3 + 2];
    if (a.zq_out) a.zq_out[m] = (int32_t)rne(f2 * a.resolution);
    float res = 0.0f, gate = 0.0f;
    if (a.use_prompt) {
        const int64_t HW = (int64_t)a.H * a.W;
        const int b = (int)(m / HW);
        const int p = (int)(m - b * HW);
        const int i = p / a.W, j = p - (p / a.W) * a.W;
        prompt_feats(a, b, i, j, f2, res, gate);
    }
    float h[C];
#pragma unroll
    for (int n = 0; n < C; ++n) {
        float y = a.in_b[n] + a.in_w[3 * n] * f0;
        y = y + a.in_w[3 * n + 1] * f1;
        y = y + a.in_w[3 * n + 2] * f2;
        if (a.use_prompt) {
            float pp = a.pr_b[n] + a.pr_w[2 * n] * res;
            pp = pp + a.pr_w[2 * n + 1] * gate;
            y = y + pp;
        }
        h[n] = y;
    }
    store_row<C>(a.x_out + m * C, h);
    ln_silu_row<C>(h, a.gamma, a.beta, a.eps);
    if constexpr (F16)
        store_h_row<C>(h, (_Float16*)a.q_out + m * C);
    else
        store_q_row<C>(h, a.out_scale, (int8_t*)a.q_out + m * C);
}

// ------------------------------------------------------------------------------------------------------------
#define PMG_C_SWITCH(C, BODY)               \
    switch (C) {                            \
        case 16: { constexpr int CC = 16; BODY; break; } \
        case 32: { constexpr int CC = 32; BODY; break; } \
        case 48: { constexpr int CC = 48; BODY; break; } \
        case 64: { constexpr int CC = 64; BODY; break; } \
        case 96: { constexpr int CC = 96; BODY; break; } \
        case 128: { constexpr int CC = 128; BODY; break; } \
        default: return fail(PMG_E_INVALID, "unsupported channel count " + std::to_string(C)); \
    }

bool supported_width(int C) { return C == 16 || C == 32 || C == 48 || C == 64 || C == 96 || C == 128; }

int launch_ln_silu(const float* x, int64_t M, int C, const float* gamma, const float* beta, float eps,
                   float out_scale, void* out, bool f16, hipStream_t s) {
    if (M == 0) return PMG_OK;
    const dim3 g((unsigned)((M + 255) / 256));
    if (f16) {
        PMG_C_SWITCH(C, hipLaunchKernelGGL((ln_silu_k<CC, true>), g, dim3(256), 0, s, x, M, gamma, beta, eps,
                                           out_scale, out));
    } else {
        PMG_C_SWITCH(C, hipLaunchKernelGGL((ln_silu_k<CC, false>), g, dim3(256), 0, s, x, M, gamma, beta, eps,
                                           out_scale, out));
    }
    return check_launch("ln_silu_k");
}

int launch_input_stage(const InputStage& in, bool f16, hipStream_t s) {
    InputArgs a{in.points, in.B, in.H, in.W, in.lidar, in.conf, in.dh, in.dw, in.st, in.use_prompt, in.soft_gate,
                in.in_w, in.in_b, in.pr_w, in.pr_b, in.x_out, in.gamma, in.beta, in.eps, in.out_scale, in.q_out,
                in.resolution, in.zq_out};
    const int64_t M = (int64_t)in.B * in.H * in.W;
    const dim3 g((unsigned)((M + 255) / 256));
    if (f16) {
        PMG_C_SWITCH(in.C, hipLaunchKernelGGL((input_stage_k<CC, true>), g, dim3(256), 0, s, a));
    } else {
        PMG_C_SWITCH(in.C, hipLaunchKernelGGL((input_stage_k<CC, false>), g, dim3(256), 0, s, a));
    }
    return check_launch("input_stage_k");
}

// ------------------------------------------------------------------------------------------------------------
__device__ __host__ inline float math_op(int op, float x) {
    return op == 0 ? exp_f32(x) : (op == 1 ? log_f32(x) : silu_f32(x));
}

__global__ void math_k(int op, const float* in, float* out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = math_op(op, in[i]);
}

}  // namespace pmg

using namespace pmg;

extern "C" {

int pmg_ln_silu_quant(const float* x, int64_t M, int C, const float* gamma, const float* beta, float eps,
                      float out_scale, int8_t* q, void* stream) {
    PMG_REQUIRE(x && gamma && beta && q, "null buffer");
    PMG_REQUIRE(M >= 0, "bad voxel count");
    PMG_REQUIRE(out_scale > 0.0f, "out_scale must be positive");
    PMG_REQUIRE(aligned16(x) && aligned16(q), "x and q must be 16-byte aligned");
    return launch_ln_silu(x, M, C, gamma, beta, eps, out_scale, q, false, (hipStream_t)stream);
}

int pmg_ln_silu_f16(const float* x, int64_t M, int C, const float* gamma, const float* beta, float eps,
                    uint16_t* h, void* stream) {
    PMG_REQUIRE(x && gamma && beta && h, "null buffer");
    PMG_REQUIRE(M >= 0, "bad voxel count");
    PMG_REQUIRE(aligned16(x) && aligned16(h), "x and h must be 16-byte aligned");
    return launch_ln_silu(x, M, C, gamma, beta, eps, 1.0f, h, true, (hipStream_t)stream);
}

int pmg_math_host(int op, const float* in, float* out, int64_t n) {
    PMG_REQUIRE(op >= 0 && op <= 2 && in && out && n >= 0, "bad argument");
    for (int64_t i = 0; i < n; ++i) out[i] = math_op(op, in[i]);
    return PMG_OK;
}

int pmg_math_device(int op, const float* in, float* out, int64_t n, void* stream) {
    PMG_REQUIRE(op >= 0 && op <= 2 && in && out && n >= 0, "bad argument");
    if (n == 0) return PMG_OK;
    hipLaunchKernelGGL(math_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, op, in, out,
                       n);
    return check_launch("math_k");
}

}  // extern "C"
