// Per-voxel row operations of the refiner: the fused input stage (voxel keys, prompt residual, input/prompt
// projections, the first block's LayerNorm/SiLU/quantise) and the standalone LayerNorm/SiLU/quantise, both in the
// 16-rows-per-wave layout of the fused convolution epilogues, with every sum in a fixed order so that the NumPy
// restatement reproduces the bits.
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

// Standalone LayerNorm -> SiLU -> int8 codes (or fp16) in the row layout of the fused epilogues: a wave covers 16
// rows, lane l row l % 16 and channels 16j + 4g + i (g = l / 16), so the sums run in the same quad order and the
// stores are 4- and 16-byte vectors.
template <int C, bool F16>
__global__ __launch_bounds__(256) void ln_silu_k(const float* __restrict__ x, int64_t M,
                                                 const float* __restrict__ gamma, const float* __restrict__ beta,
                                                 float eps, float out_mult, void* __restrict__ out) {
    constexpr int NB = C / 16;
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const int64_t m = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 16 + r;
    const bool ok = m < M;
    const int64_t mo = ok ? m : 0;
    float y[NB][4];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const float4 v = *(const float4*)(x + mo * C + 16 * j + 4 * g);
        y[j][0] = v.x;
        y[j][1] = v.y;
        y[j][2] = v.z;
        y[j][3] = v.w;
    }
    ln_silu_quad<NB, F16>(y, gamma, beta, eps, g);
    if (!ok) return;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int64_t o = mo * C + 16 * j + 4 * g;
        if constexpr (F16)
            store_half4(y[j], (_Float16*)out + o);
        else
            store_silu_codes4(y[j], out_mult, (int8_t*)out + o);
    }
}

// ------------------------------------------------------------------------------------------------------------
// Fused input stage of one refiner step (single level):
//   prompt residual and gate          MoGeModel._lidar_in_affine_frame, v3.py:373-383, and v3.py:552-555
//   h = input_proj(x/z, y/z, logz) (+ prompt_proj(residual, gate))   sparse_unet.py:189-192
//   x_out = h (the residual stream; or NULL when the first block's conv recomputes h: rg_out then keeps the prompt
//   features for it), then the first block's LayerNorm/SiLU and quantise (or fp16).
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
    float out_mult;
    void* q_out;        // int8 or fp16 [M][C]
    float resolution;   // voxel keys: zq = rint(logz * resolution) (v3.py:332)
    int32_t* zq_out;    // [M] or NULL
    const float* prompt_in;  // [M][2] given prompt features (residual, gate), or NULL: computed from the LiDAR
    const int32_t* zkeys;    // given voxel z keys (coords[:, 3], element stride zkey_stride), or NULL
    int64_t zkey_stride;
    float* rg_out;  // [M][2] the prompt features (residual, gate) of each row, or NULL
};

__device__ inline void prompt_feats(const InputArgs& a, int b, int i, int j, float logz, float& res, float& gate) {
    float d, c;
    lidar_at(a.lidar, a.conf, b, i, j, a.H, a.W, a.dh, a.dw, d, c);
    const bool valid = __builtin_isfinite(d) && d > 0.0f;
    const float s = a.st[2 * b], t = a.st[2 * b + 1];
    const float daff = (d - t) / fmax_(s, 1e-6f);
    const bool ok = valid && daff > 1e-4f;
    const float lda = ok ? log_f32(fmax_(daff, 1e-4f)) : logz;
    const float okf = ok ? 1.0f : 0.0f;
    gate = a.soft_gate ? (0.15f + 0.85f * c) * okf : c * okf;
    res = (lda - logz) * gate;
}

// One row per lane: the lane forms all C channels of its row in registers, so the row's own work (voxel key, LiDAR
// lookup and prompt features, the LayerNorm statistics) is done once per row rather than once per lane group, and
// the codes of a row are stored as 16-byte vectors. The per-channel constants are the same for every lane (scalar
// loads). The LayerNorm sums keep the quad order of the row layout of the epilogues -- partial sums s_g over
// channels 16j + 4g + i (j outer, i inner), then ((s0 + s1) + (s2 + s3)) -- so the codes are those of that layout.
template <int C, bool F16>
__global__ __launch_bounds__(256) void input_stage_k(InputArgs a) {
    constexpr int NB = C / 16, NQ = C / 4;
    // in_w [C][3], in_b, pr_w [C][2], pr_b, gamma, beta: read by every lane at the same address (LDS broadcast)
    __shared__ __attribute__((aligned(16))) float s_c[9 * C];
    for (int e = threadIdx.x; e < 9 * C; e += 256) {
        float v;
        if (e < 3 * C) v = a.in_w[e];
        else if (e < 4 * C) v = a.in_b[e - 3 * C];
        else if (e < 6 * C) v = a.use_prompt ? a.pr_w[e - 4 * C] : 0.0f;
        else if (e < 7 * C) v = a.use_prompt ? a.pr_b[e - 6 * C] : 0.0f;
        else if (e < 8 * C) v = a.gamma[e - 7 * C];
        else v = a.beta[e - 8 * C];
        s_c[e] = v;
    }
    typedef const __attribute__((address_space(3))) v4f* c4;
    const c4 c_inw = (c4)s_c, c_inb = (c4)(s_c + 3 * C), c_prw = (c4)(s_c + 4 * C), c_prb = (c4)(s_c + 6 * C);
    const c4 c_gam = (c4)(s_c + 7 * C), c_bet = (c4)(s_c + 8 * C);
    const int64_t M = (int64_t)a.B * a.H * a.W;
    const int64_t m0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const bool ok = m0 < M;
    const int64_t m = ok ? m0 : M - 1;
    const float f0 = a.points[m * 3 + 0], f1 = a.points[m * 3 + 1], f2 = a.points[m * 3 + 2];
    if (ok && a.zq_out) a.zq_out[m] = a.zkeys ? a.zkeys[m * a.zkey_stride] : (int32_t)rne(f2 * a.resolution);
    float res = 0.0f, gate = 0.0f;
    if (a.prompt_in) {  // Sparse3DUNet.forward's prompt_feats (sparse_unet.py:191-193)
        res = a.prompt_in[m * 2];
        gate = a.prompt_in[m * 2 + 1];
    } else if (a.use_prompt) {
        const int64_t HW = (int64_t)a.H * a.W;
        const int b = (int)(m / HW);
        const int p = (int)(m - b * HW);
        const int i = p / a.W, j = p - (p / a.W) * a.W;
        prompt_feats(a, b, i, j, f2, res, gate);
    }
    if (ok && a.rg_out) *(float2*)(a.rg_out + m * 2) = make_float2(res, gate);
    __syncthreads();  // constants staged
    const bool prompt = a.use_prompt;
    // (one quad of channels between scheduling barriers: the constants of one quad are live at a time)
    float y[NQ][4];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const v4f w0 = c_inw[3 * q], w1 = c_inw[3 * q + 1], w2 = c_inw[3 * q + 2], b = c_inb[q];
        const v4f p0 = c_prw[2 * q], p1 = c_prw[2 * q + 1], pb = c_prb[q];
        const float wi[12] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
        const float pw[8] = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
#pragma unroll
        for (int i = 0; i < 4; ++i)
            y[q][i] = x0_channel(wi[3 * i], wi[3 * i + 1], wi[3 * i + 2], b[i], f0, f1, f2, prompt, pw[2 * i],
                                 pw[2 * i + 1], pb[i], res, gate);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (ok && a.x_out) {
#pragma unroll
        for (int q = 0; q < NQ; ++q)
            *(float4*)(a.x_out + m * C + 4 * q) = make_float4(y[q][0], y[q][1], y[q][2], y[q][3]);
    }
    // LayerNorm (two-pass) + affine, in the quad order
    float sg[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) sg[g] = sg[g] + y[4 * j + g][i];
    const float mean = ((sg[0] + sg[1]) + (sg[2] + sg[3])) / (float)C;
    float vg[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float d = y[4 * j + g][i] - mean;
                vg[g] = vg[g] + d * d;
            }
    const float var = ((vg[0] + vg[1]) + (vg[2] + vg[3])) / (float)C;
    const float rstd = 1.0f / __builtin_sqrtf(var + a.eps);
    // per 16 channels: normalise, then the fp16 SiLU or the int8 codes, one 16-byte store (fp16: two)
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        float t[4][4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const v4f gm = c_gam[4 * j + q], bt = c_bet[4 * j + q];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float v = (y[4 * j + q][i] - mean) * rstd;
                v = v * gm[i];
                v = v + bt[i];
                t[q][i] = F16 ? silu_fast(v) : v;
            }
        }
        if constexpr (F16) {
            typedef _Float16 h8 __attribute__((ext_vector_type(8)));
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                h8 hv;
#pragma unroll
                for (int i = 0; i < 8; ++i) hv[i] = (_Float16)t[2 * h + i / 4][i % 4];
                if (ok) *(h8*)((_Float16*)a.q_out + m * C + 16 * j + 8 * h) = hv;
            }
        } else {
            uint32_t pk[4];
            silu_codes_packed<4>(t, a.out_mult, pk);
            if (ok) *(v4i*)((int8_t*)a.q_out + m * C + 16 * j) = v4i{(int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3]};
        }
        __builtin_amdgcn_sched_barrier(0);
    }
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
                   float out_mult, void* out, bool f16, hipStream_t s) {
    if (M == 0) return PMG_OK;
    const dim3 g((unsigned)((M + 63) / 64));
    if (f16) {
        PMG_C_SWITCH(C, hipLaunchKernelGGL((ln_silu_k<CC, true>), g, dim3(256), 0, s, x, M, gamma, beta, eps,
                                           out_mult, out));
    } else {
        PMG_C_SWITCH(C, hipLaunchKernelGGL((ln_silu_k<CC, false>), g, dim3(256), 0, s, x, M, gamma, beta, eps,
                                           out_mult, out));
    }
    return check_launch("ln_silu_k");
}

int launch_input_stage(const InputStage& in, bool f16, hipStream_t s) {
    InputArgs a{in.points, in.B, in.H, in.W, in.lidar, in.conf, in.dh, in.dw, in.st, in.use_prompt, in.soft_gate,
                in.in_w, in.in_b, in.pr_w, in.pr_b, in.x_out, in.gamma, in.beta, in.eps, in.out_mult, in.q_out,
                in.resolution, in.zq_out, in.prompt_in, in.zkeys, in.zkey_stride, in.rg_out};
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
    if (i >= n) return;
    if (op == 3)
        out[i] = (float)silu_quant_i8(in[2 * i], in[2 * i + 1]);
    else
        out[i] = math_op(op, in[i]);
}

// One thread per pixel: the elastic anchor of the refined logz toward the LiDAR in its affine frame (v3.py:570-573,
// _lidar_in_affine_frame 362-383 with the hard gate), fp32 in the reference's operation order.
__global__ __launch_bounds__(256) void anchor_k(float* points, int B, int H, int W, const float* lidar,
                                                const float* conf, int dh, int dw, const float* st, float beta) {
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int HW = H * W;
    if (m >= (int64_t)B * HW) return;
    const int b = (int)(m / HW), pix = (int)(m - (int64_t)b * HW);
    const int i = pix / W, j = pix - (pix / W) * W;
    float d, c;
    lidar_at(lidar, conf, b, i, j, H, W, dh, dw, d, c);
    const float lz = points[m * 3 + 2];
    const bool valid = __builtin_isfinite(d) && d > 0.0f;
    const float s = st[2 * b], t = st[2 * b + 1];
    const float daff = (d - t) / fmax_(s, 1e-6f);
    const bool ok = valid && daff > 1e-4f;
    const float lda = ok ? log_f32(fmax_(daff, 1e-4f)) : lz;
    const float gate = c * (ok ? 1.0f : 0.0f);
    points[m * 3 + 2] = lz + (beta * gate) * (lda - lz);
}

int launch_anchor(float* points, int B, int H, int W, const float* lidar, const float* conf, int dh, int dw,
                  const float* st, float beta, hipStream_t s) {
    const int64_t M = (int64_t)B * H * W;
    if (M == 0) return PMG_OK;
    hipLaunchKernelGGL(anchor_k, dim3((unsigned)((M + 255) / 256)), dim3(256), 0, s, points, B, H, W, lidar, conf, dh,
                       dw, st, beta);
    return check_launch("anchor_k");
}

}  // namespace pmg

using namespace pmg;

extern "C" {

int pmg_ln_silu_quant(const float* x, int64_t M, int C, const float* gamma, const float* beta, float eps,
                      float out_mult, int8_t* q, void* stream) {
    PMG_REQUIRE(x && gamma && beta && q, "null buffer");
    PMG_REQUIRE(M >= 0, "bad voxel count");
    PMG_REQUIRE(out_mult > 0.0f, "out_mult must be positive");
    PMG_REQUIRE(aligned16(x) && aligned16(q), "x and q must be 16-byte aligned");
    return launch_ln_silu(x, M, C, gamma, beta, eps, out_mult, q, false, (hipStream_t)stream);
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
    PMG_REQUIRE(op >= 0 && op <= 3 && in && out && n >= 0, "bad argument");
    if (n == 0) return PMG_OK;
    hipLaunchKernelGGL(math_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, op, in, out,
                       n);
    return check_launch("math_k");
}

}  // extern "C"
