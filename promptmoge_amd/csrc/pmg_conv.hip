// Submanifold 3x3x3 convolution as an output-stationary implicit GEMM on CDNA4 matrix cores.
//
//   out[m, n] = sum_v sum_c W[n, v, c] * x[nmap[v][m], c]        (submanifold_conv, _core.py:399-441)
//
// One wave owns a tile of 16 output rows and 16*NB output channels. The reduction dimension is flattened over
// (active tap, 16-byte channel chunk): a tile only visits the taps in its tap mask (written by the map build),
// and each MFMA step takes four consecutive chunks, one per 16-lane group. Because the chunk that a lane group
// loads for A (the gathered activation row x[nmap[v][m]], 16 bytes) is the same (tap, chunk) it loads for B
// (W[n][v][chunk], 16 bytes, the reference module's own (Co, 3, 3, 3, Ci) layout), the k order inside an MFMA is
// irrelevant to the result: only the row/column mapping of the 16x16 output block is used, lane l holding rows
// 4*(l/16)+i, column l%16.
//
//   int8  v_mfma_i32_16x16x64_i8    16 int8 per lane per chunk, exact int32 accumulation
//   fp16  v_mfma_f32_16x16x32_f16    8 halves per lane per chunk, fp32 accumulation (teacher)
//   fp32  v_mfma_f32_16x16x4_f32     4 floats per lane per chunk, one MFMA per float (flex_gemm shim on fp32)
//
// Rows are gathered straight from global memory into registers (16-byte loads hit L2 for the image-local
// neighbourhoods of level 0); the weights, at most 27*Co*Ci elements, stay L1/L2 resident.
#include "pmg_common.h"

namespace pmg {

struct ConvArgs {
    const uint8_t* x;
    const int32_t* nmap_t;
    const uint32_t* tmask;
    const uint8_t* w;
    int64_t M;
    int Co;
    int row_bytes;  // Ci * sizeof(T)
    int nchunk;     // row_bytes / 16
    float a_scale;
    const float* w_scale;
    const float* bias;
    float out_mult;
    const float* skip;
    void* out;
};

template <typename T>
struct Acc;
template <>
struct Acc<int8_t> {
    typedef v4i type;
};
template <>
struct Acc<_Float16> {
    typedef v4f type;
};
template <>
struct Acc<float> {
    typedef v4f type;
};

__device__ inline void mma(v4i& acc, const v4i& a, const v4i& b, int8_t) {
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
}
__device__ inline void mma(v4f& acc, const v4i& a, const v4i& b, _Float16) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), acc, 0,
                                                  0, 0);
}
__device__ inline void mma(v4f& acc, const v4i& a, const v4i& b, float) {
    const v4f af = __builtin_bit_cast(v4f, a), bf = __builtin_bit_cast(v4f, b);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af[0], bf[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af[1], bf[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af[2], bf[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(af[3], bf[3], acc, 0, 0, 0);
}

// Epilogue of one accumulator element (row m, column n).
template <typename T, int EPI>
__device__ inline void epilogue(const ConvArgs& a, int64_t m, int n, typename Acc<T>::type acc, int i) {
    const int64_t o = m * a.Co + n;
    if constexpr (sizeof(T) == 1) {
        const int32_t v = acc[i];
        if constexpr (EPI == PMG_EPI_ACC) {
            ((int32_t*)a.out)[o] = v;
        } else {
            float y = (float)v * a.a_scale;
            y = y * a.w_scale[n];
            if (a.bias) y = y + a.bias[n];
            if constexpr (EPI == PMG_EPI_Q) {
                ((int8_t*)a.out)[o] = silu_quant_i8(y, a.out_mult);
            } else if constexpr (EPI == PMG_EPI_R) {
                ((float*)a.out)[o] = y + a.skip[o];
            } else {
                ((float*)a.out)[o] = y;
            }
        }
    } else {
        float y = acc[i];
        if constexpr (EPI != PMG_EPI_ACC) {
            if (a.bias) y = y + a.bias[n];
        }
        if constexpr (EPI == PMG_EPI_SILU) {
            ((_Float16*)a.out)[o] = (_Float16)silu_f32(y);
        } else if constexpr (EPI == PMG_EPI_R) {
            ((float*)a.out)[o] = y + a.skip[o];
        } else {
            ((float*)a.out)[o] = y;
        }
    }
}

template <typename T, int NB, int EPI>
__global__ __launch_bounds__(256) void spconv_k(ConvArgs a) {
    __shared__ int8_t taps_s[4][32];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t tile = (int64_t)blockIdx.x * 4 + wv;
    const int64_t ntile = (a.M + 15) >> 4;
    const uint32_t mask = tile < ntile ? a.tmask[tile] : 0u;
    if (lane < 27 && ((mask >> lane) & 1u)) taps_s[wv][__popc(mask & ((1u << lane) - 1u))] = (int8_t)lane;
    __syncthreads();

    const int Q = __popc(mask) * a.nchunk;
    const int r = lane & 15, g = lane >> 4;
    const int64_t m0 = tile * 16;
    const int64_t row = m0 + r;
    const bool row_ok = row < a.M;
    const int n0 = blockIdx.y * 16 * NB;

    typename Acc<T>::type acc[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = typename Acc<T>::type{0, 0, 0, 0};

    for (int q0 = 0; q0 < Q; q0 += 4) {
        const int q = q0 + g;
        v4i av = {0, 0, 0, 0};
        v4i bv[NB];
        if (q < Q) {
            const int t = q / a.nchunk;
            const int c = q - t * a.nchunk;
            const int v = taps_s[wv][t];
            const int idx = row_ok ? a.nmap_t[(int64_t)v * a.M + row] : -1;
            if (idx >= 0 && idx < a.M) av = *(const v4i*)(a.x + (int64_t)idx * a.row_bytes + c * 16);
#pragma unroll
            for (int j = 0; j < NB; ++j)
                bv[j] = *(const v4i*)(a.w + ((int64_t)(n0 + 16 * j + r) * 27 + v) * a.row_bytes + c * 16);
        } else {
#pragma unroll
            for (int j = 0; j < NB; ++j) bv[j] = v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) mma(acc[j], av, bv[j], T{});
    }

#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int n = n0 + 16 * j + r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t m = m0 + 4 * g + i;
            if (m < a.M) epilogue<T, EPI>(a, m, n, acc[j], i);
        }
    }
}

template <typename T, int EPI>
static int launch_nb(const ConvArgs& a, int nb, hipStream_t s) {
    const int64_t ntile = (a.M + 15) >> 4;
    const dim3 grid((unsigned)((ntile + 3) / 4), (unsigned)(a.Co / (16 * nb)));
    switch (nb) {
        case 8: hipLaunchKernelGGL((spconv_k<T, 8, EPI>), grid, dim3(256), 0, s, a); break;
        case 6: hipLaunchKernelGGL((spconv_k<T, 6, EPI>), grid, dim3(256), 0, s, a); break;
        case 4: hipLaunchKernelGGL((spconv_k<T, 4, EPI>), grid, dim3(256), 0, s, a); break;
        case 3: hipLaunchKernelGGL((spconv_k<T, 3, EPI>), grid, dim3(256), 0, s, a); break;
        case 2: hipLaunchKernelGGL((spconv_k<T, 2, EPI>), grid, dim3(256), 0, s, a); break;
        default: hipLaunchKernelGGL((spconv_k<T, 1, EPI>), grid, dim3(256), 0, s, a); break;
    }
    return check_launch("spconv_k");
}

static int pick_nb(int Co) {
    const int b = Co / 16;
    for (int nb : {8, 6, 4, 3, 2}) if (b % nb == 0) return nb;
    return 1;
}

template <typename T>
static int conv_common(const ConvArgs& a, int Ci, int epilogue, hipStream_t s) {
    const int nb = pick_nb(a.Co);
    switch (epilogue) {
        case PMG_EPI_ACC: return launch_nb<T, PMG_EPI_ACC>(a, nb, s);
        case PMG_EPI_BIAS: return launch_nb<T, PMG_EPI_BIAS>(a, nb, s);
        case PMG_EPI_R: return launch_nb<T, PMG_EPI_R>(a, nb, s);
        case PMG_EPI_Q:
            if constexpr (sizeof(T) == 1) return launch_nb<T, PMG_EPI_Q>(a, nb, s);
            break;
        case PMG_EPI_SILU:
            if constexpr (sizeof(T) == 2) return launch_nb<T, PMG_EPI_SILU>(a, nb, s);
            break;
    }
    (void)Ci;
    return fail(PMG_E_INVALID, "spconv: epilogue not available for this precision");
}

static int validate(const void* x, const int32_t* nmap_t, const uint32_t* tile_mask, int64_t M, int Ci, int Co,
                    const void* w, void* out, int elt, const char* who) {
    if (!x || !nmap_t || !tile_mask || !w || !out)
        return fail(PMG_E_INVALID, std::string(who) + ": null buffer");
    if (M < 0 || M > INT32_MAX) return fail(PMG_E_INVALID, std::string(who) + ": bad voxel count");
    if (Co <= 0 || Co % 16 != 0 || Co > 4096) return fail(PMG_E_INVALID, std::string(who) + ": Co must be a multiple of 16");
    if (Ci <= 0 || (Ci * elt) % 16 != 0 || Ci > 4096)
        return fail(PMG_E_INVALID, std::string(who) + ": Ci*sizeof(elt) must be a multiple of 16 bytes");
    if (!aligned16(x) || !aligned16(w))
        return fail(PMG_E_INVALID, std::string(who) + ": x and w must be 16-byte aligned");
    return PMG_OK;
}

}  // namespace pmg

using namespace pmg;

extern "C" {

int pmg_spconv_i8(const int8_t* x, const int32_t* nmap_t, const uint32_t* tile_mask, int64_t M, int Ci, int Co,
                  const int8_t* w, int epilogue, float a_scale, const float* w_scale, const float* bias,
                  float out_mult, const float* skip, void* out, void* stream) {
    if (int e = validate(x, nmap_t, tile_mask, M, Ci, Co, w, out, 1, "pmg_spconv_i8")) return e;
    PMG_REQUIRE(epilogue == PMG_EPI_ACC || w_scale, "w_scale required");
    PMG_REQUIRE(epilogue != PMG_EPI_R || skip, "skip required");
    PMG_REQUIRE(epilogue != PMG_EPI_Q || out_mult > 0.0f, "out_mult must be positive");
    if (M == 0) return PMG_OK;
    ConvArgs a{(const uint8_t*)x, nmap_t, tile_mask, (const uint8_t*)w, M, Co, Ci, Ci / 16,
               a_scale, w_scale, bias, out_mult, skip, out};
    return conv_common<int8_t>(a, Ci, epilogue, (hipStream_t)stream);
}

int pmg_spconv_f16(const uint16_t* x, const int32_t* nmap_t, const uint32_t* tile_mask, int64_t M, int Ci, int Co,
                   const uint16_t* w, int epilogue, const float* bias, const float* skip, void* out, void* stream) {
    if (int e = validate(x, nmap_t, tile_mask, M, Ci, Co, w, out, 2, "pmg_spconv_f16")) return e;
    PMG_REQUIRE(epilogue != PMG_EPI_R || skip, "skip required");
    if (M == 0) return PMG_OK;
    ConvArgs a{(const uint8_t*)x, nmap_t, tile_mask, (const uint8_t*)w, M, Co, Ci * 2, Ci * 2 / 16,
               1.0f, nullptr, bias, 1.0f, skip, out};
    return conv_common<_Float16>(a, Ci, epilogue, (hipStream_t)stream);
}

int pmg_spconv_f32(const float* x, const int32_t* nmap_t, const uint32_t* tile_mask, int64_t M, int Ci, int Co,
                   const float* w, int epilogue, const float* bias, float* out, void* stream) {
    if (int e = validate(x, nmap_t, tile_mask, M, Ci, Co, w, out, 4, "pmg_spconv_f32")) return e;
    PMG_REQUIRE(epilogue == PMG_EPI_ACC || epilogue == PMG_EPI_BIAS, "fp32 supports ACC and BIAS epilogues");
    if (M == 0) return PMG_OK;
    ConvArgs a{(const uint8_t*)x, nmap_t, tile_mask, (const uint8_t*)w, M, Co, Ci * 4, Ci * 4 / 16,
               1.0f, nullptr, bias, 1.0f, nullptr, out};
    return conv_common<float>(a, Ci, epilogue, (hipStream_t)stream);
}

}  // extern "C"
