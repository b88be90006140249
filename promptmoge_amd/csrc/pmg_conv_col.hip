// Level-0 submanifold 3x3x3 convolution straight from the z-keys: the column-stencil map of
// _build_submanifold_nmap_column (_core.py:269-295) is never materialised.
//
// At level 0 every pixel is one voxel (MoGeModel._voxelize, v3.py:305-344), so the neighbour of voxel o at tap
// (di, dj, dz) is pixel o + di*W + dj when that pixel is in frame and its key equals key[o] + dz. A block owns a
// segment of SEG = 128 consecutive voxels (4 waves x 32 rows). Its neighbours all lie in three raster ranges
// [s0 + di*W - 1, s0 + di*W + SEG + 1), which are staged in LDS with coalesced 16-byte loads (the "window"), so each
// activation row is fetched from L2/HBM about three times per layer instead of once per (row, tap). The weights
// (Co, 27, Ci) stay resident in LDS for the whole persistent block when they fit.
//
// Matrix cores: D[n][m] = sum_k W[n][k] X[m][k] with v_mfma_*_16x16x* and the weights as the first operand, so a
// lane holds 4 consecutive output channels of one voxel (lane l: channels 16j + 4(l/16) + i, voxel l%16) and every
// epilogue stores 4-byte (int8) or 16-byte (fp32) vectors. The reduction runs over the wave's union of active taps
// (a 27-bit mask OR-ed over its 32 rows) x 16-byte channel chunks; the row's own tap validity zeroes the activation
// operand, so each row only accumulates its own neighbours.
//
// Epilogues (one pass over the output):
//   ACC    raw accumulator (int32 / fp32), for parity
//   Q      int8: quant(silu(acc*a_scale*w_scale + bias), out_scale);  fp16: half(silu(acc + bias))
//   R      x_new = dequant(acc) + skip                                   (fp32 residual stream)
//   RLN    R, stores x_new, then the next block's LayerNorm -> SiLU -> int8 codes (or fp16), so the residual block
//          needs no separate normalisation pass (flex_sparse_blocks.py:230-234)
//   ROUT   R, then out_proj (C -> 1) and logz += delta into the output point map (sparse_unet.py:258; v3.py:359)
// LayerNorm and out_proj sum in the "quad" order: lane group g sums its channels 16j+4g+i (j outer, i inner), then
// ((s0 + s1) + (s2 + s3)) across the four groups; every LayerNorm of the step uses that same order.
#include <climits>

#include "pmg_common.h"
#include "pmg_internal.h"

namespace pmg {

constexpr int kSeg = 128;
constexpr int kWin = kSeg + 2;

template <typename T>
struct ColAcc;
template <>
struct ColAcc<int8_t> {
    typedef v4i type;
};
template <>
struct ColAcc<_Float16> {
    typedef v4f type;
};

__device__ inline void mma_col(v4i& acc, const v4i& w, const v4i& x, int8_t) {
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(w, x, acc, 0, 0, 0);
}
__device__ inline void mma_col(v4f& acc, const v4i& w, const v4i& x, _Float16) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, w), __builtin_bit_cast(v8h, x), acc, 0, 0,
                                                  0);
}

// Sum over the four lane groups (lanes l, l^16, l^32, l^48) in the fixed order ((s0 + s1) + (s2 + s3)).
__device__ inline float quad_sum(float s) {
    const float a = s + __shfl_xor(s, 16, 64);
    return a + __shfl_xor(a, 32, 64);
}

template <typename T, int C, int EPI, bool WLDS>
__global__ __launch_bounds__(256) void spconv_col_k(ColConvArgs a) {
    constexpr int ROWB = C * (int)sizeof(T);  // bytes per activation row
    constexpr int NCH = ROWB / 16;            // 16-byte chunks per row
    constexpr int NB = C / 16;                // 16-channel output blocks
    typedef typename ColAcc<T>::type acc_t;

    __shared__ __attribute__((aligned(16))) uint8_t s_w[WLDS ? C * 27 * ROWB : 16];
    __shared__ __attribute__((aligned(16))) uint8_t s_x[3 * kWin * ROWB];
    __shared__ int8_t s_taps[4][32];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int64_t M = a.M;
    const int H = a.H, W = a.W;
    const int64_t HW = (int64_t)H * W;
    const uint8_t* __restrict__ xg = (const uint8_t*)a.x;
    const uint8_t* __restrict__ wg = (const uint8_t*)a.w;

    if constexpr (WLDS) {
        for (int e = tid; e < C * 27 * NCH; e += 256) ((v4i*)s_w)[e] = ((const v4i*)wg)[e];
    }

    const int64_t nseg = (M + kSeg - 1) / kSeg;
    for (int64_t seg = blockIdx.x; seg < nseg; seg += gridDim.x) {
        const int64_t s0 = seg * kSeg;
        __syncthreads();  // the previous segment's reads of the window are done (and the weights are staged)
        for (int e = tid; e < 3 * kWin * NCH; e += 256) {
            const int d = e / (kWin * NCH);
            const int rem = e - d * (kWin * NCH);
            const int q = rem / NCH, c = rem - (rem / NCH) * NCH;
            const int64_t p = s0 + (int64_t)(d - 1) * W - 1 + q;
            v4i val = {0, 0, 0, 0};
            if (p >= 0 && p < M) val = *(const v4i*)(xg + p * ROWB + c * 16);
            ((v4i*)s_x)[e] = val;
        }

        // 27-bit tap masks of the wave's 32 rows: lane l < 32 computes row l.
        uint32_t mk = 0;
        {
            const int lr = lane & 31;
            const int64_t m = s0 + 32 * wv + lr;
            if (lane < 32 && m < M) {
                const int64_t pix = m % HW;
                const int i = (int)(pix / W), j = (int)(pix - (pix / W) * W);
                const int zc = a.zq[m];
#pragma unroll
                for (int di = -1; di <= 1; ++di)
#pragma unroll
                    for (int dj = -1; dj <= 1; ++dj) {
                        const int ni = i + di, nj = j + dj;
                        if (ni >= 0 && ni < H && nj >= 0 && nj < W) {
                            const int64_t dz = (int64_t)a.zq[m + (int64_t)di * W + dj] - zc;
                            if (dz >= -1 && dz <= 1) mk |= 1u << ((di + 1) * 9 + (dj + 1) * 3 + (int)(dz + 1));
                        }
                    }
            }
        }
        uint32_t uni = mk;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) uni |= __shfl_xor(uni, o, 64);
        const uint32_t mrow0 = __shfl(mk, r, 64), mrow1 = __shfl(mk, 16 + r, 64);
        if (lane < 27 && ((uni >> lane) & 1u)) s_taps[wv][__popc(uni & ((1u << lane) - 1u))] = (int8_t)lane;
        __syncthreads();

        acc_t acc[2][NB];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int j = 0; j < NB; ++j) acc[rb][j] = acc_t{0, 0, 0, 0};

        const int Q = __popc(uni) * NCH;
        const int lr0 = 32 * wv + r;  // window-relative row of this lane in row block 0
        for (int q0 = 0; q0 < Q; q0 += 4) {
            const int q = q0 + g;
            v4i xa0 = {0, 0, 0, 0}, xa1 = {0, 0, 0, 0};
            v4i wb[NB];
            if (q < Q) {
                const int t = q / NCH, c = q - (q / NCH) * NCH;
                const int v = s_taps[wv][t];
                const int di = v / 9, dj = (v / 3) % 3;  // +1 offsets
                const int base = di * kWin + dj;          // window row of the neighbour of lr = 0
                if ((mrow0 >> v) & 1u) xa0 = *(const v4i*)(s_x + (base + lr0) * ROWB + c * 16);
                if ((mrow1 >> v) & 1u) xa1 = *(const v4i*)(s_x + (base + lr0 + 16) * ROWB + c * 16);
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const int off = ((16 * j + r) * 27 + v) * ROWB + c * 16;
                    if constexpr (WLDS)
                        wb[j] = *(const v4i*)(s_w + off);
                    else
                        wb[j] = *(const v4i*)(wg + off);
                }
            } else {
#pragma unroll
                for (int j = 0; j < NB; ++j) wb[j] = v4i{0, 0, 0, 0};
            }
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                mma_col(acc[0][j], wb[j], xa0, T{});
                mma_col(acc[1][j], wb[j], xa1, T{});
            }
        }

        // ---- epilogue: lane holds channels 16j + 4g + i of voxel m
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            const int64_t m = s0 + 32 * wv + 16 * rb + r;
            const bool ok = m < M;
            const int64_t mo = ok ? m : 0;
            float y[NB][4];
            if constexpr (EPI != PMG_EPI_ACC) {
#pragma unroll
                for (int j = 0; j < NB; ++j)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int n = 16 * j + 4 * g + i;
                        if constexpr (sizeof(T) == 1) {
                            float t = (float)acc[rb][j][i] * a.a_scale;
                            t = t * a.w_scale[n];
                            if (a.bias) t = t + a.bias[n];
                            y[j][i] = t;
                        } else {
                            float t = acc[rb][j][i];
                            if (a.bias) t = t + a.bias[n];
                            y[j][i] = t;
                        }
                    }
            }
            if constexpr (EPI == PMG_EPI_ACC) {
                if (ok) {
#pragma unroll
                    for (int j = 0; j < NB; ++j) {
                        const int64_t o = mo * C + 16 * j + 4 * g;
                        if constexpr (sizeof(T) == 1)
                            *(v4i*)((int32_t*)a.out + o) = acc[rb][j];
                        else
                            *(v4f*)((float*)a.out + o) = acc[rb][j];
                    }
                }
            } else if constexpr (EPI == PMG_EPI_Q) {
                if (ok) {
#pragma unroll
                    for (int j = 0; j < NB; ++j) {
                        const int64_t o = mo * C + 16 * j + 4 * g;
                        if constexpr (sizeof(T) == 1) {
                            uint32_t pk = 0;
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                pk |= (uint32_t)(uint8_t)quant_i8(silu_f32(y[j][i]), a.out_scale) << (8 * i);
                            *(uint32_t*)((int8_t*)a.out + o) = pk;
                        } else {
                            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                            h4 hv;
#pragma unroll
                            for (int i = 0; i < 4; ++i) hv[i] = (_Float16)silu_f32(y[j][i]);
                            *(h4*)((_Float16*)a.out + o) = hv;
                        }
                    }
                }
            } else {
                // residual: x_new = y + skip
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const int64_t o = mo * C + 16 * j + 4 * g;
                    const v4f sk = *(const v4f*)(a.skip + o);
#pragma unroll
                    for (int i = 0; i < 4; ++i) y[j][i] = y[j][i] + sk[i];
                    if (EPI != PMG_EPI_ROUT && ok) *(v4f*)((float*)a.out + o) = v4f{y[j][0], y[j][1], y[j][2], y[j][3]};
                }
                if constexpr (EPI == PMG_EPI_RLN) {
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
                    const float rstd = 1.0f / __builtin_sqrtf(var + a.ln_eps);
                    if (ok) {
#pragma unroll
                        for (int j = 0; j < NB; ++j) {
                            float h[4];
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const int n = 16 * j + 4 * g + i;
                                float t = (y[j][i] - mean) * rstd;
                                t = t * a.ln_gamma[n];
                                t = t + a.ln_beta[n];
                                h[i] = silu_f32(t);
                            }
                            const int64_t o = mo * C + 16 * j + 4 * g;
                            if constexpr (sizeof(T) == 1) {
                                uint32_t pk = 0;
#pragma unroll
                                for (int i = 0; i < 4; ++i)
                                    pk |= (uint32_t)(uint8_t)quant_i8(h[i], a.next_scale) << (8 * i);
                                *(uint32_t*)((int8_t*)a.next_q + o) = pk;
                            } else {
                                typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                                h4 hv;
#pragma unroll
                                for (int i = 0; i < 4; ++i) hv[i] = (_Float16)h[i];
                                *(h4*)((_Float16*)a.next_q + o) = hv;
                            }
                        }
                    }
                } else if constexpr (EPI == PMG_EPI_ROUT) {
                    float p = 0.0f;
#pragma unroll
                    for (int j = 0; j < NB; ++j)
#pragma unroll
                        for (int i = 0; i < 4; ++i) p = p + a.out_w[16 * j + 4 * g + i] * y[j][i];
                    const float d = a.out_b[0] + quad_sum(p);
                    if (ok && g == 0) {
                        const float p0 = a.points[mo * 3 + 0], p1 = a.points[mo * 3 + 1], p2 = a.points[mo * 3 + 2];
                        a.points_out[mo * 3 + 0] = p0;
                        a.points_out[mo * 3 + 1] = p1;
                        a.points_out[mo * 3 + 2] = p2 + d;
                    }
                }
            }
        }
    }
}

template <typename T, int C, int EPI>
static int launch_col3(const ColConvArgs& a, hipStream_t s) {
    constexpr size_t wbytes = (size_t)C * 27 * C * sizeof(T);
    constexpr bool WLDS = wbytes <= 64 * 1024;
    const int64_t nseg = (a.M + kSeg - 1) / kSeg;
    static int per_cu = -1;
    if (per_cu < 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, spconv_col_k<T, C, EPI, WLDS>, 256, 0) != hipSuccess ||
            n < 1)
            n = 1;
        per_cu = n;
    }
    int64_t grid = (int64_t)per_cu * num_cus();
    if (grid > nseg) grid = nseg;
    hipLaunchKernelGGL((spconv_col_k<T, C, EPI, WLDS>), dim3((unsigned)grid), dim3(256), 0, s, a);
    return check_launch("spconv_col_k");
}

template <typename T, int C>
static int launch_col2(const ColConvArgs& a, int epi, hipStream_t s) {
    switch (epi) {
        case PMG_EPI_ACC: return launch_col3<T, C, PMG_EPI_ACC>(a, s);
        case PMG_EPI_Q: return launch_col3<T, C, PMG_EPI_Q>(a, s);
        case PMG_EPI_R: return launch_col3<T, C, PMG_EPI_R>(a, s);
        case PMG_EPI_RLN: return launch_col3<T, C, PMG_EPI_RLN>(a, s);
        case PMG_EPI_ROUT: return launch_col3<T, C, PMG_EPI_ROUT>(a, s);
    }
    return fail(PMG_E_INVALID, "pmg_spconv_col: unknown epilogue");
}

int launch_conv_col(int precision, const ColConvArgs& a, int C, int epi, hipStream_t s) {
    if (precision == PMG_PREC_INT8) {
        switch (C) {
            case 16: return launch_col2<int8_t, 16>(a, epi, s);
            case 32: return launch_col2<int8_t, 32>(a, epi, s);
            case 48: return launch_col2<int8_t, 48>(a, epi, s);
            case 64: return launch_col2<int8_t, 64>(a, epi, s);
            case 128: return launch_col2<int8_t, 128>(a, epi, s);
        }
    } else {
        switch (C) {
            case 16: return launch_col2<_Float16, 16>(a, epi, s);
            case 32: return launch_col2<_Float16, 32>(a, epi, s);
            case 48: return launch_col2<_Float16, 48>(a, epi, s);
            case 64: return launch_col2<_Float16, 64>(a, epi, s);
            case 128: return launch_col2<_Float16, 128>(a, epi, s);
        }
    }
    return fail(PMG_E_INVALID, "pmg_spconv_col: C must be 16, 32, 48, 64 or 128");
}

}  // namespace pmg

using namespace pmg;

extern "C" int pmg_spconv_col(int precision, const void* x, const int32_t* zq, int B, int H, int W, int C,
                              const void* w, int epilogue, const pmg_conv_epilogue* e, void* stream) {
    PMG_REQUIRE(x && zq && w && e && e->out || (e && epilogue == PMG_EPI_ROUT && x && zq && w), "null buffer");
    PMG_REQUIRE(precision == PMG_PREC_INT8 || precision == PMG_PREC_FP16, "bad precision");
    PMG_REQUIRE(B > 0 && H > 0 && W > 0, "bad shape");
    const int64_t M = (int64_t)B * H * W;
    PMG_REQUIRE(M <= INT_MAX, "too many voxels");
    PMG_REQUIRE(aligned16(x) && aligned16(w), "x and w must be 16-byte aligned");
    const bool i8 = precision == PMG_PREC_INT8;
    PMG_REQUIRE(!i8 || epilogue == PMG_EPI_ACC || e->w_scale, "int8 needs w_scale");
    PMG_REQUIRE(epilogue != PMG_EPI_Q || !i8 || e->out_scale > 0.0f, "out_scale must be positive");
    const bool res = epilogue == PMG_EPI_R || epilogue == PMG_EPI_RLN || epilogue == PMG_EPI_ROUT;
    PMG_REQUIRE(!res || (e->skip && aligned16(e->skip)), "residual epilogues need a 16-byte aligned skip");
    PMG_REQUIRE(epilogue == PMG_EPI_ROUT || aligned16(e->out), "out must be 16-byte aligned");
    PMG_REQUIRE(epilogue != PMG_EPI_RLN || (e->ln_gamma && e->ln_beta && e->next_q && (!i8 || e->next_scale > 0.0f)),
                "RLN needs LayerNorm parameters and next_q");
    PMG_REQUIRE(epilogue != PMG_EPI_ROUT || (e->out_w && e->out_b && e->points && e->points_out),
                "ROUT needs out_proj weights and the point maps");
    ColConvArgs a{};
    a.x = x;
    a.zq = zq;
    a.w = w;
    a.M = M;
    a.H = H;
    a.W = W;
    a.a_scale = i8 ? e->a_scale : 1.0f;
    a.w_scale = e->w_scale;
    a.bias = e->bias;
    a.out_scale = e->out_scale;
    a.skip = e->skip;
    a.out = e->out;
    a.ln_gamma = e->ln_gamma;
    a.ln_beta = e->ln_beta;
    a.ln_eps = e->ln_eps;
    a.next_scale = e->next_scale;
    a.next_q = e->next_q;
    a.out_w = e->out_w;
    a.out_b = e->out_b;
    a.points = e->points;
    a.points_out = e->points_out;
    return launch_conv_col(precision, a, C, epilogue, (hipStream_t)stream);
}
