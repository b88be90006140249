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
#include <type_traits>

#include "pmg_common.h"
#include "pmg_internal.h"

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
    const int32_t* order;  // output row of each processing position, or NULL for 0 .. M-1; the map's columns and
                           // the tile masks are in processing order
    const int64_t* m_dev;  // spconv_k: the row count on the device (<= M, which is then the map's row stride and
                           // the grid's capacity), or NULL for M rows
    int32_t* part;         // device-sized spconv_g2_k: int32 partial sums of a tap split ([Z][rows][Co]), or NULL
};

// Tap split of the device-sized weight-staged convolution: when a level has few chunks (a coarse U-Net level of a
// few thousand rows keeps a handful of CUs busy for 27 dependent taps), each (chunk, range of taps) is a unit of
// its own and stores exact int32 partial sums; split_epilogue_k, the next launch on the stream, adds them in order
// and applies the epilogue. (Finishing in the last unit to arrive instead needs an agent-scope release per unit,
// an L2 write-back on CDNA: measured slower than the second launch.) The factor follows from the row count on the
// device: as many units as fit one round of blocks.
constexpr int kSplitUnits = 256;  // units aimed at (chunks x output slices x Z): one block per CU of MI355X
constexpr int kSplitMax = 9;
__host__ __device__ inline int split_factor(int nchunk, int nslice) {
    const int cs = nchunk * nslice;
    const int z = cs > 0 ? kSplitUnits / cs : 1;
    return z < 1 ? 1 : (z > kSplitMax ? kSplitMax : z);
}

// Row m, output channels c .. c+3 of a tap-split launch: the Z partial sums added in order (int32: exact, the
// unsplit accumulator) and the epilogue of the device-sized convolution in the same arithmetic.
template <int EPI>
__device__ inline void split_finish(const ConvArgs& a, int Z, int M, int64_t m, int c) {
    const int Co = a.Co;
    v4i acc = *(const v4i*)(a.part + m * Co + c);
    for (int z = 1; z < Z; ++z) acc += *(const v4i*)(a.part + ((int64_t)z * M + m) * Co + c);
    const int64_t o = m * Co + c;
    if constexpr (EPI == PMG_EPI_ACC) {
        *(v4i*)((int32_t*)a.out + o) = acc;
    } else {
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float u = (float)acc[i] * a.a_scale;
            u = u * a.w_scale[c + i];
            if (a.bias) u = u + a.bias[c + i];
            y[i] = u;
        }
        if constexpr (EPI == PMG_EPI_Q) {
            store_silu_codes4(y, a.out_mult, (int8_t*)a.out + o);
        } else if constexpr (EPI == PMG_EPI_QLIN) {
            store_codes4(y, a.out_mult, (int8_t*)a.out + o);
        } else if constexpr (EPI == PMG_EPI_R) {
            const v4f sk = *(const v4f*)(a.skip + o);
            *(v4f*)((float*)a.out + o) = v4f{y[0] + sk[0], y[1] + sk[1], y[2] + sk[2], y[3] + sk[3]};
        } else {
            *(v4f*)((float*)a.out + o) = v4f{y[0], y[1], y[2], y[3]};
        }
    }
}

// The second launch of a tap split: the row count and Z read again on the device exactly as spconv_g2_k reads
// them (CHUNK rows per chunk, nslice output slices); nothing to do when that launch did not split.
template <int EPI, int CHUNK>
__global__ __launch_bounds__(256) void split_epilogue_k(ConvArgs a, int nslice) {
    const int M = (int)*a.m_dev;
    const int Z = split_factor((M + CHUNK - 1) / CHUNK, nslice);
    if (Z < 2) return;
    const int Q4 = a.Co / 4;
    const int64_t total = (int64_t)M * Q4;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < total; e += (int64_t)gridDim.x * 256) {
        const int64_t m = e / Q4;
        split_finish<EPI>(a, Z, M, m, 4 * (int)(e - m * Q4));
    }
}

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
template <>
struct Acc<__bf16> {
    typedef v4f type;
};

__device__ inline void mma(v4i& acc, const v4i& a, const v4i& b, int8_t) {
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
}
__device__ inline void mma(v4f& acc, const v4i& a, const v4i& b, _Float16) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), acc, 0,
                                                  0, 0);
}
__device__ inline void mma(v4f& acc, const v4i& a, const v4i& b, __bf16) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), acc, 0,
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
            } else if constexpr (EPI == PMG_EPI_QLIN) {
                ((int8_t*)a.out)[o] = quant_i8(y, a.out_mult);
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
            ((_Float16*)a.out)[o] = (_Float16)silu_fast(y);
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
    const int64_t Mr = a.m_dev ? *a.m_dev : a.M;  // rows; a.M is the map's row stride
    if ((int64_t)blockIdx.x * 64 >= Mr) return;   // the whole block lies beyond the rows (device-sized grids)
    const int64_t ntile = (Mr + 15) >> 4;
    const uint32_t mask = tile < ntile ? a.tmask[tile] : 0u;
    if (lane < 27 && ((mask >> lane) & 1u)) taps_s[wv][__popc(mask & ((1u << lane) - 1u))] = (int8_t)lane;
    __syncthreads();

    const int Q = __popc(mask) * a.nchunk;
    const int r = lane & 15, g = lane >> 4;
    const int64_t m0 = tile * 16;
    const int64_t row = m0 + r;
    const bool row_ok = row < Mr;
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
            if (idx >= 0 && idx < Mr) av = *(const v4i*)(a.x + (int64_t)idx * a.row_bytes + c * 16);
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
            if (m < Mr) epilogue<T, EPI>(a, m, n, acc[j], i);
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

// ---------------------------------------------------------------------------------------------------------------
// int8, Ci = Co = C in {64, 128}: block-tiled, weight-staged variant for large maps (the 1M-voxel microbench).
//
// A persistent 8-wave block owns chunks of 512 output rows (64 rows per wave in four 16-row tiles) and all C output
// channels. The taps' C x C weights pass through LDS in MFMA operand order (one 1 KB block per 16 output channels
// and 64-wide K step: conflict-free 16-byte reads), a group of taps at a time, double-buffered. Every wave gathers
// its rows' neighbour codes x[nmap[v][m]] straight from global memory into registers one tap ahead, and the map
// indices three taps ahead. Each LDS weight read feeds four tiles, each gathered chunk NB column blocks. Operands
// are swapped (D = W * X^T): a lane ends with 4 consecutive output channels of one row and the epilogue stores
// vectors. Chunks are assigned so that the blocks of one XCD (block b runs on XCD b % 8) process adjacent row
// ranges and share their neighbours in L2.
//
// Every global load of the tap loop is issued unconditionally and none goes straight to LDS, so the compiler's
// vmcnt waits name exactly the load they need: an MFMA waits for its own tap's codes, not for the loads issued
// after them (an LDS-DMA weight load made every weight read wait for all outstanding loads, and a branch around a
// gather made the waits at the join conservative). Counters show the kernel limited by the L1 path of the gathers
// (texture data unit busy 75 % at C = 128, most of it waiting on the cache; each 512-row chunk gathers ~27 times
// its own rows), not by the gather latency: a three-tap-deep gather ring at C = 64 was no faster.
// Code epilogues (Q: SiLU requant, QLIN: linear requant) of a wave's T tiles of 16 rows x 16 NB channels: the
// dequantised accumulators (a_scale, per-channel scale and bias from LDS) packed into words of 4 codes, regrouped
// between the lanes of each row (lane_groups_transpose4) and stored as one 16-byte vector per lane and 64-channel
// block. Rows at or beyond M compute but do not store (the transpose needs every lane of the wave).
template <int EPI, int T, int NB>
__device__ inline void store_tile_codes(const ConvArgs& a, const v4i (&acc)[T][NB], const float* s_scale,
                                        const float* s_bias, const int (&orow)[T], int pos0, int M, int Co, int n0,
                                        int g) {
    static_assert(NB % 4 == 0, "64-channel blocks");
#pragma unroll
    for (int t = 0; t < T; ++t) {
        uint32_t w[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            float y[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int n = 16 * j + 4 * g + i;
                float u = (float)acc[t][j][i] * a.a_scale;
                u = u * s_scale[n];
                if (a.bias) u = u + s_bias[n];
                y[i] = u;
            }
            w[j] = EPI == PMG_EPI_Q ? pack_silu_codes4(y, a.out_mult) : pack_codes4(y, a.out_mult);
        }
#pragma unroll
        for (int h = 0; h < NB / 4; ++h) {
            uint32_t q[4] = {w[4 * h], w[4 * h + 1], w[4 * h + 2], w[4 * h + 3]};
            lane_groups_transpose4(q);
            if (pos0 + 16 * t < M)
                *(v4i*)((int8_t*)a.out + (int64_t)orow[t] * Co + n0 + 64 * h + 16 * g) =
                    v4i{(int)q[0], (int)q[1], (int)q[2], (int)q[3]};
        }
    }
}

// Host-sized generic-map launches deal groups of kXcdGroup consecutive chunks round-robin over the 8 XCDs (block b
// runs on XCD b % 8): neighbouring chunks (rows that share neighbours) stay on one XCD's L2, and the work evens out
// where it varies along the row order (rows sorted by tap mask; measured at C = 128 on the 1M-voxel surface set:
// 0.369 ms with one contiguous band per XCD, 0.324 ms dealt in groups of 16). Launches with fewer than 8 groups of
// chunks (every device-sized launch of a coarse level, small host-sized sets) keep one contiguous band per XCD:
// groups would put all of the work on the first XCDs (21 chunks: 16 on XCD 0, 5 on XCD 1, the other six idle).
constexpr int kXcdGroup = 16;
__host__ __device__ inline int xcd_group(int64_t nunits) { return nunits >= 8 * kXcdGroup ? kXcdGroup : 0; }

constexpr int kBufWord3 = 0x00020000;  // buffer descriptor word 3 for raw (untyped) loads on gfx9
constexpr int kG2Threads = 512;       // 8 waves: two per SIMD, 256 registers each
constexpr int kG2Waves = kG2Threads / 64;
constexpr int kG2Tiles = 4;           // 16-row tiles per wave
constexpr int kG2Chunk = kG2Waves * kG2Tiles * 16;  // 512 rows per block step

// Generic-map int8 convolution for Ci = Co = C in {64, 128} (C = 64 launches spconv_g2r_k below instead): a
// persistent block per CU walks chunks of 512 output rows (in `order` if given); each of its 8 waves owns 64 rows
// (4 tiles of 16) with 4 x C/16 int32 accumulator tiles. The 27 taps run in fixed order in groups of GRP taps (4 at
// C = 64, 2 at C = 128: registers); the next
// group's weights are loaded into registers during this group and stored into the other LDS buffer, so the block
// meets at one barrier per group. Each LDS weight operand feeds the wave's 4 tiles (4 MFMAs of 16 cycles) and the
// next operand is read before they issue. A wave skips the MFMAs of taps none of its 4 tiles has; an absent
// neighbour (index -1), and every index of such a tap, becomes an out-of-range buffer offset, which loads zeros.
//
// NB < C / 16 splits the output channels into slices of 16 NB, one per blockIdx.y (Co = 256: 8 column blocks of 16
// at a time, which is what fits the registers), and T sets the rows per wave (16 T; chunks of 128 T rows). With
// a.m_dev the row count is read on the device: a.M is then the capacity, the row stride of the map. PF = how many
// weight operands ahead a wave reads from LDS; RS = 4 gathers codes three taps ahead instead of one and requests
// a group's weights a whole group ahead (a few hundred rows per block, as on the coarse levels of a U-Net, leave
// each tap waiting on both otherwise).
template <int C, int EPI, int NB = C / 16, int T = kG2Tiles, int PF = 1, int RS = 2, bool DEV = (RS == 4),
          typename E = int8_t>
__global__ __launch_bounds__(kG2Threads, 1) void spconv_g2_k(ConvArgs a) {
    constexpr int RB = C * (int)sizeof(E);               // row bytes: the kernel moves 64-byte K chunks of any type
    // taps per LDS buffer: GRP taps of NF 1 KB fragments each, two buffers within the LDS
    constexpr int GRP = RB == 64 ? 4 : (RB * NB <= 2048 ? 2 : 1);
    constexpr int KS = RB / 64;
    constexpr int NF = NB * KS;                          // 1 KB operand fragments per tap
    constexpr int WPT = GRP * NF / kG2Waves;             // fragments staged per wave per group
    constexpr int NG = (27 + GRP - 1) / GRP;             // tap groups; taps >= 27 of the last one are empty
    constexpr int NG2 = (NG + 1) / 2;                    // loop trips of two groups (one per LDS buffer)
    constexpr int CHUNK = kG2Waves * T * 16;             // rows per block step
    constexpr int NS = 16 * NB;                          // output channels of the block
    static_assert(RB == 64 || RB == 128 || RB == 256 || RB == 512 || RB == 1024, "rows of 64 .. 1024 bytes");
    static_assert(2 * GRP * NB * (RB / 64) <= 128, "two LDS buffers of GRP taps' weights");
    static_assert(sizeof(E) == 1 || !DEV, "device-sized launches are int8");
    typedef typename Acc<E>::type acc_t;
    static_assert(GRP * NF % kG2Waves == 0, "staging split");
    static_assert(T == 1 || T == 2 || T == 4, "tiles per wave");
    static_assert(RS == 2 || RS == 4, "ring slots: the tap parity or v mod 4 of a trip");
    constexpr int GD = RS - 1;                           // gather distance in taps
    constexpr bool kDev = DEV;                           // the device-sized launch (tap split allowed)

    __shared__ __attribute__((aligned(16))) v4i s_w[2][GRP * NF * 64];
    __shared__ float s_k[2][NS];
    __shared__ uint32_t s_um[kG2Waves];  // each wave's tap mask, for the chunk's union

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int S = (int)a.M;                               // map row stride (the capacity)
    const int M = a.m_dev ? (int)*a.m_dev : S;            // rows
    const int64_t ntile = (M + 15) >> 4;
    const int Co = NS == C ? C : a.Co;
    const int n0 = NS == C ? 0 : (int)blockIdx.y * NS;    // first output channel of the block
    typedef const __attribute__((address_space(3))) v4i lds_v4i;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)(a.M * RB), kBufWord3);
    const __amdgpu_buffer_rsrc_t nr =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.nmap_t, (short)0, (int)(a.M * 27 * 4), kBufWord3);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, Co * 27 * RB, kBufWord3);

    for (int e = tid; e < 2 * NS; e += kG2Threads) {
        const int q = e / NS, n = e - (e / NS) * NS;
        const float* src = q == 0 ? a.w_scale : a.bias;
        s_k[q][n] = src ? src[n0 + n] : 0.0f;
    }

    const int nchunk = (M + CHUNK - 1) / CHUNK;
    // units: (chunk, z) with z the z-th of Z ranges of taps; Z = 1 (a unit is a chunk, all 27 taps) unless this is
    // a device-sized launch with a partials buffer and few chunks
    const int Z = kDev && a.part ? split_factor(nchunk, (int)gridDim.y) : 1;
    const int nunit = nchunk * Z;
    const int G = gridDim.x, b = blockIdx.x;
    const int nx = G >= 8 ? 8 : 1;
    const int x = b % nx, bi = b / nx, nbx = (G - x + nx - 1) / nx;
    const int c0 = (int)((int64_t)nunit * x / nx), c1 = (int)((int64_t)nunit * (x + 1) / nx);
    int t0 = 0, t1 = 27;  // the unit's taps [t0, t1)

    // Weights of group grp through registers into LDS (no LDS DMA: the compiler then keeps exact vmcnt waits for
    // the gathers). Fragment f = wv + 8k of the group is tap slot q = f / NF, operand js = f % NF = (j, s), and
    // lane l holds W[16j + (l & 15)][v][64s + 16(l >> 4) .. +16] of the [Co][27][Ci] tensor; taps >= t1 load
    // zeros (out-of-range buffer offset).
    const int wlane = ((n0 + r) * 27) * RB + 16 * g;
    // staged in PARTS pieces of WPP fragments per wave, one piece per tap of the group where that divides evenly
    // (C = 128: 8 registers held for one tap instead of 16 for the whole group)
    constexpr int PARTS = WPT % GRP == 0 ? GRP : 1, WPP = WPT / PARTS;
    // Union walk: the block runs only the taps that some row of its chunk has, in ascending order (a map in
    // mask-sorted row order leaves ~12 of 27 per 512-row chunk). Each tap slot of a group is then one staging
    // part, and three scalar cursors pop the union's taps for the weight loads, the index loads and the MFMAs.
    constexpr bool UW = !kDev && PARTS == GRP;
    // With the union walk (UW) a part is one tap slot and `vt` names its tap (27: none, zeros).
    auto w_load = [&](int grp, int part, v4i (&st)[WPP], int vt) {
#pragma unroll
        for (int kk = 0; kk < WPP; ++kk) {
            const int f = wv + kG2Waves * (part * WPP + kk);
            const int q = f / NF, js = f - (f / NF) * NF;
            const int j = js / KS, s2 = js - (js / KS) * KS;
            const int v = UW ? vt : t0 + GRP * grp + q;
            const int off = v < t1 ? wlane + ((16 * j * 27) + v) * RB + 64 * s2 : (int)0x80000000;
            st[kk] = __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, 0);
        }
    };
    auto w_store = [&](v4i* dst, int part, const v4i (&st)[WPP]) {
#pragma unroll
        for (int kk = 0; kk < WPP; ++kk) dst[(wv + kG2Waves * (part * WPP + kk)) * 64 + lane] = st[kk];
    };

    const int gi = kDev ? 0 : xcd_group(nunit);
    for (int kq = bi;; kq += nbx) {
        const int un = gi ? ((kq / gi) * nx + x) * gi + kq % gi : c0 + kq;
        if (un >= (gi ? nunit : c1)) break;
        const int ch = Z == 1 ? un : un / Z, z = un - ch * Z;
        if constexpr (kDev) {
            t0 = 27 * z / Z;
            t1 = 27 * (z + 1) / Z;
        }
        int trips = kDev ? (t1 - t0 + 3) / 4 : NG2;  // trips of 4 taps (two groups)
        const int pos0 = ch * CHUNK + wv * (16 * T) + r;
        // map column of each tile's row (a map in processing order) and the row its outputs go to; rows beyond M
        // get an out-of-range map offset (their indices load as 0)
        int roff[T], orow[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int p = pos0 + 16 * t;
            roff[t] = p < M ? 4 * p : (int)0x80000000;
            orow[t] = p < M && a.order ? a.order[p] : p;
        }
        uint32_t wmask;
        {
            const int64_t tl = (int64_t)ch * (CHUNK / 16) + wv * T + (lane & (T - 1));
            uint32_t mk = (lane < T && tl < ntile) ? a.tmask[tl] : 0u;
#pragma unroll
            for (int o = 1; o < T; o <<= 1) mk |= __shfl_xor(mk, o, 64);
            wmask = (uint32_t)__builtin_amdgcn_readfirstlane((int)mk);
        }
        // the chunk's tap union: every wave publishes its mask; the previous chunk's readers have all passed at
        // least one group barrier since (trips >= 1)
        uint32_t cw = 0, ci = 0, cm = 0;  // cursors: weight loads, index loads, MFMAs
        if constexpr (UW) {
            if (lane == 0) s_um[wv] = wmask;
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_s_barrier();
            uint32_t um = 0;
#pragma unroll
            for (int k = 0; k < kG2Waves; ++k) um |= s_um[k];
            um = (uint32_t)__builtin_amdgcn_readfirstlane((int)um);
            const int ntap = __builtin_popcount(um);
            trips = ntap > 0 ? (ntap + 2 * GRP - 1) / (2 * GRP) : 1;  // two groups of GRP taps per trip
            cw = ci = cm = um;
        }
        auto pop = [](uint32_t& rem) {
            const int v = rem ? (int)__builtin_ctz(rem) : 27;
            rem = rem ? rem & (rem - 1) : 0u;
            return v;
        };
        acc_t acc[T][NB];
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int j = 0; j < NB; ++j) acc[t][j] = acc_t{0, 0, 0, 0};

        // map indices of tap v (taps >= t1: out-of-range, zeros); gathers of the rows they name (absent: zeros).
        // Every load is issued unconditionally, so the compiler's vmcnt waits stay exact.
        auto idx_load = [&](int v, int (&id)[T]) {
            const int vo = (v < t1 ? v : 27) * S * 4;
#pragma unroll
            for (int t = 0; t < T; ++t) id[t] = __builtin_amdgcn_raw_buffer_load_b32(nr, roff[t], vo, 0);
        };
        auto gather = [&](const int (&id)[T], v4i (&xs)[T][KS]) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int off = id[t] >= 0 ? id[t] * RB + 16 * g : (int)0x80000000;
#pragma unroll
                for (int s2 = 0; s2 < KS; ++s2) xs[t][s2] = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 64 * s2, 0);
            }
        };
        // operand q of the tap is (s2, j) = (q / NB, q % NB), read PF operands ahead of its MFMAs
        auto mma_tap = [&](const v4i* wslot, const v4i (&xs)[T][KS]) {
            const v4i* wb = wslot + lane;
            v4i wop[PF];
#pragma unroll
            for (int k = 0; k < PF; ++k) wop[k] = *(lds_v4i*)(wb + ((k % NB) * KS + k / NB) * 64);
#pragma unroll
            for (int q = 0; q < NF; ++q) {
                const int s2 = q / NB, j = q - (q / NB) * NB;
                const v4i cur = wop[q % PF];
                if (q + PF < NF) {
                    const int s3 = (q + PF) / NB, j3 = (q + PF) - ((q + PF) / NB) * NB;
                    wop[q % PF] = *(lds_v4i*)(wb + (j3 * KS + s3) * 64);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int t = 0; t < T; ++t)
                    mma(acc[t][j], cur, xs[t][s2], E{});
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        // Rings of RS slots (tap u in slot u mod RS): the codes of tap u are gathered GD = RS - 1 taps ahead of its
        // MFMAs and its map indices two taps before that; an index slot is reloaded once its gather has read it.
        int I[RS][T];
        v4i X[RS][T][KS];
#pragma unroll
        for (int part = 0; part < PARTS; ++part) {
            v4i st[WPP];
            w_load(0, part, st, UW ? pop(cw) : 0);
            w_store(s_w[0], part, st);
        }
        if constexpr (RS == 2) {
            int i0[T];
            idx_load(UW ? pop(ci) : 0, i0);
            idx_load(UW ? pop(ci) : 1, I[1]);
            idx_load(UW ? pop(ci) : 2, I[0]);
            gather(i0, X[0]);
        } else {
#pragma unroll
            for (int u = 0; u < RS; ++u) idx_load(UW ? pop(ci) : t0 + u, I[u]);
#pragma unroll
            for (int u = 0; u < GD; ++u) gather(I[u], X[u]);
            idx_load(UW ? pop(ci) : t0 + RS, I[0]);
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's weight stores are in LDS
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);

        // One group: weights of the next group are loaded at its start and stored into the other buffer at its end
        // (every wave left that buffer at the last barrier); per tap v, the codes of tap v+GD and the indices of
        // tap v+GD+2 are requested before tap v's MFMAs. H = the buffer (group parity), compile-time, so the X and
        // I ring slots are too.
        auto group = [&](auto Hc, int grp) {
            constexpr int H = decltype(Hc)::value;
            v4i sta[RS == 2 ? 1 : PARTS][WPP];  // RS = 4: the next group's weights, all requested at its start
#pragma unroll
            for (int q = 0; q < GRP; ++q) {
                const int v = UW ? pop(cm) : t0 + GRP * grp + q;
                const int p = (GRP * H + q) & 3;  // (v - t0) mod 4 (GRP * grp = 4 * trip + GRP * H)
                v4i st[WPP];
                if constexpr (RS == 2) {
                    if (q < PARTS) w_load(grp + 1, q, st, UW ? pop(cw) : 0);
                } else if (q == 0) {
#pragma unroll
                    for (int pp = 0; pp < PARTS; ++pp) w_load(grp + 1, pp, sta[pp], UW ? pop(cw) : 0);
                }
                gather(I[(p + GD) % RS], X[(p + GD) % RS]);
                idx_load(UW ? pop(ci) : v + GD + 2, I[(p + GD + 2) % RS]);
                __builtin_amdgcn_sched_barrier(0);
                if (v < t1 && ((wmask >> v) & 1u)) mma_tap(s_w[H] + q * NF * 64, X[p % RS]);
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (RS == 2) {
                    if (q < PARTS) w_store(s_w[H ^ 1], q, st);
                } else if (q == GRP - 1) {
#pragma unroll
                    for (int pp = 0; pp < PARTS; ++pp) w_store(s_w[H ^ 1], pp, sta[pp]);
                }
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
        };
#pragma unroll 1
        for (int it = 0; it < trips; ++it) {
            group(std::integral_constant<int, 0>{}, 2 * it);
            group(std::integral_constant<int, 1>{}, 2 * it + 1);
        }

        if constexpr (kDev) {
            if (Z > 1) {  // a tap range: the exact partial sums, [Z][M][Co]
#pragma unroll
            for (int t = 0; t < T; ++t) {
                if (pos0 + 16 * t >= M) continue;
                const int m = orow[t];
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    *(v4i*)(a.part + ((int64_t)z * M + m) * Co + n0 + 16 * j + 4 * g) = acc[t][j];
            }
            continue;  // split_epilogue_k adds the Z partials and applies the epilogue
            }
        }
        if constexpr (sizeof(E) != 1) {  // fp16 / fp32 features: fp32 accumulators, bias from LDS
#pragma unroll
            for (int t = 0; t < T; ++t) {
                if (pos0 + 16 * t >= M) continue;
                const int m = orow[t];
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const int64_t o = (int64_t)m * Co + n0 + 16 * j + 4 * g;
                    float y[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        y[i] = acc[t][j][i];
                        if constexpr (EPI != PMG_EPI_ACC) {
                            if (a.bias) y[i] = y[i] + s_k[1][16 * j + 4 * g + i];
                        }
                    }
                    if constexpr (EPI == PMG_EPI_SILU) {
                        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                        h4 hv;
#pragma unroll
                        for (int i = 0; i < 4; ++i) hv[i] = (_Float16)silu_fast(y[i]);
                        *(h4*)((_Float16*)a.out + o) = hv;
                    } else if constexpr (EPI == PMG_EPI_R) {
                        const v4f sk = *(const v4f*)(a.skip + o);
                        *(v4f*)((float*)a.out + o) = v4f{y[0] + sk[0], y[1] + sk[1], y[2] + sk[2], y[3] + sk[3]};
                    } else {
                        *(v4f*)((float*)a.out + o) = v4f{y[0], y[1], y[2], y[3]};
                    }
                }
            }
        } else if constexpr (EPI == PMG_EPI_Q || EPI == PMG_EPI_QLIN) {
            store_tile_codes<EPI, T, NB>(a, acc, s_k[0], s_k[1], orow, pos0, M, Co, n0, g);
        } else {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                if (pos0 + 16 * t >= M) continue;
                const int m = orow[t];
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const int64_t o = (int64_t)m * Co + n0 + 16 * j + 4 * g;
                    if constexpr (EPI == PMG_EPI_ACC) {
                        *(v4i*)((int32_t*)a.out + o) = acc[t][j];
                    } else {
                        float y[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int n = 16 * j + 4 * g + i;
                            float u = (float)acc[t][j][i] * a.a_scale;
                            u = u * s_k[0][n];
                            if (a.bias) u = u + s_k[1][n];
                            y[i] = u;
                        }
                        if constexpr (EPI == PMG_EPI_R) {
                            const v4f sk = *(const v4f*)(a.skip + o);
                            *(v4f*)((float*)a.out + o) = v4f{y[0] + sk[0], y[1] + sk[1], y[2] + sk[2], y[3] + sk[3]};
                        } else {
                            *(v4f*)((float*)a.out + o) = v4f{y[0], y[1], y[2], y[3]};
                        }
                    }
                }
            }
        }
    }
}

// Ci = Co = 64: every tap's weights fit in LDS (27 x 4 KB in operand order), so the block loads them once and
// meets at no barrier afterwards -- each wave runs its chunks' taps on its own, and a wave that skips a tap (none
// of its tiles has it) gains the time instead of waiting for the others at the next group barrier. The tap loop
// is that of spconv_g2_k without the weight staging: a ring of RS slots gathers the codes RS - 1 taps ahead of
// their MFMAs and the map indices two taps before that. NWV waves per block (NWV = 16: four per SIMD, fewer
// registers each): each wave spends most of a tap waiting for its gathers, so more waves and deeper rings keep
// more of them in flight.
template <int C, int EPI, int T = kG2Tiles, int PF = 1, int RS = 2, int NWV = kG2Waves>
__global__ __launch_bounds__(64 * NWV, 1) void spconv_g2r_k(ConvArgs a) {
    constexpr int NB = C / 16, KS = C / 64;
    constexpr int NF = NB * KS;
    constexpr int CHUNK = NWV * T * 16;
    constexpr int NTH = 64 * NWV;
    constexpr int GD = RS - 1;                 // gather distance in taps
    constexpr int UNR = RS % 2 == 0 ? RS : 2 * RS;  // steps per loop trip: the X ring (RS) and the index pair (2)
    static_assert(C == 64, "resident weights: C = 64");
    static_assert(RS >= 2 && RS <= 4, "ring slots");
    __shared__ __attribute__((aligned(16))) v4i s_w[27 * NF * 64];
    __shared__ float s_k[2][C];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int S = (int)a.M;                     // map row stride (the capacity)
    const int M = a.m_dev ? (int)*a.m_dev : S;  // rows
    const int64_t ntile = (M + 15) >> 4;
    typedef const __attribute__((address_space(3))) v4i lds_v4i;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)(a.M * C), kBufWord3);
    const __amdgpu_buffer_rsrc_t nr =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.nmap_t, (short)0, (int)(a.M * 27 * 4), kBufWord3);
    for (int e = tid; e < 2 * C; e += NTH) {
        const int q = e / C, n = e - (e / C) * C;
        const float* src = q == 0 ? a.w_scale : a.bias;
        s_k[q][n] = src ? src[n] : 0.0f;
    }
    for (int e = tid; e < 27 * NF * 64; e += NTH) {
        const int f = e >> 6, l = e & 63;
        const int v = f / NF, js = f - (f / NF) * NF;
        const int j = js / KS, s2 = js - (js / KS) * KS;
        s_w[e] = *(const v4i*)((const uint8_t*)a.w + ((l & 15) * 27) * C + 16 * (l >> 4) + ((16 * j * 27) + v) * C + 64 * s2);
    }
    __syncthreads();

    const int nchunk = (M + CHUNK - 1) / CHUNK;
    const int G = gridDim.x, b = blockIdx.x;
    const int nx = G >= 8 ? 8 : 1;
    const int x = b % nx, bi = b / nx, nbx = (G - x + nx - 1) / nx;
    const int c0 = (int)((int64_t)nchunk * x / nx), c1 = (int)((int64_t)nchunk * (x + 1) / nx);
    // each wave takes the block's chunks independently: wave wv of chunk ch owns rows [16 T wv, 16 T (wv + 1))
    const int gi = a.m_dev ? 0 : xcd_group(nchunk);
    for (int kq = bi;; kq += nbx) {
        const int ch = gi ? ((kq / gi) * nx + x) * gi + kq % gi : c0 + kq;
        if (ch >= (gi ? nchunk : c1)) break;
        const int pos0 = ch * CHUNK + wv * (16 * T) + r;
        int roff[T], orow[T];  // map column (processing order) and output row; rows beyond M: out-of-range offset
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int p = pos0 + 16 * t;
            roff[t] = p < M ? 4 * p : (int)0x80000000;
            orow[t] = p < M && a.order ? a.order[p] : p;
        }
        uint32_t wmask;
        {
            const int64_t tl = (int64_t)ch * (CHUNK / 16) + wv * T + (lane & (T - 1));
            uint32_t mk = (lane < T && tl < ntile) ? a.tmask[tl] : 0u;
#pragma unroll
            for (int o = 1; o < T; o <<= 1) mk |= __shfl_xor(mk, o, 64);
            wmask = (uint32_t)__builtin_amdgcn_readfirstlane((int)mk);
        }
        v4i acc[T][NB];
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int j = 0; j < NB; ++j) acc[t][j] = v4i{0, 0, 0, 0};
        auto idx_load = [&](int v, int (&id)[T]) {
            const int vo = (v < 27 ? v : 27) * S * 4;
#pragma unroll
            for (int t = 0; t < T; ++t) id[t] = __builtin_amdgcn_raw_buffer_load_b32(nr, roff[t], vo, 0);
        };
        auto gather = [&](const int (&id)[T], v4i (&xs)[T][KS]) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
                const int off = id[t] >= 0 ? id[t] * C + 16 * g : (int)0x80000000;
#pragma unroll
                for (int s2 = 0; s2 < KS; ++s2) xs[t][s2] = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 64 * s2, 0);
            }
        };
        auto mma_tap = [&](int v, const v4i (&xs)[T][KS]) {
            const v4i* wb = s_w + v * NF * 64 + lane;
            v4i wop[PF];
#pragma unroll
            for (int k = 0; k < PF; ++k) wop[k] = *(lds_v4i*)(wb + ((k % NB) * KS + k / NB) * 64);
#pragma unroll
            for (int q = 0; q < NF; ++q) {
                const int s2 = q / NB, j = q - (q / NB) * NB;
                const v4i cur = wop[q % PF];
                if (q + PF < NF) {
                    const int s3 = (q + PF) / NB, j3 = (q + PF) - ((q + PF) / NB) * NB;
                    wop[q % PF] = *(lds_v4i*)(wb + (j3 * KS + s3) * 64);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int t = 0; t < T; ++t)
                    acc[t][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur, xs[t][s2], acc[t][j], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        // The wave walks only its own active taps (no barrier binds it to the block's union): a scalar queue holds
        // the taps of this step and the next GD + 2 (27 after the last: out-of-range indices, zeros, no MFMAs).
        uint32_t rem = wmask;
        auto pop = [&]() {
            const int v = rem ? (int)__builtin_ctz(rem) : 27;
            rem = rem ? rem & (rem - 1) : 0u;
            return v;
        };
        const int ntap = __builtin_popcount(wmask);
        int q[GD + 3];
#pragma unroll
        for (int u = 0; u < GD + 3; ++u) q[u] = pop();
        int I[2][T];
        v4i X[RS][T][KS];
#pragma unroll
        for (int u = 0; u < GD; ++u) {
            int iu[T];
            idx_load(q[u], iu);
            gather(iu, X[u]);
        }
        idx_load(q[GD], I[GD & 1]);
        idx_load(q[GD + 1], I[(GD + 1) & 1]);
        // step k: the codes of tap k+GD (indices loaded two steps ago) and the indices of tap k+GD+2 are
        // requested, then tap k's MFMAs run
        auto tap = [&](auto Kc) {
            constexpr int k = decltype(Kc)::value;
            constexpr int xs = (k + GD) % RS, is = (k + GD) & 1;
            gather(I[is], X[xs]);
            idx_load(q[GD + 2], I[is]);
            __builtin_amdgcn_sched_barrier(0);
            if (q[0] < 27) mma_tap(q[0], X[k % RS]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < GD + 2; ++u) q[u] = q[u + 1];
            q[GD + 2] = pop();
        };
#pragma unroll 1
        for (int k = 0; k < ntap; k += UNR) {
            tap(std::integral_constant<int, 0>{});
            tap(std::integral_constant<int, 1>{});
            if constexpr (UNR > 2) {
                tap(std::integral_constant<int, 2>{});
                tap(std::integral_constant<int, 3>{});
            }
            if constexpr (UNR > 4) {
                tap(std::integral_constant<int, 4>{});
                tap(std::integral_constant<int, 5>{});
            }
        }
        if constexpr (EPI == PMG_EPI_Q || EPI == PMG_EPI_QLIN) {
            store_tile_codes<EPI, T, NB>(a, acc, s_k[0], s_k[1], orow, pos0, M, C, 0, g);
            continue;
        }
#pragma unroll
        for (int t = 0; t < T; ++t) {
            if (pos0 + 16 * t >= M) continue;
            const int m = orow[t];
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int64_t o = (int64_t)m * C + 16 * j + 4 * g;
                if constexpr (EPI == PMG_EPI_ACC) {
                    *(v4i*)((int32_t*)a.out + o) = acc[t][j];
                } else {
                    float y[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int n = 16 * j + 4 * g + i;
                        float u = (float)acc[t][j][i] * a.a_scale;
                        u = u * s_k[0][n];
                        if (a.bias) u = u + s_k[1][n];
                        y[i] = u;
                    }
                    if constexpr (EPI == PMG_EPI_Q) {
                        store_silu_codes4(y, a.out_mult, (int8_t*)a.out + o);
                    } else if constexpr (EPI == PMG_EPI_QLIN) {
                        store_codes4(y, a.out_mult, (int8_t*)a.out + o);
                    } else if constexpr (EPI == PMG_EPI_R) {
                        const v4f sk = *(const v4f*)(a.skip + o);
                        *(v4f*)((float*)a.out + o) = v4f{y[0] + sk[0], y[1] + sk[1], y[2] + sk[2], y[3] + sk[3]};
                    } else {
                        *(v4f*)((float*)a.out + o) = v4f{y[0], y[1], y[2], y[3]};
                    }
                }
            }
        }
    }
}

// The host-sized C = 64 launch: 16-row tiles per wave, gather ring slots, waves per block.
constexpr int kG2rT = 4, kG2rRS = 2, kG2rWaves = 8;

template <int C>
static int launch_g2r(const ConvArgs& a, int epilogue, hipStream_t s) {
    static int cus = -1;
    if (cus < 0) cus = num_cus();
    constexpr int T = kG2rT, RS = kG2rRS, NWV = kG2rWaves, CHUNK = NWV * T * 16;
    const int64_t nchunk = (a.M + CHUNK - 1) / CHUNK;
    const dim3 grid((unsigned)(nchunk < cus ? nchunk : cus)), blk(64 * NWV);
    switch (epilogue) {
        case PMG_EPI_ACC: hipLaunchKernelGGL((spconv_g2r_k<C, PMG_EPI_ACC, T, 1, RS, NWV>), grid, blk, 0, s, a); break;
        case PMG_EPI_Q: hipLaunchKernelGGL((spconv_g2r_k<C, PMG_EPI_Q, T, 1, RS, NWV>), grid, blk, 0, s, a); break;
        case PMG_EPI_QLIN: hipLaunchKernelGGL((spconv_g2r_k<C, PMG_EPI_QLIN, T, 1, RS, NWV>), grid, blk, 0, s, a); break;
        case PMG_EPI_R: hipLaunchKernelGGL((spconv_g2r_k<C, PMG_EPI_R, T, 1, RS, NWV>), grid, blk, 0, s, a); break;
        case PMG_EPI_BIAS: hipLaunchKernelGGL((spconv_g2r_k<C, PMG_EPI_BIAS, T, 1, RS, NWV>), grid, blk, 0, s, a); break;
        default: return fail(PMG_E_INVALID, "spconv: epilogue not available for this precision");
    }
    return check_launch("spconv_g2r_k");
}

// The host-sized C = 128 launch: 16-row tiles per wave and gather ring slots.
constexpr int kG2T128 = 4, kG2RS128 = 2;

template <int C>
static int launch_g2(const ConvArgs& a, int epilogue, hipStream_t s) {
    if constexpr (C == 64) {
        return launch_g2r<64>(a, epilogue, s);
    } else {
        static int cus = -1;
        if (cus < 0) cus = num_cus();
        constexpr int T = kG2T128, RS = kG2RS128, CHUNK = kG2Waves * T * 16;
        const int64_t nchunk = (a.M + CHUNK - 1) / CHUNK;
        const dim3 grid((unsigned)(nchunk < cus ? nchunk : cus)), blk(kG2Threads);
        switch (epilogue) {
            case PMG_EPI_ACC: hipLaunchKernelGGL((spconv_g2_k<C, PMG_EPI_ACC, C / 16, T, 1, RS, false>), grid, blk, 0, s, a); break;
            case PMG_EPI_Q: hipLaunchKernelGGL((spconv_g2_k<C, PMG_EPI_Q, C / 16, T, 1, RS, false>), grid, blk, 0, s, a); break;
            case PMG_EPI_QLIN: hipLaunchKernelGGL((spconv_g2_k<C, PMG_EPI_QLIN, C / 16, T, 1, RS, false>), grid, blk, 0, s, a); break;
            case PMG_EPI_R: hipLaunchKernelGGL((spconv_g2_k<C, PMG_EPI_R, C / 16, T, 1, RS, false>), grid, blk, 0, s, a); break;
            case PMG_EPI_BIAS: hipLaunchKernelGGL((spconv_g2_k<C, PMG_EPI_BIAS, C / 16, T, 1, RS, false>), grid, blk, 0, s, a); break;
            default: return fail(PMG_E_INVALID, "spconv: epilogue not available for this precision");
        }
        return check_launch("spconv_g2_k");
    }
}

// fp16 / bf16 / fp32 features, Ci = Co = C with rows of 64 - 1024 bytes: the weight-staged kernel on K chunks of 32
// halves (v_mfma_f32_16x16x32_f16 / _bf16) or 16 floats (four v_mfma_f32_16x16x4f32), fp32 accumulators. Rows of
// 256 bytes hold 16 tiles of accumulators per wave at T = 4, so they run T = 2; rows of 512 and 1024 bytes (fp16
// C = 256, 512) split the output channels into slices of 64 (blockIdx.y: a tap's weights fit the LDS buffers) and
// run T = 2 and 1 (the gathered rows of the two ring slots fill the registers).
template <typename E, int C>
static int launch_g2f(const ConvArgs& a, int epilogue, hipStream_t s) {
    static int cus = -1;
    if (cus < 0) cus = num_cus();
    constexpr int RB = C * (int)sizeof(E);
    constexpr int NB = RB <= 256 ? C / 16 : 4;
    constexpr int T = RB <= 128 ? 4 : (RB <= 512 ? 2 : 1), CHUNK = kG2Waves * T * 16;
    constexpr int PFV = RB >= 512 ? 4 : 1;  // weight operands read ahead (measured: 3 % faster at C = 256 / 512)
    const int64_t nchunk = (a.M + CHUNK - 1) / CHUNK;
    const dim3 grid((unsigned)(nchunk < cus ? nchunk : cus), (unsigned)(C / (16 * NB))), blk(kG2Threads);
    switch (epilogue) {
        case PMG_EPI_ACC: hipLaunchKernelGGL((spconv_g2_k<C, PMG_EPI_ACC, NB, T, PFV, 2, false, E>), grid, blk, 0, s, a); break;
        case PMG_EPI_BIAS: hipLaunchKernelGGL((spconv_g2_k<C, PMG_EPI_BIAS, NB, T, PFV, 2, false, E>), grid, blk, 0, s, a); break;
        case PMG_EPI_R: hipLaunchKernelGGL((spconv_g2_k<C, PMG_EPI_R, NB, T, PFV, 2, false, E>), grid, blk, 0, s, a); break;
        case PMG_EPI_SILU:
            if constexpr (std::is_same<E, _Float16>::value) {
                hipLaunchKernelGGL((spconv_g2_k<C, PMG_EPI_SILU, NB, T, PFV, 2, false, E>), grid, blk, 0, s, a);
                break;
            }
            [[fallthrough]];
        default: return fail(PMG_E_INVALID, "spconv: epilogue not available for this precision");
    }
    return check_launch("spconv_g2_k");
}

// Whether the fp staged kernel takes this convolution: Ci = Co >= 32 with rows of 64 - 256 bytes (fp16 / bf16 32,
// 64, 128; fp32 32, 64), or fp16 / bf16 rows of 512 or 1024 bytes (C = 256, 512: slices of 64 output channels),
// 32-bit buffer offsets and aligned vectors.
static bool g2f_fits(const ConvArgs& a, int Ci, int elt, int epilogue) {
    const int rb = Ci * elt;
    return Ci == a.Co && Ci >= 32 && Ci % 16 == 0 &&
           (rb == 64 || rb == 128 || rb == 256 || (elt == 2 && (rb == 512 || rb == 1024))) &&
           a.M * 27 * 4 < ((int64_t)1 << 31) && a.M * rb < ((int64_t)1 << 31) && aligned16(a.out) &&
           (epilogue != PMG_EPI_R || aligned16(a.skip));
}

// Device-sized launches of the staged kernels (Ci = Co = C): the grid covers the capacity's chunks, at most one
// block per CU in x (blockIdx.y: the output-channel slice), and every block reads the row count and takes its XCD
// band's share of the chunks that hold rows; the others return at once.
template <int C, int NB, int T, int PF, int RS>
static int launch_g2_dev(const ConvArgs& a, int epilogue, hipStream_t s) {
    static int cus = -1;
    if (cus < 0) cus = num_cus();
    constexpr int CHUNK = kG2Waves * T * 16;
    const int64_t nchunk = (a.M + CHUNK - 1) / CHUNK;
    const dim3 grid((unsigned)(nchunk < cus ? nchunk : cus), (unsigned)(a.Co / (16 * NB)));
    if constexpr (C == 64) {
        static_assert(NB == 4, "C = 64 keeps all 64 output channels");
        static_assert(RS == 2, "the resident-weight kernel has no tap split");
        // gathers three taps ahead (a 4-slot ring): on the U-Net's level 1 (183k voxels) 2.5 us faster per conv
        // than one tap ahead
        switch (epilogue) {
            case PMG_EPI_ACC: hipLaunchKernelGGL((spconv_g2r_k<C, PMG_EPI_ACC, T, PF, 4>), grid, dim3(kG2Threads), 0, s, a); break;
            case PMG_EPI_Q: hipLaunchKernelGGL((spconv_g2r_k<C, PMG_EPI_Q, T, PF, 4>), grid, dim3(kG2Threads), 0, s, a); break;
            case PMG_EPI_R: hipLaunchKernelGGL((spconv_g2r_k<C, PMG_EPI_R, T, PF, 4>), grid, dim3(kG2Threads), 0, s, a); break;
            default: hipLaunchKernelGGL((spconv_g2r_k<C, PMG_EPI_BIAS, T, PF, 4>), grid, dim3(kG2Threads), 0, s, a); break;
        }
        return check_launch("spconv_g2r_k");
    } else {
        switch (epilogue) {
            case PMG_EPI_ACC: hipLaunchKernelGGL((spconv_g2_k<C, PMG_EPI_ACC, NB, T, PF, RS>), grid, dim3(kG2Threads), 0, s, a); break;
            case PMG_EPI_Q: hipLaunchKernelGGL((spconv_g2_k<C, PMG_EPI_Q, NB, T, PF, RS>), grid, dim3(kG2Threads), 0, s, a); break;
            case PMG_EPI_R: hipLaunchKernelGGL((spconv_g2_k<C, PMG_EPI_R, NB, T, PF, RS>), grid, dim3(kG2Threads), 0, s, a); break;
            default: hipLaunchKernelGGL((spconv_g2_k<C, PMG_EPI_BIAS, NB, T, PF, RS>), grid, dim3(kG2Threads), 0, s, a); break;
        }
        return check_launch("spconv_g2_k");
    }
}

// A device-sized weight-staged launch with the tap split allowed when the partials buffer holds its largest case
// (Z * rows * Co * 4 bytes: at most kSplitUnits * chunk * Co / slices * 4, since Z * chunks * slices <= kSplitUnits),
// followed by split_epilogue_k.
template <int C, int NB, int T, int PF>
static int launch_g2_dev_split(ConvArgs a, int epilogue, int32_t* part, int64_t part_bytes, hipStream_t s) {
    constexpr int CHUNK = kG2Waves * T * 16;
    const int64_t need = (int64_t)kSplitUnits * CHUNK * (16 * NB) * 4;
    a.part = part && part_bytes >= need ? part : nullptr;
    const int rc = launch_g2_dev<C, NB, T, PF, 4>(a, epilogue, s);
    if (rc || !a.part) return rc;
    const int nslice = a.Co / (16 * NB);
    const int64_t blocks = (a.M * (a.Co / 4) + 255) / 256;
    const dim3 grid((unsigned)(blocks < 1024 ? blocks : 1024));
    switch (epilogue) {
        case PMG_EPI_ACC: hipLaunchKernelGGL((split_epilogue_k<PMG_EPI_ACC, CHUNK>), grid, dim3(256), 0, s, a, nslice); break;
        case PMG_EPI_Q: hipLaunchKernelGGL((split_epilogue_k<PMG_EPI_Q, CHUNK>), grid, dim3(256), 0, s, a, nslice); break;
        case PMG_EPI_R: hipLaunchKernelGGL((split_epilogue_k<PMG_EPI_R, CHUNK>), grid, dim3(256), 0, s, a, nslice); break;
        default: hipLaunchKernelGGL((split_epilogue_k<PMG_EPI_BIAS, CHUNK>), grid, dim3(256), 0, s, a, nslice); break;
    }
    return check_launch("split_epilogue_k");
}

int64_t conv_split_bytes(int C) {
    if (C == 128) return (int64_t)kSplitUnits * (kG2Waves * 2 * 16) * 128 * 4;
    if (C == 256) return (int64_t)kSplitUnits * (kG2Waves * 1 * 16) * 128 * 4;
    return 0;
}

int launch_conv_i8_dev(const DevConv& d, hipStream_t s) {
    PMG_REQUIRE(d.x && d.nmap_t && d.tile_mask && d.w && d.out && d.m_dev, "null buffer");
    PMG_REQUIRE(d.Ci % 16 == 0 && d.Co % 16 == 0 && d.Ci > 0 && d.Co > 0, "channels must be multiples of 16");
    PMG_REQUIRE(d.epilogue == PMG_EPI_Q || d.epilogue == PMG_EPI_R || d.epilogue == PMG_EPI_BIAS ||
                    d.epilogue == PMG_EPI_ACC,
                "unsupported epilogue");
    PMG_REQUIRE(d.epilogue != PMG_EPI_R || d.skip, "skip required");
    if (d.cap == 0) return PMG_OK;
    ConvArgs a{};
    a.x = (const uint8_t*)d.x;
    a.nmap_t = d.nmap_t;
    a.tmask = d.tile_mask;
    a.w = (const uint8_t*)d.w;
    a.M = d.cap;
    a.Co = d.Co;
    a.row_bytes = d.Ci;
    a.nchunk = d.Ci / 16;
    a.a_scale = d.a_scale;
    a.w_scale = d.w_scale;
    a.bias = d.bias;
    a.out_mult = d.out_mult;
    a.skip = d.skip;
    a.out = d.out;
    a.m_dev = d.m_dev;
    // the staged kernels' buffer offsets are 32-bit
    const bool fits32 = d.cap * 27 * 4 < ((int64_t)1 << 31) && d.cap * d.Ci < ((int64_t)1 << 31);
    if (fits32 && d.Ci == d.Co) {
        if (d.Ci == 64) return launch_g2_dev<64, 4, 2, 2, 2>(a, d.epilogue, s);
        if (d.Ci == 128) return launch_g2_dev_split<128, 8, 2, 3>(a, d.epilogue, d.part, d.part_bytes, s);
        if (d.Ci == 256) return launch_g2_dev_split<256, 8, 1, 3>(a, d.epilogue, d.part, d.part_bytes, s);
    }
    const int nb = pick_nb(d.Co);
    switch (d.epilogue) {
        case PMG_EPI_Q: return launch_nb<int8_t, PMG_EPI_Q>(a, nb, s);
        case PMG_EPI_R: return launch_nb<int8_t, PMG_EPI_R>(a, nb, s);
        case PMG_EPI_BIAS: return launch_nb<int8_t, PMG_EPI_BIAS>(a, nb, s);
        default: return launch_nb<int8_t, PMG_EPI_ACC>(a, nb, s);
    }
}

template <typename T>
static int conv_common(const ConvArgs& a, int Ci, int epilogue, hipStream_t s);

// The fp16 teacher's convolution on a device-sized level (the int8 one's counterpart): x and w fp16, fp32
// accumulation; epilogues SILU (bias, SiLU, fp16 out: conv1), R (bias + skip, fp32: conv2), BIAS, ACC. The
// weight-staged kernel takes Ci = Co = 32, 64, 128 (it reads the row count on the device); other widths the generic
// one-wave-per-16-rows kernel.
int launch_conv_f16_dev(const DevConv& d, hipStream_t s) {
    PMG_REQUIRE(d.x && d.nmap_t && d.tile_mask && d.w && d.out && d.m_dev, "null buffer");
    PMG_REQUIRE(d.Ci % 16 == 0 && d.Co % 16 == 0 && d.Ci > 0 && d.Co > 0, "channels must be multiples of 16");
    PMG_REQUIRE(d.epilogue == PMG_EPI_SILU || d.epilogue == PMG_EPI_R || d.epilogue == PMG_EPI_BIAS ||
                    d.epilogue == PMG_EPI_ACC,
                "unsupported epilogue");
    PMG_REQUIRE(d.epilogue != PMG_EPI_R || d.skip, "skip required");
    if (d.cap == 0) return PMG_OK;
    ConvArgs a{};
    a.x = (const uint8_t*)d.x;
    a.nmap_t = d.nmap_t;
    a.tmask = d.tile_mask;
    a.w = (const uint8_t*)d.w;
    a.M = d.cap;
    a.Co = d.Co;
    a.row_bytes = 2 * d.Ci;
    a.nchunk = 2 * d.Ci / 16;
    a.a_scale = 1.0f;
    a.bias = d.bias;
    a.skip = d.skip;
    a.out = d.out;
    a.m_dev = d.m_dev;
    if (g2f_fits(a, d.Ci, 2, d.epilogue)) {
        if (d.Ci == 32) return launch_g2f<_Float16, 32>(a, d.epilogue, s);
        if (d.Ci == 64) return launch_g2f<_Float16, 64>(a, d.epilogue, s);
        if (d.Ci == 128) return launch_g2f<_Float16, 128>(a, d.epilogue, s);
        if (d.Ci == 256) return launch_g2f<_Float16, 256>(a, d.epilogue, s);
        return launch_g2f<_Float16, 512>(a, d.epilogue, s);
    }
    return conv_common<_Float16>(a, d.Ci, d.epilogue, s);
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
        case PMG_EPI_QLIN:
            if constexpr (sizeof(T) == 1) return launch_nb<T, PMG_EPI_QLIN>(a, nb, s);
            break;
        case PMG_EPI_SILU:
            if constexpr (std::is_same<T, _Float16>::value) return launch_nb<T, PMG_EPI_SILU>(a, nb, s);
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
    PMG_REQUIRE((epilogue != PMG_EPI_Q && epilogue != PMG_EPI_QLIN) || out_mult > 0.0f, "out_mult must be positive");
    if (M == 0) return PMG_OK;
    ConvArgs a{(const uint8_t*)x, nmap_t, tile_mask, (const uint8_t*)w, M, Co, Ci, Ci / 16,
               a_scale, w_scale, bias, out_mult, skip, out};
    // The block-tiled kernel addresses x and the map through 32-bit buffer offsets.
    const bool fits32 = M * 27 * 4 < ((int64_t)1 << 31) && M * Ci < ((int64_t)1 << 31);
    if (Ci == Co && (Ci == 64 || Ci == 128) && fits32 && epilogue != PMG_EPI_SILU && aligned16(out) &&
        aligned16(x) && aligned16(w) && (epilogue != PMG_EPI_R || aligned16(skip))) {
        if (Ci == 64) return launch_g2<64>(a, epilogue, (hipStream_t)stream);
        return launch_g2<128>(a, epilogue, (hipStream_t)stream);
    }
    return conv_common<int8_t>(a, Ci, epilogue, (hipStream_t)stream);
}

int pmg_spconv_i8_ordered(const int8_t* x, const int32_t* nmap_o, const int32_t* order, const uint32_t* order_tile_mask,
                          int64_t M, int Ci, int Co, const int8_t* w, int epilogue, float a_scale,
                          const float* w_scale, const float* bias, float out_mult, const float* skip, void* out,
                          void* stream) {
    if (int e = validate(x, nmap_o, order_tile_mask, M, Ci, Co, w, out, 1, "pmg_spconv_i8_ordered")) return e;
    PMG_REQUIRE(order, "null order");
    PMG_REQUIRE(epilogue == PMG_EPI_ACC || w_scale, "w_scale required");
    PMG_REQUIRE(epilogue != PMG_EPI_R || skip, "skip required");
    PMG_REQUIRE((epilogue != PMG_EPI_Q && epilogue != PMG_EPI_QLIN) || out_mult > 0.0f, "out_mult must be positive");
    PMG_REQUIRE(Ci == Co && (Ci == 64 || Ci == 128), "pmg_spconv_i8_ordered: Ci = Co = 64 or 128");
    PMG_REQUIRE(M * 27 * 4 < ((int64_t)1 << 31) && M * Ci < ((int64_t)1 << 31), "pmg_spconv_i8_ordered: M too large");
    PMG_REQUIRE(epilogue != PMG_EPI_SILU && aligned16(out) && aligned16(x) && aligned16(w) &&
                    (epilogue != PMG_EPI_R || aligned16(skip)),
                "pmg_spconv_i8_ordered: unsupported epilogue or unaligned x / w / output");
    if (M == 0) return PMG_OK;
    ConvArgs a{(const uint8_t*)x, nmap_o, order_tile_mask, (const uint8_t*)w, M, Co, Ci, Ci / 16,
               a_scale, w_scale, bias, out_mult, skip, out, order};
    if (Ci == 64) return launch_g2<64>(a, epilogue, (hipStream_t)stream);
    return launch_g2<128>(a, epilogue, (hipStream_t)stream);
}

int pmg_spconv_f16(const uint16_t* x, const int32_t* nmap_t, const uint32_t* tile_mask, int64_t M, int Ci, int Co,
                   const uint16_t* w, int epilogue, const float* bias, const float* skip, void* out, void* stream) {
    if (int e = validate(x, nmap_t, tile_mask, M, Ci, Co, w, out, 2, "pmg_spconv_f16")) return e;
    PMG_REQUIRE(epilogue != PMG_EPI_R || skip, "skip required");
    if (M == 0) return PMG_OK;
    ConvArgs a{(const uint8_t*)x, nmap_t, tile_mask, (const uint8_t*)w, M, Co, Ci * 2, Ci * 2 / 16,
               1.0f, nullptr, bias, 1.0f, skip, out};
    if (g2f_fits(a, Ci, 2, epilogue)) {
        if (Ci == 32) return launch_g2f<_Float16, 32>(a, epilogue, (hipStream_t)stream);
        if (Ci == 64) return launch_g2f<_Float16, 64>(a, epilogue, (hipStream_t)stream);
        if (Ci == 128) return launch_g2f<_Float16, 128>(a, epilogue, (hipStream_t)stream);
        if (Ci == 256) return launch_g2f<_Float16, 256>(a, epilogue, (hipStream_t)stream);
        return launch_g2f<_Float16, 512>(a, epilogue, (hipStream_t)stream);
    }
    return conv_common<_Float16>(a, Ci, epilogue, (hipStream_t)stream);
}

int pmg_spconv_bf16(const uint16_t* x, const int32_t* nmap_t, const uint32_t* tile_mask, int64_t M, int Ci, int Co,
                    const uint16_t* w, int epilogue, const float* bias, const float* skip, float* out, void* stream) {
    if (int e = validate(x, nmap_t, tile_mask, M, Ci, Co, w, out, 2, "pmg_spconv_bf16")) return e;
    PMG_REQUIRE(epilogue == PMG_EPI_ACC || epilogue == PMG_EPI_BIAS || epilogue == PMG_EPI_R,
                "bf16 supports the ACC, BIAS and R epilogues");
    PMG_REQUIRE(epilogue != PMG_EPI_R || skip, "skip required");
    if (M == 0) return PMG_OK;
    ConvArgs a{(const uint8_t*)x, nmap_t, tile_mask, (const uint8_t*)w, M, Co, Ci * 2, Ci * 2 / 16,
               1.0f, nullptr, bias, 1.0f, skip, out};
    if (g2f_fits(a, Ci, 2, epilogue)) {
        if (Ci == 32) return launch_g2f<__bf16, 32>(a, epilogue, (hipStream_t)stream);
        if (Ci == 64) return launch_g2f<__bf16, 64>(a, epilogue, (hipStream_t)stream);
        if (Ci == 128) return launch_g2f<__bf16, 128>(a, epilogue, (hipStream_t)stream);
        if (Ci == 256) return launch_g2f<__bf16, 256>(a, epilogue, (hipStream_t)stream);
        return launch_g2f<__bf16, 512>(a, epilogue, (hipStream_t)stream);
    }
    return conv_common<__bf16>(a, Ci, epilogue, (hipStream_t)stream);
}

int pmg_spconv_f32(const float* x, const int32_t* nmap_t, const uint32_t* tile_mask, int64_t M, int Ci, int Co,
                   const float* w, int epilogue, const float* bias, float* out, void* stream) {
    if (int e = validate(x, nmap_t, tile_mask, M, Ci, Co, w, out, 4, "pmg_spconv_f32")) return e;
    PMG_REQUIRE(epilogue == PMG_EPI_ACC || epilogue == PMG_EPI_BIAS, "fp32 supports ACC and BIAS epilogues");
    if (M == 0) return PMG_OK;
    ConvArgs a{(const uint8_t*)x, nmap_t, tile_mask, (const uint8_t*)w, M, Co, Ci * 4, Ci * 4 / 16,
               1.0f, nullptr, bias, 1.0f, nullptr, out};
    if (g2f_fits(a, Ci, 4, epilogue)) {
        if (Ci == 32) return launch_g2f<float, 32>(a, epilogue, (hipStream_t)stream);
        return launch_g2f<float, 64>(a, epilogue, (hipStream_t)stream);
    }
    return conv_common<float>(a, Ci, epilogue, (hipStream_t)stream);
}

}  // extern "C"
