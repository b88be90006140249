// Level-0 submanifold 3x3x3 convolution straight from the voxel keys: the column-stencil map of
// _build_submanifold_nmap_column (_core.py:269-295) is never materialised.
//
// At level 0 every pixel is one voxel (MoGeModel._voxelize, v3.py:305-344), so the neighbour of voxel o at tap
// (di, dj, dz) is pixel o + di*W + dj when that pixel is in frame and its key equals key[o] + dz.
//
// Work decomposition. A persistent block of 8 waves owns segments of SEG = 256 consecutive voxels (32 rows per
// wave). All neighbours of a segment lie in three raster ranges [s0 + di*W - 1, s0 + di*W + SEG + 1) -- the
// "window" -- which is staged in LDS together with the window's keys. The next segment's window is loaded into
// registers while the current one is computed and written to the second LDS buffer afterwards, so HBM latency is
// overlapped with the matrix work. Each activation row is fetched about three times per layer (once per window
// that contains it) instead of once per (row, tap). The weights (Co, 27, Ci) stay resident in LDS for the whole
// block when they fit.
//
// Matrix cores: D[n][m] = sum_k W[n][k] X[m][k] with v_mfma_*_16x16x* and the weights as the first operand, so a
// lane holds 4 consecutive output channels of one voxel (lane l: channels 16j + 4(l/16) + i, voxel l%16) and every
// epilogue stores 4-byte (int8) or 16-byte (fp32) vectors. The reduction runs over the wave's union of active taps
// (a 27-bit mask OR-ed over its 32 rows) x 16-byte channel chunks, iterated as a scalar (wave-uniform) loop with the
// operands of the next step loaded before the current step's MFMAs issue. A row whose own tap is absent contributes
// a zero operand, so each row accumulates exactly its own neighbours.
//
// Epilogues (one pass over the output):
//   ACC    raw accumulator (int32 / fp32), for parity
//   Q      int8: clamp(rint(silu(acc*a_scale*w_scale + bias) * out_mult), +-127);  fp16: half(silu(acc + bias)),
//          SiLU by the hardware exp2/reciprocal (silu_fast: within one fp16 ulp of the exact form)
//   R      x_new = dequant(acc) + skip                                   (fp32 residual stream)
//   RLN    R, stores x_new, then the next block's LayerNorm -> SiLU -> int8 codes (or fp16), so the residual block
//          needs no separate normalisation pass (flex_sparse_blocks.py:230-234)
//   ROUT   R, then out_proj (C -> 1) and logz += delta into the output point map (sparse_unet.py:258; v3.py:359)
// Requantisation multiplies by 127/clip as the reference's deployed kernels do (SparseConvInt8.metal:109,
// Refiner.metal:120, with 127/clip from Refiner.swift:148). LayerNorm and out_proj sum in the "quad" order: lane
// group g sums its channels 16j+4g+i (j outer, i inner), then ((s0 + s1) + (s2 + s3)) across the four groups; every
// LayerNorm of the step uses that same order.
#include <climits>
#include <type_traits>

#include "pmg_common.h"
#include "pmg_internal.h"

namespace pmg {

constexpr int kColThreads = 512;
constexpr int kColWaves = kColThreads / 64;
constexpr int kSeg = 32 * kColWaves;  // 256 voxels per segment
constexpr int kWin = kSeg + 2;
constexpr int kZFar = INT_MIN / 2;  // key of a window slot outside the map (never within +-1 of a real key)

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

__device__ inline uint32_t sgpr(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// Geometry of the LDS buffers for one instantiation.
template <typename T, int C>
struct ColGeom {
    static constexpr int ROWB = C * (int)sizeof(T);
    static constexpr int NCH = ROWB / 16;
    static constexpr int XBYTES = 3 * kWin * ROWB;
    static constexpr int ZBYTES = 3 * kWin * 4;
    static constexpr int WBYTES = C * 27 * ROWB;
    static constexpr bool WLDS = WBYTES <= 64 * 1024;
    static constexpr int LDS1 = (WLDS ? WBYTES : 0) + XBYTES + ZBYTES;
    static constexpr int NBUF = (LDS1 + XBYTES + ZBYTES) <= 150 * 1024 ? 2 : 1;
    static constexpr bool FITS = LDS1 <= 150 * 1024;
    static constexpr int PF = (3 * kWin * NCH + kColThreads - 1) / kColThreads;  // x chunks per thread
    static constexpr int PFZ = (3 * kWin + kColThreads - 1) / kColThreads;        // keys per thread
};

// Per-channel epilogue constants, read through a pointer type P (global, or LDS when a kernel stages them).
template <class P>
struct EpiConst {
    P ws, bs, gamma, beta, ow;
    bool has_bias;
};
__device__ inline EpiConst<const float*> epi_global(const ColConvArgs& a) {
    return EpiConst<const float*>{a.w_scale, a.bias, a.ln_gamma, a.ln_beta, a.out_w, a.bias != nullptr};
}

// Epilogue of one 16-voxel tile: lane holds channels 16j + 4g + i (j < C/16, i < 4) of voxel m.
// The skip (residual) vectors of the residual epilogues are loaded by the caller (load_skip), so that a kernel can
// issue them for several tiles before it needs them.
template <int C>
__device__ inline void load_skip(const ColConvArgs& a, int m, int M, int g, v4f (&sk)[C / 16]) {
    const int64_t mo = m < M ? m : 0;
#pragma unroll
    for (int j = 0; j < C / 16; ++j) sk[j] = *(const v4f*)(a.skip + mo * C + 16 * j + 4 * g);
}

// The 4-float vector pointer of the address space of a float pointer type (global or LDS constants).
template <class P>
struct P4Of {
    typedef const v4f* type;
};
template <>
struct P4Of<const __attribute__((address_space(3))) float*> {
    typedef const __attribute__((address_space(3))) v4f* type;
};
template <class P>
using P4 = typename P4Of<P>::type;

// The first block's skip recomputed from the level-0 inputs (ColConvArgs::x0_feats): the row's (x/z, y/z, logz,
// residual, gate) are loaded first (x0_load, issued early like load_skip), then the lane's channels of h are formed
// from the staged input_proj / prompt_proj constants (x0_skip; the layout of ColConvArgs: in_w [C][3], in_b [C],
// pr_w [C][2], pr_b [C] at offsets 0, 3C, 4C, 6C).
__device__ inline void x0_load(const ColConvArgs& a, int m, int M, float (&in)[5]) {
    const int64_t mo = m < M ? m : 0;
    in[0] = a.x0_feats[mo * 3 + 0];
    in[1] = a.x0_feats[mo * 3 + 1];
    in[2] = a.x0_feats[mo * 3 + 2];
    if (a.x0_rg) {
        const float2 rg = *(const float2*)(a.x0_rg + mo * 2);
        in[3] = rg.x;
        in[4] = rg.y;
    } else {
        in[3] = in[4] = 0.0f;
    }
}

template <int C, class P>
__device__ inline void x0_skip(P c, bool prompt, const float (&in)[5], int g, v4f (&sk)[C / 16]) {
#pragma unroll
    for (int j = 0; j < C / 16; ++j) {
        const int n0 = 16 * j + 4 * g;
        const v4f w0 = *(P4<P>)(c + 3 * n0), w1 = *(P4<P>)(c + 3 * n0 + 4), w2 = *(P4<P>)(c + 3 * n0 + 8);
        const v4f b = *(P4<P>)(c + 3 * C + n0);
        const v4f p0 = *(P4<P>)(c + 4 * C + 2 * n0), p1 = *(P4<P>)(c + 4 * C + 2 * n0 + 4);
        const v4f pb = *(P4<P>)(c + 6 * C + n0);
        const float wi[12] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3], w2[0], w2[1], w2[2], w2[3]};
        const float pw[8] = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
#pragma unroll
        for (int i = 0; i < 4; ++i)
            sk[j][i] = x0_channel(wi[3 * i], wi[3 * i + 1], wi[3 * i + 2], b[i], in[0], in[1], in[2], prompt,
                                  pw[2 * i], pw[2 * i + 1], pb[i], in[3], in[4]);
        if constexpr (C / 16 >= 4) __builtin_amdgcn_sched_barrier(0);  // one block's constants live at a time
    }
}

template <typename T, int C, int EPI, class P = const float*>
__device__ inline void col_epilogue(const ColConvArgs& a, const typename ColAcc<T>::type (&acc)[C / 16], int m,
                                    int M, int g, const EpiConst<P>& k, const v4f (&sk)[C / 16]) {
    constexpr int NB = C / 16;
    const bool ok = m < M;
    const int64_t mo = ok ? m : 0;
    float y[NB][4];
    if constexpr (EPI != PMG_EPI_ACC) {
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (sizeof(T) == 1) {
                    const float t = (float)acc[j][i] * a.a_scale;
                    y[j][i] = t * k.ws[16 * j + 4 * g + i];
                } else {
                    y[j][i] = acc[j][i];
                }
            }
        // the bias in one branch, uniform over the launch, instead of a select per element
        if (k.has_bias) {
#pragma unroll
            for (int j = 0; j < NB; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) y[j][i] = y[j][i] + k.bs[16 * j + 4 * g + i];
        }
    }
    if constexpr (EPI == PMG_EPI_ACC) {
        if (ok) {
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int64_t o = mo * C + 16 * j + 4 * g;
                if constexpr (sizeof(T) == 1)
                    *(v4i*)((int32_t*)a.out + o) = acc[j];
                else
                    *(v4f*)((float*)a.out + o) = acc[j];
            }
        }
    } else if constexpr (EPI == PMG_EPI_Q) {
        if constexpr (sizeof(T) == 1) {
            uint32_t pk[NB];
            silu_codes_packed<NB>(y, a.out_mult, pk);
            if (ok) {
#pragma unroll
                for (int j = 0; j < NB; ++j) *(uint32_t*)((int8_t*)a.out + mo * C + 16 * j + 4 * g) = pk[j];
            }
        } else if (ok) {
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int64_t o = mo * C + 16 * j + 4 * g;
                {
                    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                    h4 hv;
#pragma unroll
                    for (int i = 0; i < 4; ++i) hv[i] = (_Float16)silu_fast(y[j][i]);
                    *(h4*)((_Float16*)a.out + o) = hv;
                }
            }
        }
    } else {
        // residual: x_new = y + skip
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int64_t o = mo * C + 16 * j + 4 * g;
#pragma unroll
            for (int i = 0; i < 4; ++i) y[j][i] = y[j][i] + sk[j][i];
            if (EPI != PMG_EPI_ROUT && ok) *(v4f*)((float*)a.out + o) = v4f{y[j][0], y[j][1], y[j][2], y[j][3]};
        }
        if constexpr (EPI == PMG_EPI_RLN) {
            ln_silu_quad<NB, sizeof(T) != 1>(y, k.gamma, k.beta, a.ln_eps, g);
            if constexpr (sizeof(T) == 1) {
                uint32_t pk[NB];
                silu_codes_packed<NB>(y, a.next_mult, pk);
                if (ok) {
#pragma unroll
                    for (int j = 0; j < NB; ++j)
                        *(uint32_t*)((int8_t*)a.next_q + mo * C + 16 * j + 4 * g) = pk[j];
                }
            } else if (ok) {
#pragma unroll
                for (int j = 0; j < NB; ++j) store_half4(y[j], (_Float16*)a.next_q + mo * C + 16 * j + 4 * g);
            }
        } else if constexpr (EPI == PMG_EPI_ROUT) {
            float p = 0.0f;
#pragma unroll
            for (int j = 0; j < NB; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) p = p + k.ow[16 * j + 4 * g + i] * y[j][i];
            const float d = a.out_b[0] + quad_sum(p);
            if (ok && g == 0) {
                if (a.points) {  // _refine_logz: logz + out (v3.py:359)
                    const float p0 = a.points[mo * 3 + 0], p1 = a.points[mo * 3 + 1], p2 = a.points[mo * 3 + 2];
                    float lz = p2 + d;
                    if (a.gate_lidar) {  // output gate: cur + g * (refined - cur) (v3.py:565-569)
                        const int HW = a.H * a.W;
                        const int b = (int)(mo / HW), pix = (int)(mo - (int64_t)b * HW);
                        const int i = pix / a.W, jj = pix - (pix / a.W) * a.W;
                        float ld, lc;
                        lidar_at(a.gate_lidar, a.gate_conf, b, i, jj, a.H, a.W, a.gate_dh, a.gate_dw, ld, lc);
                        const float gu = a.gate_floor + a.gate_scale * lidar_uncertainty(ld, lc);
                        lz = p2 + gu * (lz - p2);
                    }
                    a.points_out[mo * 3 + 0] = p0;
                    a.points_out[mo * 3 + 1] = p1;
                    a.points_out[mo * 3 + 2] = lz;
                } else {  // the refiner module's own output, (M, 1) (sparse_unet.py:258)
                    ((float*)a.out)[mo] = d;
                }
            }
        }
    }
}

template <typename T, int C, int EPI>
__global__ __launch_bounds__(kColThreads) void spconv_col_k(ColConvArgs a) {
    typedef ColGeom<T, C> G;
    constexpr int ROWB = G::ROWB, NCH = G::NCH, NB = C / 16, NBUF = G::NBUF;
    constexpr bool WLDS = G::WLDS;
    static_assert(NCH <= 4 || NCH % 4 == 0, "a tap's chunks must fill whole MFMA steps");
    typedef typename ColAcc<T>::type acc_t;

    __shared__ __attribute__((aligned(16))) uint8_t s_w[WLDS ? G::WBYTES : 16];
    __shared__ __attribute__((aligned(16))) uint8_t s_x[NBUF][G::XBYTES];
    __shared__ int s_z[NBUF][3 * kWin];
    __shared__ __attribute__((aligned(16))) uint8_t s_zero[16];  // operand of absent taps and padding lanes

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int M = (int)a.M;
    const int H = a.H, W = a.W;
    const int HW = H * W;
    const uint8_t* __restrict__ xg = (const uint8_t*)a.x;
    const uint8_t* __restrict__ wg = (const uint8_t*)a.w;

    if constexpr (WLDS) {
        for (int e = tid; e < G::WBYTES / 16; e += kColThreads) ((v4i*)s_w)[e] = ((const v4i*)wg)[e];
    }
    if (tid == 0) *(v4i*)s_zero = v4i{0, 0, 0, 0};

    // Window of segment `sg`: slice d in {0,1,2} holds voxels s0 + (d-1)*W - 1 + q, q in [0, kWin).
    v4i pf[G::PF];
    int pfz[G::PFZ];
    auto fetch = [&](int sg) {
        const int s0 = sg * kSeg;
#pragma unroll
        for (int k = 0; k < G::PF; ++k) {
            const int e = tid + k * kColThreads;
            pf[k] = v4i{0, 0, 0, 0};
            if (e < 3 * kWin * NCH) {
                const int d = e / (kWin * NCH);
                const int rem = e - d * (kWin * NCH);
                const int q = rem / NCH, c = rem - (rem / NCH) * NCH;
                const int p = s0 + (d - 1) * W - 1 + q;
                if (p >= 0 && p < M) pf[k] = *(const v4i*)(xg + (int64_t)p * ROWB + c * 16);
            }
        }
#pragma unroll
        for (int k = 0; k < G::PFZ; ++k) {
            const int e = tid + k * kColThreads;
            pfz[k] = kZFar;
            if (e < 3 * kWin) {
                const int d = e / kWin, q = e - (e / kWin) * kWin;
                const int p = s0 + (d - 1) * W - 1 + q;
                if (p >= 0 && p < M) pfz[k] = a.zq[p];
            }
        }
    };
    auto commit = [&](int buf) {
#pragma unroll
        for (int k = 0; k < G::PF; ++k) {
            const int e = tid + k * kColThreads;
            if (e < 3 * kWin * NCH) ((v4i*)s_x[buf])[e] = pf[k];
        }
#pragma unroll
        for (int k = 0; k < G::PFZ; ++k) {
            const int e = tid + k * kColThreads;
            if (e < 3 * kWin) s_z[buf][e] = pfz[k];
        }
    };

    // XCD-aware segment order (as spconv_colv_k): one contiguous band of segments per XCD (block b runs on XCD
    // b % 8), dealt round-robin to that XCD's blocks, so the image rows a band's windows share stay in its L2.
    const int nx = gridDim.x < 8 ? (int)gridDim.x : 8;
    const int xcd = (int)blockIdx.x % nx, ib = (int)blockIdx.x / nx;
    const int nbx = ((int)gridDim.x - xcd + nx - 1) / nx;
    const int nseg_all = (M + kSeg - 1) / kSeg;
    const int nseg = (int)((int64_t)nseg_all * (xcd + 1) / nx);  // end of this XCD's band
    int seg = (int)((int64_t)nseg_all * xcd / nx) + ib;
    if (seg < nseg) {
        fetch(seg);
        commit(0);
    }
    for (int it = 0; seg < nseg; seg += nbx, ++it) {
        const int buf = NBUF == 2 ? (it & 1) : 0;
        const int s0 = seg * kSeg;
        const int nxt = seg + nbx;
        __syncthreads();  // window `buf` (and the weights) visible to all waves
        if constexpr (NBUF == 2) {
            if (nxt < nseg) fetch(nxt);  // in flight during this segment's compute (issued after the barrier,
                                         // which waits for all outstanding memory operations)
        }

        // ---- 27-bit tap masks of the wave's 32 rows (lane l < 32 computes row l), branch-free
        uint32_t mk = 0;
        {
            const int lr = 32 * wv + (lane & 31);
            const int m = s0 + lr;
            if (lane < 32 && m < M) {
                const int pix = m % HW;
                const int i = pix / W, j = pix - (pix / W) * W;
                const int zc = s_z[buf][kWin + lr + 1];
#pragma unroll
                for (int di = 0; di < 3; ++di)
#pragma unroll
                    for (int dj = 0; dj < 3; ++dj) {
                        const bool in = (unsigned)(i + di - 1) < (unsigned)H && (unsigned)(j + dj - 1) < (unsigned)W;
                        const int64_t dz = (int64_t)s_z[buf][di * kWin + lr + dj] - zc;
                        const bool hit = in && dz >= -1 && dz <= 1;
                        mk |= (hit ? 1u : 0u) << (di * 9 + dj * 3 + (int)(dz + 1 < 0 ? 0 : (dz + 1 > 2 ? 2 : dz + 1)));
                    }
            }
        }
        uint32_t uni = mk;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) uni |= __shfl_xor(uni, o, 64);
        uni = sgpr(uni);
        const uint32_t mrow0 = __shfl(mk, r, 64), mrow1 = __shfl(mk, 16 + r, 64);

        // ---- reduction over (active tap, 16-byte chunk) units
        acc_t acc[2][NB];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int j = 0; j < NB; ++j) acc[rb][j] = acc_t{0, 0, 0, 0};

        const int lr0 = 32 * wv + r;  // window-relative row of this lane in row block 0
        // Operand addresses: lane-constant LDS byte offsets plus a wave-uniform (scalar) offset per tap. A lane whose
        // row lacks the tap, or whose chunk is padding (c >= NCH), reads the zero slot instead of branching.
        constexpr int SPT = NCH >= 4 ? NCH / 4 : 1;  // MFMA steps per tap (chunk 4s + g)
        constexpr int TPS = NCH >= 3 ? 1 : 4 / NCH;  // taps per MFMA step (slot g / NCH, chunk g % NCH)
        constexpr int WSTR = 16 * 27 * ROWB;         // byte distance between 16-channel weight blocks
        const int slot = TPS == 1 ? 0 : g / NCH;
        const int cl = TPS == 1 ? (g < NCH ? g : 0) : g - slot * NCH;  // chunk of this lane (step 0)
        const bool lane_on = TPS == 1 ? g < NCH || NCH >= 4 : true;
        const uint32_t mk0 = lane_on ? mrow0 : 0u, mk1 = lane_on ? mrow1 : 0u;
        typedef const __attribute__((address_space(3))) uint8_t* lds_ptr;
        const lds_ptr xbase = (lds_ptr)(s_x[buf]) + (lr0 * ROWB + cl * 16);
        const lds_ptr zslot = (lds_ptr)s_zero;
        const lds_ptr wbase = (lds_ptr)s_w + (WLDS ? r * 27 * ROWB + cl * 16 : 0);
        const uint8_t* wgl = wg + (r * 27 * ROWB + cl * 16);

        struct Ops {
            v4i x0, x1, w[NB];
        };
        // v: this lane's tap (wave-uniform when TPS == 1); st: step within the tap (wave-uniform)
        auto load = [&](int v, int st, Ops& o) {
            const int vv = v < 0 ? 0 : v;
            const int xo = ((vv / 9) * kWin + (vv / 3) % 3) * ROWB + st * 64;
            const bool h0 = v >= 0 && ((mk0 >> vv) & 1u);
            const bool h1 = v >= 0 && ((mk1 >> vv) & 1u);
            const lds_ptr p0 = h0 ? xbase + xo : zslot;
            const lds_ptr p1 = h1 ? xbase + (xo + 16 * ROWB) : zslot;
            o.x0 = *(const __attribute__((address_space(3))) v4i*)p0;
            o.x1 = *(const __attribute__((address_space(3))) v4i*)p1;
            const int wo = vv * ROWB + st * 64;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                if constexpr (WLDS)
                    o.w[j] = *(const __attribute__((address_space(3))) v4i*)(wbase + (wo + j * WSTR));
                else
                    o.w[j] = *(const v4i*)(wgl + (wo + j * WSTR));
            }
        };
        auto mma_all = [&](const Ops& o) {
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                mma_col(acc[0][j], o.w[j], o.x0, T{});
                mma_col(acc[1][j], o.w[j], o.x1, T{});
            }
        };
        // Scalar unit iterator over the active taps; after the last unit it yields v = -1 (zero operands), so the
        // operand loads of the next unit are issued unconditionally and the LDS wait counts stay static.
        uint32_t rem = uni;
        int cur_v = -1, cur_s = SPT;
        auto next = [&](int& v, int& st) {
            if constexpr (TPS == 1) {
                if (cur_s == SPT) {
                    cur_v = rem ? (int)__builtin_ctz(rem) : -1;
                    rem = rem ? rem & (rem - 1) : 0u;
                    cur_s = 0;
                }
                v = cur_v;
                st = cur_s++;
            } else {
                int vs[TPS];
#pragma unroll
                for (int k = 0; k < TPS; ++k) {
                    vs[k] = rem ? (int)__builtin_ctz(rem) : -1;
                    rem = rem ? rem & (rem - 1) : 0u;
                }
                int vl = vs[0];
#pragma unroll
                for (int k = 1; k < TPS; ++k) vl = slot == k ? vs[k] : vl;
                v = vl;
                st = 0;
            }
        };
        const int ntap = __builtin_popcount(uni);
        const int nunits = TPS == 1 ? ntap * SPT : (ntap + TPS - 1) / TPS;
        if (nunits > 0) {
            Ops A, B;
            int v, st;
            next(v, st);
            load(v, st, A);
            // sched_barrier keeps the next unit's operand loads ahead of the current unit's MFMAs, so LDS latency
            // overlaps the matrix work instead of being sunk next to its use.
            for (int k = 0;; k += 2) {
                next(v, st);
                load(v, st, B);
                __builtin_amdgcn_sched_barrier(0);
                mma_all(A);
                __builtin_amdgcn_sched_barrier(0);
                if (k + 1 >= nunits) break;
                next(v, st);
                load(v, st, A);
                __builtin_amdgcn_sched_barrier(0);
                mma_all(B);
                __builtin_amdgcn_sched_barrier(0);
                if (k + 2 >= nunits) break;
            }
        }

        // ---- epilogue
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            v4f sk[NB];
            if constexpr (EPI == PMG_EPI_R || EPI == PMG_EPI_RLN || EPI == PMG_EPI_ROUT)
                load_skip<C>(a, s0 + 32 * wv + 16 * rb + r, M, g, sk);
            col_epilogue<T, C, EPI>(a, acc[rb], s0 + 32 * wv + 16 * rb + r, M, g, epi_global(a), sk);
        }

        // ---- hand the next window to the other buffer (or, single-buffered, reload this one)
        if constexpr (NBUF == 2) {
            if (nxt < nseg) commit(buf ^ 1);
        } else {
            if (nxt < nseg) {
                fetch(nxt);
                __syncthreads();  // every wave is done reading this window
                commit(0);
            }
        }
    }
}

// Weights beyond LDS residency (int8 C = 128, fp16 C = 48 / 64: 124-442 KB): the taps staged, on 2-D tiles. A
// block takes tiles of WV image rows x 32 columns (wave w: row w, two 16-voxel MFMA tiles) and keeps the tile's
// window -- (WV + 2) x 34 pixels, codes and keys -- in LDS: 1.3 x the tile's pixels where a 256-voxel run of one
// image row needs a 3 x 258 window (2.3 x less window traffic), so two windows fit beside the staged weights and
// the next tile's window is loaded during this tile's taps and epilogue. The block walks the union of its waves'
// active taps in ascending order; each tap's weights (C x 27 x Ci -> C x Ci) are staged once per block into LDS in
// MFMA operand order -- lane (r, g) of fragment (s, j) holds W[16j + r][v][chunk 4s + g], zero where 4s + g is
// past the row (the K padding of C = 48 in fp16) -- and feed all the waves. Tap t + 1's weights are written while
// tap t's MFMAs run (two LDS buffers, one barrier per tap); their global loads are issued two taps ahead, and the
// next window right after the tile's last weight load (the memory counter completes in order, so a window
// requested earlier would hold every later weight store behind it). A wave whose rows lack a tap skips its MFMAs.
template <typename T, int C, int EPI, int WV>
__global__ __launch_bounds__(64 * WV) void spconv_cols_k(ColConvArgs a) {
    constexpr int kThreads = 64 * WV;
    constexpr int TC = 32, WR = WV + 2, WC = TC + 2, WPIX = WR * WC;  // tile columns; window rows, columns
    constexpr int ROWB = C * (int)sizeof(T), NCH = ROWB / 16, NB = C / 16;
    constexpr int XBYTES = WPIX * ROWB;
    constexpr int PF = (WPIX * NCH + kThreads - 1) / kThreads;  // window chunks per thread
    constexpr int PFZ = (WPIX + kThreads - 1) / kThreads;       // window keys per thread
    constexpr int SPT = (NCH + 3) / 4;       // MFMA steps per tap; lane group g of step s takes chunk 4s + g
    constexpr int FR = SPT * NB;             // 1 KB operand fragments per tap
    constexpr int WPT = (FR * 64 + kThreads - 1) / kThreads;  // staged 16-byte pieces per thread per tap
    constexpr bool kPre = NB <= 4;
    typedef typename ColAcc<T>::type acc_t;
    static_assert(2 * XBYTES + 2 * FR * 1024 + 2 * WPIX * 4 + 64 <= 160 * 1024, "two windows and two taps must fit LDS");

    __shared__ __attribute__((aligned(16))) v4i s_w[2][FR * 64];
    __shared__ __attribute__((aligned(16))) uint8_t s_x[2][XBYTES];
    __shared__ int s_z[2][WPIX];
    __shared__ __attribute__((aligned(16))) uint8_t s_zero[16];
    __shared__ uint32_t s_uni[WV];

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int M = (int)a.M;
    const int H = a.H, W = a.W;
    const int HW = H * W;
    const int th = (H + WV - 1) / WV, tw = (W + TC - 1) / TC;  // tiles per frame: th x tw
    const uint8_t* __restrict__ xg = (const uint8_t*)a.x;
    const uint8_t* __restrict__ wg = (const uint8_t*)a.w;
    if (tid == 0) *(v4i*)s_zero = v4i{0, 0, 0, 0};

    // staged weights of tap v (v < 0: none) into registers; piece e = tid + k * kThreads is lane e % 64 of
    // fragment f = e / 64 = s * NB + j
    auto w_load = [&](int v, v4i (&st)[WPT]) {
#pragma unroll
        for (int k = 0; k < WPT; ++k) {
            const int e = tid + k * kThreads;
            const int f = e >> 6, l = e & 63;
            const int s2 = f / NB, j = f - (f / NB) * NB;
            const int ch = 4 * s2 + (l >> 4);
            st[k] = v4i{0, 0, 0, 0};
            if (v >= 0 && e < FR * 64 && ch < NCH)
                st[k] = *(const v4i*)(wg + ((int64_t)(16 * j + (l & 15)) * 27 + v) * ROWB + ch * 16);
        }
    };
    auto w_store = [&](int buf, const v4i (&st)[WPT]) {
#pragma unroll
        for (int k = 0; k < WPT; ++k) {
            const int e = tid + k * kThreads;
            if (e < FR * 64) s_w[buf][e] = st[k];
        }
    };

    // tile t of the batch: frame b, image rows i0 .. i0 + WV - 1, columns j0 .. j0 + TC - 1
    auto tile_origin = [&](int t, int& b, int& i0, int& j0) {
        b = t / (th * tw);
        const int q = t - b * (th * tw);
        i0 = (q / tw) * WV;
        j0 = (q - (q / tw) * tw) * TC;
    };
    // Window of tile t: slot (wr, wc) holds pixel (i0 - 1 + wr, j0 - 1 + wc) of the frame; slots outside the frame
    // hold zero codes and a key no voxel matches. Rows of 34 pixels are contiguous in memory (coalesced loads).
    v4i pf[PF];
    int pfz[PFZ];
    auto fetch = [&](int t) {
        int b, i0, j0;
        tile_origin(t, b, i0, j0);
        const int64_t fb = (int64_t)b * HW;
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            const int e = tid + k * kThreads;
            pf[k] = v4i{0, 0, 0, 0};
            if (e < WPIX * NCH) {
                const int px = e / NCH, c = e - (e / NCH) * NCH;
                const int i = i0 - 1 + px / WC, j = j0 - 1 + (px - (px / WC) * WC);
                if ((unsigned)i < (unsigned)H && (unsigned)j < (unsigned)W)
                    pf[k] = *(const v4i*)(xg + (fb + (int64_t)i * W + j) * ROWB + c * 16);
            }
        }
#pragma unroll
        for (int k = 0; k < PFZ; ++k) {
            const int e = tid + k * kThreads;
            pfz[k] = kZFar;
            if (e < WPIX) {
                const int i = i0 - 1 + e / WC, j = j0 - 1 + (e - (e / WC) * WC);
                if ((unsigned)i < (unsigned)H && (unsigned)j < (unsigned)W) pfz[k] = a.zq[fb + (int64_t)i * W + j];
            }
        }
    };
    auto commit = [&](int buf) {
#pragma unroll
        for (int k = 0; k < PF; ++k) {
            const int e = tid + k * kThreads;
            if (e < WPIX * NCH) ((v4i*)s_x[buf])[e] = pf[k];
        }
#pragma unroll
        for (int k = 0; k < PFZ; ++k) {
            const int e = tid + k * kThreads;
            if (e < WPIX) s_z[buf][e] = pfz[k];
        }
    };

    // XCD-aware tile order: one contiguous band of tiles (raster order) per XCD (block b runs on XCD b % 8), dealt
    // round-robin to that XCD's blocks, so the rows and columns neighbouring tiles share stay in its L2.
    const int nx = gridDim.x < 8 ? (int)gridDim.x : 8;
    const int xcd = (int)blockIdx.x % nx, ib = (int)blockIdx.x / nx;
    const int nbx = ((int)gridDim.x - xcd + nx - 1) / nx;
    const int ntile = (M / HW) * th * tw;  // M = frames x H x W
    const int tend = (int)((int64_t)ntile * (xcd + 1) / nx);  // end of this XCD's band
    int tile = (int)((int64_t)ntile * xcd / nx) + ib;
    if (tile < tend) {
        fetch(tile);
        commit(0);
    }
    typedef const __attribute__((address_space(3))) uint8_t* lds_ptr;
    typedef const __attribute__((address_space(3))) v4i lds_v4i;
    for (int it = 0; tile < tend; tile += nbx, ++it) {
        const int xb = it & 1;  // this tile's window buffer
        const int nxt = tile + nbx;
        int b, i0, j0;
        tile_origin(tile, b, i0, j0);
        __syncthreads();  // window visible; every wave has left the previous tile's window and weight buffers
        const uint8_t* const sx = s_x[xb];
        const int* const sz = s_z[xb];

        // ---- 27-bit tap masks of the wave's 32 voxels (lane l < 32: column l of row wv), the wave's union and the
        // block's
        const int i = i0 + wv;
        uint32_t mk = 0;
        {
            const int lr = lane & 31;
            const int j = j0 + lr;
            if (lane < 32 && i < H && j < W) {
                const int zc = sz[(wv + 1) * WC + lr + 1];
#pragma unroll
                for (int di = 0; di < 3; ++di)
#pragma unroll
                    for (int dj = 0; dj < 3; ++dj) {
                        const bool in = (unsigned)(i + di - 1) < (unsigned)H && (unsigned)(j + dj - 1) < (unsigned)W;
                        const int64_t dz = (int64_t)sz[(wv + di) * WC + lr + dj] - zc;
                        const bool hit = in && dz >= -1 && dz <= 1;
                        mk |= (hit ? 1u : 0u) << (di * 9 + dj * 3 + (int)(dz + 1 < 0 ? 0 : (dz + 1 > 2 ? 2 : dz + 1)));
                    }
            }
        }
        uint32_t uni = mk;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) uni |= __shfl_xor(uni, o, 64);
        uni = sgpr(uni);
        const uint32_t mrow0 = __shfl(mk, r, 64), mrow1 = __shfl(mk, 16 + r, 64);
        if (lane == 0) s_uni[wv] = uni;
        __syncthreads();
        uint32_t bu = 0;
#pragma unroll
        for (int w2 = 0; w2 < WV; ++w2) bu |= s_uni[w2];
        bu = sgpr(bu);

        acc_t acc[2][NB];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int j = 0; j < NB; ++j) acc[rb][j] = acc_t{0, 0, 0, 0};

        // operand addresses: lane-constant LDS offsets plus a wave-uniform offset per (tap, step); a lane whose
        // voxel lacks the tap, or whose chunk is padding, reads the zero slot. Window slot of the neighbour (di, dj)
        // of column c of row wv: (wv + di) * WC + c + dj.
        const lds_ptr xbase = (lds_ptr)sx + ((wv * WC + r) * ROWB + g * 16);
        const lds_ptr zslot = (lds_ptr)s_zero;

        // tap sequence: ascending bits of bu, -1 after the last
        uint32_t rem = bu;
        auto pop = [&]() {
            const int v = rem ? (int)__builtin_ctz(rem) : -1;
            rem = rem ? rem & (rem - 1) : 0u;
            return v;
        };
        const int ntap = __builtin_popcount(bu);
        int v0 = pop(), v1 = pop(), v2 = pop();
        v4i wa[WPT], wb[WPT];
        w_load(v0, wa);
        w_load(v1, wb);
        w_store(0, wa);
        __syncthreads();

        // (the next window is requested during the taps up to 64 output channels; beyond, the registers of its
        // pieces would spill, and it is requested after the epilogue)
        bool fetched = nxt >= tend || !kPre;
        auto tap = [&](int buf, int v, const v4i (&wnext)[WPT], v4i (&wlater)[WPT], int vlater) {
            // the weights two taps ahead are requested before this tap's matrix work
            w_load(vlater, wlater);
            if (!fetched && vlater < 0) {
                fetch(nxt);
                fetched = true;
            }
            if ((uni >> v) & 1u) {
                const int xo = ((v / 9) * WC + (v / 3) % 3) * ROWB;
                const bool h0 = (mrow0 >> v) & 1u, h1 = (mrow1 >> v) & 1u;
                // every operand of the tap is requested before its first MFMA (LDS returns in order, so the MFMAs
                // of step 0 wait only for step 0's reads)
                v4i x0[SPT], x1[SPT], wo[SPT][NB];
#pragma unroll
                for (int s2 = 0; s2 < SPT; ++s2) {
                    const bool on = 4 * s2 + g < NCH;
                    const lds_ptr p0 = h0 && on ? xbase + (xo + s2 * 64) : zslot;
                    const lds_ptr p1 = h1 && on ? xbase + (xo + 16 * ROWB + s2 * 64) : zslot;
                    x0[s2] = *(const __attribute__((address_space(3))) v4i*)p0;
                    x1[s2] = *(const __attribute__((address_space(3))) v4i*)p1;
#pragma unroll
                    for (int j = 0; j < NB; ++j) wo[s2][j] = *(lds_v4i*)(&s_w[buf][(s2 * NB + j) * 64 + lane]);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int s2 = 0; s2 < SPT; ++s2)
#pragma unroll
                    for (int j = 0; j < NB; ++j) {
                        mma_col(acc[0][j], wo[s2][j], x0[s2], T{});
                        mma_col(acc[1][j], wo[s2][j], x1[s2], T{});
                    }
                __builtin_amdgcn_sched_barrier(0);
            }
            w_store(buf ^ 1, wnext);
            __syncthreads();
        };
        // two taps per trip so the buffer and register-set indices are compile-time
        for (int t = 0; t < ntap; t += 2) {
            tap(0, v0, wb, wa, v2);
            v0 = v1;
            v1 = v2;
            v2 = pop();
            if (t + 1 >= ntap) break;
            tap(1, v0, wa, wb, v2);
            v0 = v1;
            v1 = v2;
            v2 = pop();
        }

        if (kPre && !fetched) fetch(nxt);  // at most two taps: every weight load came before the loop

        // ---- epilogue: voxel of row wv, column 16 rb + r (M: outside the frame, nothing stored)
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            const int j = j0 + 16 * rb + r;
            const int m = i < H && j < W ? b * HW + i * W + j : M;
            v4f sk[NB];
            if constexpr (EPI == PMG_EPI_R || EPI == PMG_EPI_RLN || EPI == PMG_EPI_ROUT) load_skip<C>(a, m, M, g, sk);
            col_epilogue<T, C, EPI>(a, acc[rb], m, M, g, epi_global(a), sk);
        }

        // ---- the next tile's window into the other buffer (every wave left it before this tile began)
        if (nxt < tend) {
            if constexpr (!kPre) fetch(nxt);
            commit(xb ^ 1);
        }
    }
}

template <typename T, int C, int EPI>
static int launch_col3(const ColConvArgs& a, hipStream_t s) {
    if constexpr (!ColGeom<T, C>::FITS) {
        return fail(PMG_E_INVALID, "pmg_spconv_col: this precision/width does not fit the LDS window");
    } else {
        const int64_t nseg = (a.M + kSeg - 1) / kSeg;
        if constexpr (!ColGeom<T, C>::WLDS) {
            // 8-wave blocks of 8 x 32-voxel tiles, one per CU (LDS)
            constexpr int WV = 8;
            const int64_t HW = (int64_t)a.H * a.W;
            const int64_t nseg4 = (a.M / HW) * ((a.H + WV - 1) / WV) * ((a.W + 31) / 32);
            static int per_cu = -1;
            if (per_cu < 0) {
                int n = 0;
                if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, spconv_cols_k<T, C, EPI, WV>, 64 * WV, 0) !=
                        hipSuccess ||
                    n < 1)
                    n = 1;
                per_cu = n;
            }
            int64_t grid = (int64_t)per_cu * num_cus();
            if (grid > nseg4) grid = nseg4;
            hipLaunchKernelGGL((spconv_cols_k<T, C, EPI, WV>), dim3((unsigned)grid), dim3(64 * WV), 0, s, a);
            return check_launch("spconv_cols_k");
        } else {
            static int per_cu = -1;
            if (per_cu < 0) {
                int n = 0;
                if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, spconv_col_k<T, C, EPI>, kColThreads, 0) !=
                        hipSuccess ||
                    n < 1)
                    n = 1;
                per_cu = n;
            }
            int64_t grid = (int64_t)per_cu * num_cus();
            if (grid > nseg) grid = nseg;
            hipLaunchKernelGGL((spconv_col_k<T, C, EPI>), dim3((unsigned)grid), dim3(kColThreads), 0, s, a);
            return check_launch("spconv_col_k");
        }
    }
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

// ---------------------------------------------------------------------------------------------------------------
// int8, C <= 64: neighbour-pixel-major reduction, two wave groups in ping-pong.
//
// A persistent block holds two groups of WG waves (WG = 4: one wave of each group per SIMD). Each group owns its own
// LDS window buffer and walks its own segments of 16 * TT * WG voxels (16 * TT rows per wave in TT 16-row tiles). The
// groups run half a period apart: while one group's waves issue the matrix work of a segment (after the global
// loads of their next window and, where registers allow, of the segment's residual inputs), the other group's
// waves (on the same SIMDs) write their next window to LDS and run the previous segment's epilogue. Every half
// period ends at one block barrier (LDS waits only; global stores are not waited for), so the MFMA pipe and the
// VALU of a SIMD are busy at the same time instead of in turn.
//
// Matrix work of a segment. At level 0 a row's neighbour at pixel offset (di, dj) is at most one of the three taps
// (di, dj, dz), dz = key_nb - key_row, and the centre offset holds only the row itself (one voxel per pixel). So the
// reduction runs over K = 8 offsets x 3 taps x C + C instead of 27 x C: the four lane groups of an MFMA operand
// (16 K-values each) take four different offsets -- group G = 0 takes offsets 0..3, G = 1 offsets 5..8 -- and one
// MFMA step covers (tap dz, channel chunk c) of all four: lane group g supplies chunk c of its offset's neighbour
// row, or zeros unless that neighbour's dz is the step's. Per 16-channel output block that is 6 * C/16 + 1 steps
// (the first one the centre tap, lane groups >= C/16 zero) instead of 27 with up to 75 % K padding: 19 instead of
// 27 MFMAs at C = 48, 13 at C = 32. A lane reads its step operand per tile straight from LDS, from its neighbour row
// or, when that neighbour is not the step's tap, from a 16-byte zero slot (one address select instead of zeroing
// four registers: the matrix phase shares its SIMD's VALU with the other group's epilogue). The weights of a step
// are one conflict-free 16-byte read per lane from LDS, laid out in the MFMA operand order; both operands are read
// two steps ahead, and each weight read feeds the TT tiles' MFMAs.
// The weights stay in LDS for the whole block; per-channel epilogue constants are staged in LDS too, so the
// epilogue issues no dependent global loads.
template <int C, int TT, int WG>
struct ColvGeom {
    static constexpr int kThreads = 128 * WG;       // two groups
    static constexpr int kGroupThreads = 64 * WG;
    static constexpr int kRows = 16 * TT;           // rows per wave
    static constexpr int kSeg = kRows * WG;         // rows per segment (one group)
    static constexpr int kWin = kSeg + 2;
    static constexpr int ROWB = C;
    static constexpr int NCH = C / 16;
    static constexpr int NB = C / 16;
    static constexpr int XBYTES = 3 * kWin * ROWB;
    static constexpr int ZWORDS = 3 * kWin;
    static constexpr int NSTEP = 6 * NCH + 1;       // MFMA steps per 16-channel output block
    static constexpr int WBYTES = NSTEP * NB * 1024;  // one 64-lane x 16-byte operand per (step, block)
    static constexpr int NCHUNK = 3 * kWin * NCH;
    static constexpr int PF = (NCHUNK + kGroupThreads - 1) / kGroupThreads;  // window chunks per thread
    static constexpr int PFZ = (ZWORDS + kGroupThreads - 1) / kGroupThreads;  // window keys per thread
    static constexpr int LDS = WBYTES + 2 * XBYTES + 2 * ZWORDS * 4 + 5 * C * 4 + 7 * C * 4;  // (+ x0 constants)
};

// X0: the residual epilogue's skip is the first block's h, recomputed per row (x0_load / x0_skip) instead of read.
template <int C, int EPI, int TT, int WG, bool X0>
__global__ __launch_bounds__(128 * WG, 1) void spconv_colv_k(ColConvArgs a) {
    typedef ColvGeom<C, TT, WG> G;
    constexpr int kRows = G::kRows, kSeg = G::kSeg, kWin = G::kWin, GT = G::kGroupThreads;
    constexpr int ROWB = G::ROWB, NCH = G::NCH, NB = G::NB;
    static_assert(C == 16 || C == 32 || C == 48 || C == 64, "this kernel covers C <= 64");
    static_assert(G::LDS <= 160 * 1024, "weights and two windows must fit the 160 KB of LDS");

    __shared__ __attribute__((aligned(16))) uint8_t s_w[G::WBYTES];
    __shared__ __attribute__((aligned(16))) uint8_t s_x[2][G::XBYTES];
    __shared__ int s_z[2][G::ZWORDS];
    __shared__ float s_k[5][C];  // w_scale, bias, ln gamma, ln beta, out_w
    __shared__ __attribute__((aligned(16))) float s_x0[X0 ? 7 * C : 4];  // in_w [C][3], in_b, pr_w [C][2], pr_b
    __shared__ __attribute__((aligned(16))) v4i s_zx;  // the operand of a neighbour that is not the step's tap

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int grp = wv / WG, wq = wv - grp * WG, gtid = tid - grp * GT;
    const int r = lane & 15, g = lane >> 4;
    const int gc = g < NCH ? g : NCH - 1;  // chunk read by this lane; lanes g >= NCH are zeroed (K padding)
    const bool kin = g < NCH;
    const int M = (int)a.M;
    const int H = a.H, W = a.W;
    const int HW = H * W;
    const uint8_t* __restrict__ xg = (const uint8_t*)a.x;
    const uint8_t* __restrict__ wg = (const uint8_t*)a.w;

    // weights: operand (step st, block j) at ((st * NB + j) * 64 + lane) * 16. Step 1 + (G * 3 + d) * NCH + c, lane
    // (r, q): W[16j + r][tap 3 * (5G + q) + d][chunk c]; step 0 (centre), lane (r, q): W[16j + r][13][chunk q],
    // zero for q >= NCH. All of a thread's loads are issued before its first LDS store.
    constexpr int WCH = G::NSTEP * NB * 64, WPT = (WCH + G::kThreads - 1) / G::kThreads;
    v4i wtmp[WPT];
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        const int e = tid + k * G::kThreads;
        const int rr = e % 16, q = (e / 16) % 4, sj = e / 64;
        const int st = sj / NB, j = sj - (sj / NB) * NB;
        const int u = st - 1, gi = u / (3 * NCH), d = (u / NCH) % 3, c = u % NCH;
        const int v = st == 0 ? 13 : 3 * (5 * gi + q) + d, ch = st == 0 ? q : c;
        const bool ok = e < WCH && (st > 0 || q < NCH);
        wtmp[k] = ok ? *(const v4i*)(wg + ((int64_t)(16 * j + rr) * 27 + v) * ROWB + 16 * ch) : v4i{0, 0, 0, 0};
    }
    for (int e = tid; e < 5 * C; e += G::kThreads) {
        const int q = e / C, n = e - (e / C) * C;
        const float* src = q == 0 ? a.w_scale : q == 1 ? a.bias : q == 2 ? a.ln_gamma : q == 3 ? a.ln_beta : a.out_w;
        s_k[q][n] = src ? src[n] : 0.0f;
    }
    if constexpr (X0) {
        const bool pr = a.x0_rg != nullptr;
        for (int e = tid; e < 7 * C; e += G::kThreads)
            s_x0[e] = e < 3 * C ? a.x0_in_w[e]
                      : e < 4 * C ? a.x0_in_b[e - 3 * C]
                      : !pr       ? 0.0f
                      : e < 6 * C ? a.x0_pr_w[e - 4 * C]
                                  : a.x0_pr_b[e - 6 * C];
    }
    typedef const __attribute__((address_space(3))) float* kptr;
    const EpiConst<kptr> kc{(kptr)s_k[0], (kptr)s_k[1], (kptr)s_k[2], (kptr)s_k[3], (kptr)s_k[4], a.bias != nullptr};

    // window of segment sg: slice d in {0,1,2} holds voxels s0 + (d-1)*W - 1 + q, q in [0, kWin); loaded by the
    // group's threads into registers, then written to the group's LDS buffer
    v4i pf[G::PF];
    int pfz[G::PFZ];
    auto fetch = [&](int sg) {
        const int s0 = sg * kSeg;
#pragma unroll
        for (int k = 0; k < G::PF; ++k) {
            const int e = gtid + k * GT;
            pf[k] = v4i{0, 0, 0, 0};
            if (e < G::NCHUNK) {
                const int d = e / (kWin * NCH);
                const int rem = e - d * (kWin * NCH);
                const int q = rem / NCH, c = rem - (rem / NCH) * NCH;
                const int p = s0 + (d - 1) * W - 1 + q;
                if (p >= 0 && p < M) pf[k] = *(const v4i*)(xg + (int64_t)p * ROWB + c * 16);
            }
        }
#pragma unroll
        for (int k = 0; k < G::PFZ; ++k) {
            const int e = gtid + k * GT;
            pfz[k] = kZFar;
            if (e < G::ZWORDS) {
                const int d = e / kWin, q = e - (e / kWin) * kWin;
                const int p = s0 + (d - 1) * W - 1 + q;
                if (p >= 0 && p < M) pfz[k] = a.zq[p];
            }
        }
    };
    uint8_t* const xbuf = s_x[grp];
    int* const zbuf = s_z[grp];
    auto commit = [&]() {
#pragma unroll
        for (int k = 0; k < G::PF; ++k) {
            const int e = gtid + k * GT;
            if (e < G::NCHUNK) ((v4i*)xbuf)[e] = pf[k];
        }
#pragma unroll
        for (int k = 0; k < G::PFZ; ++k) {
            const int e = gtid + k * GT;
            if (e < G::ZWORDS) zbuf[e] = pfz[k];
        }
    };

    typedef const __attribute__((address_space(3))) uint8_t lds_u8;
    typedef const __attribute__((address_space(3))) v4i lds_v4i;
    typedef const __attribute__((address_space(3))) int lds_int;
    const int lr0 = kRows * wq + r;  // window-relative row of tile 0
    // this lane's pixel offset in group G: o = 5G + g, (di, dj) = (o / 3, o % 3); window row of the neighbour of
    // local row lr: di * kWin + lr + dj
    const int o0 = g, o1 = 5 + g;
    const int ri0 = o0 / 3 - 1, rj0 = o0 % 3 - 1, ri1 = o1 / 3 - 1, rj1 = o1 % 3 - 1;
    const lds_u8* xg0 = (lds_u8*)xbuf + (lr0 + (o0 / 3) * kWin + o0 % 3) * ROWB;
    const lds_u8* xg1 = (lds_u8*)xbuf + (lr0 + (o1 / 3) * kWin + o1 % 3) * ROWB;
    const lds_int* zg0 = (lds_int*)zbuf + lr0 + (o0 / 3) * kWin + o0 % 3;
    const lds_int* zg1 = (lds_int*)zbuf + lr0 + (o1 / 3) * kWin + o1 % 3;
    const lds_u8* xcb = (lds_u8*)xbuf + (lr0 + kWin + 1) * ROWB + gc * 16;  // the row itself, chunk g
    const lds_int* zcb = (lds_int*)zbuf + lr0 + kWin + 1;
    const lds_u8* wb = (lds_u8*)s_w + lane * 16;

    // this group's segments: first, first + stride, ...; group 0 has at least as many as group 1. XCD-aware: block
    // b runs on XCD b % 8 (workgroups are dispatched round-robin over the XCDs), and the segments -- consecutive
    // pixels in raster order -- are split into one contiguous band per XCD, dealt round-robin to that XCD's groups.
    // A segment's window reads the image rows above and below it too, i.e. rows of neighbouring segments of the
    // same band, so each row comes from HBM about once into its XCD's L2 instead of once per XCD that reads it.
    const int nseg = (M + kSeg - 1) / kSeg;
    const int nx = gridDim.x < 8 ? (int)gridDim.x : 8;
    const int xcd = (int)blockIdx.x % nx, ib = (int)blockIdx.x / nx;
    const int nbx = ((int)gridDim.x - xcd + nx - 1) / nx;  // blocks on this XCD
    const int seg_lo = (int)((int64_t)nseg * xcd / nx), seg_hi = (int)((int64_t)nseg * (xcd + 1) / nx);
    const int stride = 2 * nbx;
    const int first = seg_lo + 2 * ib + grp;
    const int nk = first < seg_hi ? (seg_hi - 1 - first) / stride + 1 : 0;
    const int first0 = seg_lo + 2 * ib;
    const int nk0 = first0 < seg_hi ? (seg_hi - 1 - first0) / stride + 1 : 0;

    if (nk > 0) fetch(first);
#pragma unroll
    for (int k = 0; k < WPT; ++k) {
        const int e = tid + k * G::kThreads;
        if (e < WCH) ((v4i*)s_w)[e] = wtmp[k];
    }
    if (nk > 0) commit();
    if (tid == 0) s_zx = v4i{0, 0, 0, 0};
    __syncthreads();  // weights, constants, the zero slot and both groups' first windows visible

    constexpr bool kRes = EPI == PMG_EPI_R || EPI == PMG_EPI_RLN || EPI == PMG_EPI_ROUT;
    constexpr bool kSkipEarly = TT * NB <= 8;  // else the residual inputs would not fit in registers beside the MFMAs
    v4i acc[TT][NB];
    v4f sk[TT][NB];      // residual inputs of the segment in flight
    float x0in[TT][5];   // (X0) the rows' level-0 inputs, from which the epilogue forms sk
    // Half periods: group 0 runs M0 E0 M1 E1 ..., group 1 runs - M0 E0 M1 E1 ... (Mk: loads of window k+1 and of
    // segment k's residual inputs issued, then the matrix work of segment k; Ek: window k+1 written to LDS, then
    // the epilogue of segment k; -: idle). The global loads thus have a whole half period to arrive. Both groups
    // walk 2 * nk0 + 1 half periods, each ended by a barrier, so the barrier counts match.
    const int steps = 2 * nk0 + 1;
    for (int step = 0, hp = -grp; step < steps; ++step, ++hp) {
        const int kk = hp >> 1;
        if (hp < 0) {
        } else if ((hp & 1) == 0) {
            if (kk < nk) {
                const int s0 = (first + kk * stride) * kSeg;
                // (X0: the rows' inputs are requested before the next window, so that forming the skip after the
                // matrix work waits for them only)
                if constexpr (kRes && kSkipEarly && X0) {
#pragma unroll
                    for (int t = 0; t < TT; ++t) x0_load(a, s0 + kRows * wq + 16 * t + r, M, x0in[t]);
                }
                if (kk + 1 < nk) fetch(first + (kk + 1) * stride);
                if constexpr (kRes && kSkipEarly && !X0) {
#pragma unroll
                    for (int t = 0; t < TT; ++t) load_skip<C>(a, s0 + kRows * wq + 16 * t + r, M, g, sk[t]);
                }
                int zc[TT], pi[TT], pj[TT];
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    const int m = s0 + kRows * wq + 16 * t + r;
                    const int pix = (m < M ? m : 0) % HW;
                    pi[t] = pix / W;
                    pj[t] = pix - pi[t] * W;
                    zc[t] = zcb[16 * t];
                }
#pragma unroll
                for (int t = 0; t < TT; ++t)
#pragma unroll
                    for (int j = 0; j < NB; ++j) acc[t][j] = v4i{0, 0, 0, 0};

                // Straight-line over the NSTEP steps, software-pipelined (see above).
                constexpr int NSTEP = G::NSTEP;
                auto load_w = [&](int st, v4i (&w)[NB]) {  // st compile-time after unrolling
#pragma unroll
                    for (int j = 0; j < NB; ++j) w[j] = *(lds_v4i*)(wb + (st * NB + j) * 1024);
                };
                v4i Wt[3][NB];
                // Each step's codes are read from LDS per tile, two steps ahead like the weights: the lane's offset
                // row, chunk c, when that neighbour is the step's tap dz, else the zero slot -- one address select
                // per tile and step instead of zeroing 16 bytes (4 selects) per tile and step.
                int dzg[2][TT];
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    const int z0 = zg0[16 * t], z1 = zg1[16 * t];
                    const bool in0 = (unsigned)(pi[t] + ri0) < (unsigned)H && (unsigned)(pj[t] + rj0) < (unsigned)W;
                    const bool in1 = (unsigned)(pi[t] + ri1) < (unsigned)H && (unsigned)(pj[t] + rj1) < (unsigned)W;
                    dzg[0][t] = in0 ? z0 - zc[t] + 1 : 3;  // 0, 1, 2: tap dz - 1; anything else: none
                    dzg[1][t] = in1 ? z1 - zc[t] + 1 : 3;
                }
                const lds_u8* zs = (lds_u8*)&s_zx;
                auto load_x = [&](int st, v4i (&xm)[TT]) {  // st compile-time after unrolling
#pragma unroll
                    for (int t = 0; t < TT; ++t) {
                        const lds_u8* p;
                        if (st == 0) {  // the centre: the row itself, lanes g >= NCH are K padding
                            p = kin ? xcb + 16 * t * ROWB : zs;
                        } else {
                            const int u = st - 1, gi = u / (3 * NCH), d = (u / NCH) % 3, c = u % NCH;
                            p = dzg[gi][t] == d ? (gi == 0 ? xg0 : xg1) + (16 * t * ROWB + 16 * c) : zs;
                        }
                        xm[t] = *(lds_v4i*)p;
                    }
                };
                v4i XM[3][TT];
                load_w(0, Wt[0]);
                load_x(0, XM[0]);
                load_w(1, Wt[1]);
                load_x(1, XM[1]);
#pragma unroll
                for (int st = 0; st < NSTEP; ++st) {
                    if (st + 2 < NSTEP) {
                        load_w(st + 2, Wt[(st + 2) % 3]);
                        load_x(st + 2, XM[(st + 2) % 3]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int j = 0; j < NB; ++j)
#pragma unroll
                        for (int t = 0; t < TT; ++t)
                            acc[t][j] =
                                __builtin_amdgcn_mfma_i32_16x16x64_i8(Wt[st % 3][j], XM[st % 3][t], acc[t][j], 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                }
                // (X0) the skip is formed here, after the matrix work is issued: the epilogue half, which sets the
                // period of the residual epilogues, keeps only the work it had with a loaded skip
                if constexpr (kRes && kSkipEarly && X0) {
#pragma unroll
                    for (int t = 0; t < TT; ++t) x0_skip<C, kptr>((kptr)s_x0, a.x0_rg != nullptr, x0in[t], g, sk[t]);
                }
            }
        } else if (kk < nk) {
            const int s0 = (first + kk * stride) * kSeg;
            if constexpr (kRes && !kSkipEarly) {
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    if constexpr (X0)
                        x0_load(a, s0 + kRows * wq + 16 * t + r, M, x0in[t]);
                    else
                        load_skip<C>(a, s0 + kRows * wq + 16 * t + r, M, g, sk[t]);
                }
            }
            if (kk + 1 < nk) commit();  // this group's matrix work on its window ended at the last barrier
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                if constexpr (kRes && !kSkipEarly && X0) x0_skip<C, kptr>((kptr)s_x0, a.x0_rg != nullptr, x0in[t], g, sk[t]);
                col_epilogue<int8_t, C, EPI, kptr>(a, acc[t], s0 + kRows * wq + 16 * t + r, M, g, kc, sk[t]);
            }
        }
        __syncthreads();
    }
}

// Rows on the critical path (the most segments either group of a block walks, times the segment size).
static int64_t colv_span(int64_t M, int64_t blocks_max, int seg) {
    const int64_t nseg = (M + seg - 1) / seg;
    const int64_t blocks = (nseg + 1) / 2 < blocks_max ? (nseg + 1) / 2 : blocks_max;
    return (nseg + 2 * blocks - 1) / (2 * blocks) * seg;
}

template <int C, int EPI, int TT, int WG>
static int launch_colv_tt(const ColConvArgs& a, hipStream_t s) {
    typedef ColvGeom<C, TT, WG> G;
    const int64_t nseg = (a.M + G::kSeg - 1) / G::kSeg;
    const int64_t cus = num_cus();
    const unsigned grid = (unsigned)((nseg + 1) / 2 < cus ? (nseg + 1) / 2 : cus);
    if constexpr (EPI == PMG_EPI_RLN) {
        if (a.x0_feats) {
            hipLaunchKernelGGL((spconv_colv_k<C, EPI, TT, WG, true>), dim3(grid), dim3(G::kThreads), 0, s, a);
            return check_launch("spconv_colv_k");
        }
    }
    hipLaunchKernelGGL((spconv_colv_k<C, EPI, TT, WG, false>), dim3(grid), dim3(G::kThreads), 0, s, a);
    return check_launch("spconv_colv_k");
}

template <int C, int EPI>
static int launch_colv(const ColConvArgs& a, hipStream_t s) {
    // the largest TT (tiles per wave) whose span is within 1/16 of the best: larger segments amortise the window
    // halo and feed each LDS weight read to more tiles. Registers allow TT = 4 up to C = 32, TT = 2 up to C = 48.
    constexpr int WG = 4;
    const int64_t cus = num_cus();
    const int64_t s4 = C <= 32 ? colv_span(a.M, cus, 64 * WG) : INT64_MAX;
    const int64_t s2 = C <= 48 ? colv_span(a.M, cus, 32 * WG) : INT64_MAX;
    const int64_t s1 = colv_span(a.M, cus, 16 * WG);
    const int64_t best = s4 < s2 ? (s4 < s1 ? s4 : s1) : (s2 < s1 ? s2 : s1);
    if constexpr (C <= 32) {
        if (s4 * 16 <= best * 17) return launch_colv_tt<C, EPI, 4, WG>(a, s);
    }
    if constexpr (C <= 48) {
        if (s2 * 16 <= best * 17) return launch_colv_tt<C, EPI, 2, WG>(a, s);
    }
    return launch_colv_tt<C, EPI, 1, WG>(a, s);
}

template <int C>
static int launch_colv2(const ColConvArgs& a, int epi, hipStream_t s) {
    switch (epi) {
        case PMG_EPI_ACC: return launch_colv<C, PMG_EPI_ACC>(a, s);
        case PMG_EPI_Q: return launch_colv<C, PMG_EPI_Q>(a, s);
        case PMG_EPI_R: return launch_colv<C, PMG_EPI_R>(a, s);
        case PMG_EPI_RLN: return launch_colv<C, PMG_EPI_RLN>(a, s);
        case PMG_EPI_ROUT: return launch_colv<C, PMG_EPI_ROUT>(a, s);
    }
    return fail(PMG_E_INVALID, "pmg_spconv_col: unknown epilogue");
}

int launch_conv_col(int precision, const ColConvArgs& a, int C, int epi, hipStream_t s) {
    if (a.x0_feats && !(precision == PMG_PREC_INT8 && C <= 64 && epi == PMG_EPI_RLN))
        return fail(PMG_E_INVALID, "pmg_spconv_col: a recomputed first-block skip needs int8, C <= 64 and RLN");
    if (precision == PMG_PREC_INT8) {
        switch (C) {
            case 16: return launch_colv2<16>(a, epi, s);
            case 32: return launch_colv2<32>(a, epi, s);
            case 48: return launch_colv2<48>(a, epi, s);
            case 64: return launch_colv2<64>(a, epi, s);
            case 128: return launch_col2<int8_t, 128>(a, epi, s);
        }
    } else {
        switch (C) {
            case 16: return launch_col2<_Float16, 16>(a, epi, s);
            case 32: return launch_col2<_Float16, 32>(a, epi, s);
            case 48: return launch_col2<_Float16, 48>(a, epi, s);
            case 64: return launch_col2<_Float16, 64>(a, epi, s);
        }
    }
    return fail(PMG_E_INVALID, "pmg_spconv_col: C must be 16, 32, 48, 64 or 128 (int8), 16..64 (fp16)");
}

}  // namespace pmg

using namespace pmg;

extern "C" int pmg_spconv_col(int precision, const void* x, const int32_t* zq, int B, int H, int W, int C,
                              const void* w, int epilogue, const pmg_conv_epilogue* e, void* stream) {
    PMG_REQUIRE(x && zq && w && e, "null buffer");
    PMG_REQUIRE(epilogue == PMG_EPI_ROUT || e->out, "null output");
    PMG_REQUIRE(precision == PMG_PREC_INT8 || precision == PMG_PREC_FP16, "bad precision");
    PMG_REQUIRE(B > 0 && H > 0 && W > 0, "bad shape");
    const int64_t M = (int64_t)B * H * W;
    PMG_REQUIRE(M + 2 * (int64_t)W + 2 * kSeg <= INT_MAX, "too many voxels");
    PMG_REQUIRE(aligned16(x) && aligned16(w), "x and w must be 16-byte aligned");
    const bool i8 = precision == PMG_PREC_INT8;
    PMG_REQUIRE(!i8 || epilogue == PMG_EPI_ACC || e->w_scale, "int8 needs w_scale");
    PMG_REQUIRE(epilogue != PMG_EPI_Q || !i8 || e->out_mult > 0.0f, "out_mult must be positive");
    const bool res = epilogue == PMG_EPI_R || epilogue == PMG_EPI_RLN || epilogue == PMG_EPI_ROUT;
    PMG_REQUIRE(!res || (e->skip && aligned16(e->skip)), "residual epilogues need a 16-byte aligned skip");
    PMG_REQUIRE(epilogue == PMG_EPI_ROUT || aligned16(e->out), "out must be 16-byte aligned");
    PMG_REQUIRE(epilogue != PMG_EPI_RLN || (e->ln_gamma && e->ln_beta && e->next_q && (!i8 || e->next_mult > 0.0f)),
                "RLN needs LayerNorm parameters and next_q");
    PMG_REQUIRE(epilogue != PMG_EPI_ROUT || (e->out_w && e->out_b && ((e->points && e->points_out) || e->out)),
                "ROUT needs out_proj weights and either the point maps or out");
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
    a.out_mult = e->out_mult;
    a.skip = e->skip;
    a.out = e->out;
    a.ln_gamma = e->ln_gamma;
    a.ln_beta = e->ln_beta;
    a.ln_eps = e->ln_eps;
    a.next_mult = e->next_mult;
    a.next_q = e->next_q;
    a.out_w = e->out_w;
    a.out_b = e->out_b;
    a.points = e->points;
    a.points_out = e->points_out;
    return launch_conv_col(precision, a, C, epilogue, (hipStream_t)stream);
}
