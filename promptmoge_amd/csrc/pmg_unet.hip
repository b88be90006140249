// The multi-level sparse U-Net refiner (Sparse3DUNet, moge/model/modules/sparse_unet.py:17-258) in the deployed
// int8 arithmetic, every level built and sized on the device.
//
// Structure. Level 0 holds one voxel per pixel in raster (b, i, j) order (MoGeModel._voxelize, v3.py:305-344).
// Level k+1 is PoolDown's perfect-partition pool of level k, stride 2 on (i, j, z) (flex_sparse_blocks.py:78-90;
// _core.py:339-395). Every level's voxels are in (b, i, j, z) order -- the order of _linearise on the pooled shape,
// i.e. the reference's sorted unique output keys -- so a level is a set of columns (b, i, j), each holding its
// voxels with increasing z: a column CSR. A coarse column merges the z / 2 lists of its (up to) four child columns:
// one thread per coarse column counts the distinct values and scans them within its block of 256 columns, and the
// same merge then writes the coarse voxels and each child's parent, each block starting after the totals of the
// blocks before it. The children of a coarse voxel in increasing row
// order are the matching runs of its child columns in raster order, the order of the reference's index_add_. This
// is the per-column design of the reference's device engine (Structure.metal:87-215) without its host-side sizing:
// the voxel count of every level stays on the device, buffers are allocated for the level-0 count (an upper bound
// of every level), and every later kernel reads the count. Submanifold maps of levels >= 1: per voxel, the 9
// neighbouring columns are scanned for z - 1, z, z + 1 (the result of _build_submanifold_nmap_sorted,
// _core.py:298-304), tap-major [27][capacity] with 16-row tile masks.
//
// Layers (int8 contract qat.py:1-16; the deployed engine's sequence, Refiner.swift:224-292, Refiner.metal:133-322):
//   level-0 blocks         the map-free column convolutions (pmg_conv_col.hip) with the next LayerNorm fused
//   blocks at levels >= 1  generic-map MFMA conv with the device row count (launch_conv_i8_dev: the weight-staged
//                          spconv_g2_k / spconv_g2r_k at C = 64 / 128 / 256, spconv_k otherwise) + a row
//                          LayerNorm kernel
//   PoolDown               one kernel: children's fp32 mean (row order, / count) quantised, int8 GEMM, and the next
//                          block's LayerNorm codes (fp16: mean-pool kernel, GEMM, row LayerNorm kernel)
//   encoder conditioning   per token: quantise-transpose of the planar feature, int8 GEMM (+ the planar bias map),
//                          gathered per voxel by its column in the concat-quantise of fuse_proj.0's input
//   fuse_proj              int8 GEMM + SiLU + requantise, int8 GEMM
//   NearestUp              one kernel per fine voxel (int8): parent row's codes, int8 GEMM, + skip, next LayerNorm
//                          (fp16: quantise, GEMM at the coarse level, then parent gather + skip + LayerNorm)
//   out_proj               in the epilogue of the last level-0 conv
#include <climits>
#include <cstring>
#include <string>
#include <vector>

#include "pmg_common.h"
#include "pmg_graph.h"
#include "pmg_internal.h"

namespace pmg {

constexpr int kMaxLevels = 8;

// ---------------------------------------------------------------------------------------------------------------
// Level structure.

// Level-0 coordinates (b, i, j, zq - zmin[b]) (v3.py:333-340), and the level-0 keys zq.
__global__ __launch_bounds__(256) void level0_coords_k(const int32_t* __restrict__ zq, const int32_t* __restrict__ zmin,
                                                       int H, int W, int64_t M, int4* __restrict__ coords) {
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (m >= M) return;
    const int64_t HW = (int64_t)H * W;
    const int b = (int)(m / HW);
    const int p = (int)(m - (int64_t)b * HW);
    coords[m] = make_int4(b, p / W, p % W, zq[m] - zmin[b]);
}

// The caller's level-0 coordinates copied into the context's own buffer, so that level 0's coordinates always live
// at one address (also across replays of graphs captured with and without given coordinates).
__global__ __launch_bounds__(256) void copy_coords_k(const int4* __restrict__ src, int64_t M, int4* __restrict__ dst) {
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (m < M) dst[m] = src[m];
}

// Voxels of column c of a level: [off[c], off[c + 1]); level 0 (off NULL) holds voxel c in column c.
__device__ inline void col_range(const int32_t* off, int64_t c, int32_t& lo, int32_t& hi) {
    if (off) {
        lo = off[c];
        hi = off[c + 1];
    } else {
        lo = (int32_t)c;
        hi = lo + 1;
    }
}

struct PoolGeom {
    const int4* coords;   // fine level [cap][4]
    const int32_t* off;   // fine column CSR [B * Hf * Wf + 1], or NULL (level 0)
    int B, Hf, Wf;        // fine column grid
    int Hc, Wc;           // coarse column grid: ceil(Hf / 2), ceil(Wf / 2)
};

// The (up to) four child columns of coarse column C = (b, I, J), in raster order: (2I, 2J), (2I, 2J+1),
// (2I+1, 2J), (2I+1, 2J+1); those outside the fine grid are empty.
__device__ inline void child_ranges(const PoolGeom& g, int64_t C, int32_t (&lo)[4], int32_t (&hi)[4]) {
    const int64_t per = (int64_t)g.Hc * g.Wc;
    const int b = (int)(C / per);
    const int rem = (int)(C - (int64_t)b * per);
    const int I = rem / g.Wc, J = rem - (rem / g.Wc) * g.Wc;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int i = 2 * I + (q >> 1), j = 2 * J + (q & 1);
        if (i < g.Hf && j < g.Wf) {
            col_range(g.off, ((int64_t)b * g.Hf + i) * g.Wf + j, lo[q], hi[q]);
        } else {
            lo[q] = 0;
            hi[q] = 0;
        }
    }
}

// The four child columns' lists merged by z / 2 (z >= 0, so z >> 1 = floor): zh[q] caches z / 2 at the head of list
// q (INT_MAX once it is exhausted), so a step reads only the heads it advances, all four loads issued together.
struct ChildMerge {
    int32_t h[4], e[4];
    int zh[4];
    __device__ inline int head_z(const int4* coords, int q) const {
        return h[q] < e[q] ? coords[h[q]].w >> 1 : INT_MAX;
    }
    __device__ inline void init(const PoolGeom& g, int64_t C) {
        child_ranges(g, C, h, e);
        int z[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) z[q] = g.coords[h[q] < e[q] ? h[q] : 0].w >> 1;
#pragma unroll
        for (int q = 0; q < 4; ++q) zh[q] = h[q] < e[q] ? z[q] : INT_MAX;
    }
    __device__ inline int min_z() const {
        int mn = zh[0];
#pragma unroll
        for (int q = 1; q < 4; ++q) mn = zh[q] < mn ? zh[q] : mn;
        return mn;
    }
    // Consumes every head equal to mn (the voxels of one coarse voxel), calling take(row) in list order.
    template <class Take>
    __device__ inline void consume(const int4* coords, int mn, Take take) {
        for (;;) {
            bool adv = false;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (zh[q] == mn) {
                    take(h[q]);
                    ++h[q];
                    adv = true;
                }
            if (!adv) break;
            int z[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) z[q] = coords[h[q] < e[q] ? h[q] : 0].w >> 1;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (zh[q] == mn) zh[q] = h[q] < e[q] ? z[q] : INT_MAX;
        }
    }
};

// One thread per coarse column: its voxel count (the distinct z / 2 of its child columns), and the exclusive scan
// of the counts within the block's 256 columns (excl) with the block's total (tile_sum).
__global__ __launch_bounds__(256) void pool_count_k(PoolGeom g, int64_t ncols, int32_t* __restrict__ excl,
                                                    int32_t* __restrict__ tile_sum) {
    __shared__ int32_t wsum[4];
    const int64_t C = (int64_t)blockIdx.x * 256 + threadIdx.x;
    int n = 0;
    if (C < ncols) {
        ChildMerge cm;
        cm.init(g, C);
        for (;;) {
            const int mn = cm.min_z();
            if (mn == INT_MAX) break;
            cm.consume(g.coords, mn, [](int32_t) {});
            ++n;
        }
    }
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t incl = wave_incl_scan_u32((uint32_t)n);
    if (lane == 63) wsum[w] = (int32_t)incl;
    __syncthreads();
    int32_t before = 0;
    for (int k = 0; k < w; ++k) before += wsum[k];
    if (C < ncols) excl[C] = before + (int32_t)incl - n;
    if (threadIdx.x == 255) tile_sum[blockIdx.x] = before + (int32_t)incl;
}

// Writes the coarse voxels of column C (coordinates and the column's CSR start), the parent of every child and, per
// coarse voxel, its children: for child column q, the first child's row | (the number of children, 0 - 2) << 30
// (a column holds at most the two voxels z = 2 Z, 2 Z + 1 of coarse voxel Z). The block's first row is the sum of
// the tile totals of the blocks before it (pool_count_k's tiling: 256 columns per block); the last block also
// writes the level's voxel count and the end of its column CSR.
__global__ __launch_bounds__(256) void pool_emit_k(PoolGeom g, int64_t ncols, const int32_t* __restrict__ excl,
                                                   const int32_t* __restrict__ tile_sum, int64_t* __restrict__ count,
                                                   int4* __restrict__ coords_c, int32_t* __restrict__ off_c,
                                                   int32_t* __restrict__ parent, int4* __restrict__ child) {
    __shared__ int32_t wsum[4];
    int32_t t = 0;
    for (int64_t q = threadIdx.x; q < (int64_t)blockIdx.x; q += 256) t += tile_sum[q];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t incl = wave_incl_scan_u32((uint32_t)t);
    if (lane == 63) wsum[w] = (int32_t)incl;
    __syncthreads();
    const int32_t tile0 = wsum[0] + wsum[1] + wsum[2] + wsum[3];
    const int64_t C = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (C >= ncols) return;
    const int32_t base = excl[C] + tile0;
    off_c[C] = base;
    if (C == ncols - 1) {  // the last column: the level's total
        const int32_t total = tile0 + tile_sum[blockIdx.x];
        *count = total;
        off_c[ncols] = total;
    }
    const int64_t per = (int64_t)g.Hc * g.Wc;
    const int b = (int)(C / per);
    const int rem = (int)(C - (int64_t)b * per);
    const int I = rem / g.Wc, J = rem - (rem / g.Wc) * g.Wc;
    ChildMerge cm;
    cm.init(g, C);
    int32_t o = base;
    for (;;) {
        const int mn = cm.min_z();
        if (mn == INT_MAX) break;
        coords_c[o] = make_int4(b, I, J, mn);
        const int32_t h0 = cm.h[0], h1 = cm.h[1], h2 = cm.h[2], h3 = cm.h[3];
        cm.consume(g.coords, mn, [&](int32_t row) { parent[row] = o; });
        child[o] = make_int4(h0 | ((cm.h[0] - h0) << 30), h1 | ((cm.h[1] - h1) << 30), h2 | ((cm.h[2] - h2) << 30),
                             h3 | ((cm.h[3] - h3) << 30));
        ++o;
    }
}

// The submanifold map of a level >= 1: nmap_t[v][o] = the row of (b, i + di, j + dj, z + dz) or -1, tap
// v = (di+1)*9 + (dj+1)*3 + (dz+1) (_core.py:65-82), found in the 9 neighbouring columns; 16-row tile masks.
__global__ __launch_bounds__(256) void nmap_level_k(const int4* __restrict__ coords, const int32_t* __restrict__ off,
                                                    const int64_t* __restrict__ count, int H, int W, int64_t cap,
                                                    int32_t* __restrict__ nmap_t, uint32_t* __restrict__ tile_mask) {
    const int64_t M = *count;
    if ((int64_t)blockIdx.x * 256 >= M) return;  // whole block beyond the level
    const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
    uint32_t rmask = 0;
    if (o < M) {
        const int4 c = coords[o];
        // the 9 neighbouring columns' voxel ranges, all loaded before any is walked
        int32_t p[9], hi[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            const int i = c.y + k / 3 - 1, j = c.z + k % 3 - 1;
            const bool in = i >= 0 && i < H && j >= 0 && j < W;
            const int64_t col = in ? ((int64_t)c.x * H + i) * W + j : 0;
            p[k] = in ? off[col] : 0;
            hi[k] = in ? off[col + 1] : 0;
        }
        // walk the columns in lock step, one voxel of each per trip (its z loaded for all 9 before any is
        // compared); a column stops at its end or above z + 1
        int32_t f[27];
#pragma unroll
        for (int v = 0; v < 27; ++v) f[v] = -1;
        for (;;) {
            int zc[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) zc[k] = coords[p[k] < hi[k] ? p[k] : 0].w;
            bool any = false;
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                if (p[k] < hi[k] && zc[k] <= c.w + 1) {
                    const int dz = zc[k] - (c.w - 1);
#pragma unroll
                    for (int d = 0; d < 3; ++d)
                        if (dz == d) f[3 * k + d] = p[k];
                    ++p[k];
                    any = true;
                } else {
                    p[k] = hi[k];
                }
            }
            if (!any) break;
        }
#pragma unroll
        for (int v = 0; v < 27; ++v) {
            nmap_t[(int64_t)v * cap + o] = f[v];
            rmask |= (f[v] >= 0 ? 1u : 0u) << v;
        }
    }
#pragma unroll
    for (int sh = 1; sh < 16; sh <<= 1) rmask |= __shfl_xor(rmask, sh, 16);
    if ((o & 15) == 0 && o < M) tile_mask[o >> 4] = rmask;
}

// ---------------------------------------------------------------------------------------------------------------
// Row kernels on device-sized levels.

// The row kernels below walk a level's rows in grid-stride loops over the count on the device: their grids are
// capped (row_grid), so a coarse level of a few thousand rows does not launch the capacity's hundreds of
// thousands of threads only to have them exit.
constexpr int64_t kRowBlocksMax = 4096;  // 16 blocks of 256 threads per CU
static unsigned row_grid(int64_t threads_cap) {
    const int64_t b = (threads_cap + 255) / 256;
    return (unsigned)(b < 1 ? 1 : (b < kRowBlocksMax ? b : kRowBlocksMax));
}

// A linear's or convolution's input activations, in the network's arithmetic: int8 codes clamp(rint(v * mult)), or
// fp16 (the teacher; mult unused).
__device__ inline void put4(int8_t* dst, const float (&h)[4], float mult) { store_codes4(h, mult, dst); }
__device__ inline void put4(_Float16* dst, const float (&h)[4], float) { store_half4(h, dst); }

// PoolDown's mean (sparse_pool 'mean', _core.py:464-476: fp32 sums in input row order from 0, divided by the
// child count) of coarse voxel o, as the pool linear's input (codes = clamp(rint(mean * mult)), or fp16). Threads
// per row = C / 4 (a float4 each).
template <typename O>
__global__ __launch_bounds__(256) void pool_quant_k(const float* __restrict__ x, int C, PoolGeom g,
                                                    const int4* __restrict__ coords_c, const int64_t* __restrict__ count,
                                                    float mult, O* __restrict__ codes) {
    const int tpr = C >> 2;
    const int64_t items = *count * tpr;
    for (int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x; gid < items; gid += (int64_t)gridDim.x * 256) {
        const int64_t o = gid / tpr;
        const int cq = (int)(gid - o * tpr);
        const int4 oc = coords_c[o];
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        int n = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = 2 * oc.y + (q >> 1), j = 2 * oc.z + (q & 1);
            if (i >= g.Hf || j >= g.Wf) continue;
            int32_t lo, hi;
            col_range(g.off, ((int64_t)oc.x * g.Hf + i) * g.Wf + j, lo, hi);
            for (int32_t p = lo; p < hi; ++p) {
                const int z = g.coords[p].w >> 1;
                if (z > oc.w) break;
                if (z == oc.w) {
                    const float4 v = *(const float4*)(x + (int64_t)p * C + 4 * cq);
                    acc.x = acc.x + v.x;
                    acc.y = acc.y + v.y;
                    acc.z = acc.z + v.z;
                    acc.w = acc.w + v.w;
                    ++n;
                }
            }
        }
        const float cnt = (float)n;
        const float h[4] = {acc.x / cnt, acc.y / cnt, acc.z / cnt, acc.w / cnt};
        put4(codes + o * C + 4 * cq, h, mult);
    }
}

// The input of NearestUp's linear from a device-sized [rows][C] fp32 array: codes = clamp(rint(x * mult)), or fp16.
template <typename O>
__global__ __launch_bounds__(256) void quant_rows_k(const float* __restrict__ x, int C, const int64_t* __restrict__ count,
                                                    float mult, O* __restrict__ codes) {
    const int64_t groups = *count * C / 4;  // groups of 4 values
    for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < groups; q += (int64_t)gridDim.x * 256) {
        const float4 v = *(const float4*)(x + q * 4);
        const float h[4] = {v.x, v.y, v.z, v.w};
        put4(codes + q * 4, h, mult);
    }
}

// Row LayerNorm / SiLU / quantise in the 16-rows-per-wave layout of the fused epilogues (lane (r, g) holds
// channels 16j + 4g + i of row r; quad-order sums), on a device-sized level:
//   UP = false: codes = quant(silu(LN(x))) of x
//   UP = true:  y = lin[parent[m]] + skip[m] (NearestUp + the U-Net's skip add, sparse_unet.py:251-254), written
//               to y_out, then (gamma non-NULL) codes of y
// The codes are int8 (O = int8_t: SiLU inside the requantisation) or fp16 (O = _Float16: silu_fast, rounded).
template <int C, bool UP, typename O>
__global__ __launch_bounds__(256) void rows_ln_k(const float* __restrict__ x, const int32_t* __restrict__ parent,
                                                 const float* __restrict__ skip, const int64_t* __restrict__ count,
                                                 const float* __restrict__ gamma, const float* __restrict__ beta,
                                                 float eps, float mult, float* __restrict__ y_out,
                                                 O* __restrict__ codes) {
    constexpr int NB = C / 16;
    const int64_t M = *count;
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    // blocks of 64 rows, grid-stride (every lane of a wave runs each trip: the LayerNorm sums cross lanes)
    for (int64_t blk = blockIdx.x; blk * 64 < M; blk += gridDim.x) {
        const int64_t m = (blk * 4 + (threadIdx.x >> 6)) * 16 + r;
        const bool ok = m < M;
        const int64_t mo = ok ? m : 0;
        float y[NB][4];
        const int64_t src = UP ? (int64_t)parent[mo] : mo;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const float4 v = *(const float4*)(x + src * C + 16 * j + 4 * g);
            y[j][0] = v.x;
            y[j][1] = v.y;
            y[j][2] = v.z;
            y[j][3] = v.w;
            if constexpr (UP) {
                const float4 k = *(const float4*)(skip + mo * C + 16 * j + 4 * g);
                y[j][0] = y[j][0] + k.x;
                y[j][1] = y[j][1] + k.y;
                y[j][2] = y[j][2] + k.z;
                y[j][3] = y[j][3] + k.w;
                if (ok) *(float4*)(y_out + mo * C + 16 * j + 4 * g) = make_float4(y[j][0], y[j][1], y[j][2], y[j][3]);
            }
        }
        if (!gamma) continue;
        if constexpr (sizeof(O) == 1) {
            ln_silu_quad<NB, false>(y, gamma, beta, eps, g);
            uint32_t pk[NB];
            silu_codes_packed<NB>(y, mult, pk);
            if (ok) {
#pragma unroll
                for (int j = 0; j < NB; ++j) *(uint32_t*)(codes + mo * C + 16 * j + 4 * g) = pk[j];
            }
        } else {
            ln_silu_quad<NB, true>(y, gamma, beta, eps, g);
            if (ok) {
#pragma unroll
                for (int j = 0; j < NB; ++j) store_half4(y[j], codes + mo * C + 16 * j + 4 * g);
            }
        }
    }
}

// The encoder feature, planar [B][K][RC] fp32, into token rows [B * RC][K] (int8 clamp(rint(v * mult)), or fp16):
// 64 x 64 tiles transposed through LDS (loads along the token index, stores along the channel).
__device__ inline int8_t to_act(float v, float mult, int8_t) { return quant_i8(v, mult); }
__device__ inline _Float16 to_act(float v, float, _Float16) { return (_Float16)v; }

template <typename O>
__global__ __launch_bounds__(256) void enc_quant_k(const float* __restrict__ planar, int K, int64_t RC, float mult,
                                                   O* __restrict__ codes) {
    __shared__ O tile[64][64 + 4];
    const int b = blockIdx.z;
    const int64_t t0 = (int64_t)blockIdx.x * 64;
    const int k0 = blockIdx.y * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int kk = ty + 4 * r;
        const int64_t t = t0 + tx;
        float v = 0.0f;
        if (t < RC && k0 + kk < K) v = planar[((int64_t)b * K + k0 + kk) * RC + t];
        tile[kk][tx] = to_act(v, mult, O{});
    }
    __syncthreads();
    const int tt = threadIdx.x >> 2, kc = (threadIdx.x & 3) * 16;
    const int64_t t = t0 + tt;
    if (t >= RC || k0 + kc >= K) return;
    O* const dst = codes + ((int64_t)b * RC + t) * K + k0 + kc;
    if constexpr (sizeof(O) == 1) {
        uint32_t w[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            w[u] = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) w[u] |= (uint32_t)(uint8_t)tile[kc + 4 * u + i][tt] << (8 * i);
        }
        *(uint4*)dst = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        h8 v0, v1;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v0[i] = tile[kc + i][tt];
            v1[i] = tile[kc + 8 + i][tt];
        }
        *(h8*)dst = v0;
        *(h8*)(dst + 8) = v1;
    }
}

// fuse_proj.0's input: cat([x, enc_tok[token of the voxel's column]]) quantised with one scale (sparse_unet.py:
// 240; the deployed concat_q8, Refiner.metal:285-300). Token of (b, i, j) = (b * R + i) * Cc + j.
template <typename O>
__global__ __launch_bounds__(256) void concat_quant_k(const float* __restrict__ x, const float* __restrict__ enc_tok,
                                                      const int4* __restrict__ coords, const int64_t* __restrict__ count,
                                                      int C, int R, int Cc, float mult, O* __restrict__ codes) {
    const int tpr = C >> 1;  // 2C channels, 4 per thread
    const int64_t items = *count * tpr;
    for (int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x; gid < items; gid += (int64_t)gridDim.x * 256) {
        const int64_t o = gid / tpr;
        const int c = 4 * (int)(gid - o * tpr);
        const float* src;
        if (c < C) {
            src = x + o * C + c;
        } else {
            const int4 v = coords[o];
            src = enc_tok + (((int64_t)v.x * R + v.y) * Cc + v.z) * C + (c - C);
        }
        const float4 v = *(const float4*)src;
        const float h[4] = {v.x, v.y, v.z, v.w};
        put4(codes + o * 2 * C + c, h, mult);
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Dense GEMM on MFMA (nn.Linear; in int8 the deployed dg8 kernels, Refiner.metal:173-250):
//   out[m][n] = (acc * a_scale) * w_scale[n] + bias[n] (+ planar_add[b][n][rc], m = b * RC + rc)      EPI_BIAS
//   codes[m][n] = quant(silu(...), out_mult)                                                           EPI_Q
// acc = sum_k A[m][k] * W[n][k] exact in int32; A [rows][K] int8 codes, W [N][K] int8 (nn.Linear's layout).
// The teacher (E = _Float16): fp16 A and W, fp32 accumulation (v_mfma_f32_16x16x32_f16), out = acc + bias[n]
// (+ planar_add), or SiLU of it rounded to fp16 (EPI_Q). One wave per 16 rows x 16 NB columns, MFMAs over the
// 16-byte K chunks with the operand layout of spconv_k (lane l: row / column l % 16, chunk l / 16 of each 64-byte
// step).
struct GemmArgs {
    const void* a;
    const void* w;
    int64_t rows_cap;
    const int64_t* rows_dev;  // rows on the device, or NULL for rows_cap
    int K, N;
    float a_scale;
    const float* w_scale;
    const float* bias;
    float out_mult;
    void* out;
    const float* planar_add;
    int64_t planar_rc;
};

__device__ inline void gemm_mma(v4i& acc, const v4i& a, const v4i& b, int8_t) {
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
}
__device__ inline void gemm_mma(v4f& acc, const v4i& a, const v4i& b, _Float16) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), acc, 0, 0,
                                                  0);
}

template <int NB, int EPI, typename E = int8_t>
__global__ __launch_bounds__(256) void gemm_i8_k(GemmArgs g) {
    typedef typename std::conditional<sizeof(E) == 1, v4i, v4f>::type acc_t;
    const int64_t rows = g.rows_dev ? *g.rows_dev : g.rows_cap;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r = lane & 15, gq = lane >> 4;
    const int n0 = blockIdx.y * 16 * NB;
    const int rowb = g.K * (int)sizeof(E);  // bytes per row of A and W
    const int nchunk = rowb >> 4;
    const uint8_t* const ga = (const uint8_t*)g.a;
    const uint8_t* const gw = (const uint8_t*)g.w;
    // blocks of 64 rows (16 per wave), grid-stride over the rows on the device
    for (int64_t mb = blockIdx.x; mb * 64 < rows; mb += gridDim.x) {
        const int64_t m0 = (mb * 4 + wv) * 16;
        if (m0 >= rows) break;
        const int64_t row = m0 + r;
        const bool row_ok = row < rows;
        acc_t acc[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[j] = acc_t{0, 0, 0, 0};
        // K in steps of 4 chunks (one per lane group), the next step's operands requested before this step's
        // MFMAs. Loads are unconditional (a clamped address; the padding chunks and rows past the end are zeroed
        // when used), so the memory waits name exactly the step they need.
        const int64_t arow = (row_ok ? row : 0) * rowb;
        auto load = [&](int q0, v4i& av, v4i (&bv)[NB]) {
            const int q = q0 + gq < nchunk ? q0 + gq : nchunk - 1;
            av = *(const v4i*)(ga + arow + q * 16);
#pragma unroll
            for (int j = 0; j < NB; ++j) bv[j] = *(const v4i*)(gw + (int64_t)(n0 + 16 * j + r) * rowb + q * 16);
        };
        auto mma = [&](int q0, const v4i& av, const v4i (&bv)[NB]) {
            const bool on = q0 + gq < nchunk;
            const v4i z = {0, 0, 0, 0};
            const v4i a = on && row_ok ? av : z;
#pragma unroll
            for (int j = 0; j < NB; ++j) gemm_mma(acc[j], a, on ? bv[j] : z, E{});
        };
        v4i a0, a1, b0[NB], b1[NB];
        load(0, a0, b0);
        for (int q0 = 0; q0 < nchunk; q0 += 8) {
            if (q0 + 4 < nchunk) load(q0 + 4, a1, b1);
            mma(q0, a0, b0);
            if (q0 + 4 >= nchunk) break;
            if (q0 + 8 < nchunk) load(q0 + 8, a0, b0);
            mma(q0 + 4, a1, b1);
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int n = n0 + 16 * j + r;
            const float ws = sizeof(E) == 1 ? g.w_scale[n] : 1.0f, bs = g.bias ? g.bias[n] : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t m = m0 + 4 * gq + i;
                if (m >= rows) continue;
                float y;
                if constexpr (sizeof(E) == 1) {
                    y = (float)acc[j][i] * g.a_scale;
                    y = y * ws;
                } else {
                    y = acc[j][i];
                }
                if (g.bias) y = y + bs;
                if constexpr (EPI == PMG_EPI_Q) {
                    if constexpr (sizeof(E) == 1)
                        ((int8_t*)g.out)[m * g.N + n] = silu_quant_i8(y, g.out_mult);
                    else
                        ((_Float16*)g.out)[m * g.N + n] = (_Float16)silu_fast(y);
                } else {
                    if (g.planar_add) {
                        const int64_t b = m / g.planar_rc, rc = m - b * g.planar_rc;
                        y = y + g.planar_add[(b * g.N + n) * g.planar_rc + rc];
                    }
                    ((float*)g.out)[m * g.N + n] = y;
                }
            }
        }
    }
}

// PoolDown as one kernel (int8): the children's mean of each coarse voxel (pool_quant_k's arithmetic), quantised,
// times the pool linear (gemm_i8_k's EPI_BIAS arithmetic) -> the coarse fp32 row, and, when the level has a block,
// that block's LayerNorm -> SiLU -> int8 codes (rows_ln_k's arithmetic). One wave per 16 coarse voxels holds all Cn
// = 16 NB output channels, so the pooled codes are formed once per voxel and the row is whole for the LayerNorm;
// the accumulators go from the MFMA layout (lane (r, g): rows 4g + i, column r) to the row layout of the
// LayerNorm (lane (r, g): row r, channels 16j + 4g + i) through the wave's LDS tile.
struct PoolLinArgs {
    const float* x;         // fine level [cap][Ck] fp32
    int Ck, Cn;
    PoolGeom g;
    const int4* coords_c;   // coarse voxels
    const int4* child;      // per coarse voxel: first child row | children << 30 per child column (pool_emit_k)
    const int64_t* count;   // coarse voxel count (device)
    float pool_mult;        // the pool linear's input quantisation
    const int8_t* w;        // [Cn][Ck]
    float a_scale;
    const float* w_scale;   // [Cn]
    const float* bias;      // [Cn] or NULL
    float* y_out;           // coarse [cap][Cn] fp32
    const float* gamma;     // next block's LayerNorm, or NULL (no codes)
    const float* beta;
    float ln_mult;
    int8_t* codes;          // coarse [cap][Cn]
};

template <int NB>
__global__ __launch_bounds__(256) void pool_linear_ln_k(PoolLinArgs a) {
    constexpr int CN = 16 * NB;
    constexpr int LDW = CN + 4;  // LDS tile row stride (floats)
    __shared__ float tile[4][16 * LDW];
    const int64_t rows = *a.count;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r = lane & 15, gq = lane >> 4;
    const int nchunk = a.Ck >> 4;  // 16-channel chunks of a fine row
    const int rowb = a.Ck;         // bytes per weight row
    float* tl = tile[wv];
    for (int64_t mb = blockIdx.x; mb * 64 < rows; mb += gridDim.x) {
        const int64_t m0 = (mb * 4 + wv) * 16;
        if (m0 >= rows) break;
        const int64_t o = m0 + r;
        const bool row_ok = o < rows;
        // the children of coarse voxel o: runs of z / 2 == oc.w in its four child columns, in row order; lane
        // group gq walks child column gq, and every lane of the row then reads the four runs
        int32_t clo[4], chi[4];
        {
            const int4 oc = a.coords_c[row_ok ? o : 0];
            int32_t p = 0, e = 0;
            const int i = 2 * oc.y + (gq >> 1), j = 2 * oc.z + (gq & 1);
            if (row_ok && i < a.g.Hf && j < a.g.Wf) {
                int32_t lo, hi;
                col_range(a.g.off, ((int64_t)oc.x * a.g.Hf + i) * a.g.Wf + j, lo, hi);
                p = lo;
                while (p < hi && (a.g.coords[p].w >> 1) < oc.w) ++p;
                e = p;
                while (e < hi && (a.g.coords[e].w >> 1) == oc.w) ++e;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                clo[q] = __shfl(p, r + 16 * q, 64);
                chi[q] = __shfl(e, r + 16 * q, 64);
            }
        }
        const float cnt = (float)((chi[0] - clo[0]) + (chi[1] - clo[1]) + (chi[2] - clo[2]) + (chi[3] - clo[3]));
        v4i acc[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[j] = v4i{0, 0, 0, 0};
        for (int q0 = 0; q0 < nchunk; q0 += 4) {
            const int ch = q0 + gq;  // this lane group's 16-channel chunk
            const bool on = ch < nchunk;
            const int qc = on ? ch : nchunk - 1;
            v4i bv[NB];
#pragma unroll
            for (int j = 0; j < NB; ++j) bv[j] = *(const v4i*)(a.w + (int64_t)(16 * j + r) * rowb + qc * 16);
            // pooled mean of the chunk's 16 channels: fp32 sums from 0 in child row order, / count, quantised
            v4i av = v4i{0, 0, 0, 0};
            if (on && row_ok) {
                float h[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) h[e] = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    for (int32_t p = clo[q]; p < chi[q]; ++p) {
                        const float* src = a.x + (int64_t)p * a.Ck + 16 * ch;
#pragma unroll
                        for (int v = 0; v < 4; ++v) {
                            const float4 f = *(const float4*)(src + 4 * v);
                            h[4 * v + 0] = h[4 * v + 0] + f.x;
                            h[4 * v + 1] = h[4 * v + 1] + f.y;
                            h[4 * v + 2] = h[4 * v + 2] + f.z;
                            h[4 * v + 3] = h[4 * v + 3] + f.w;
                        }
                    }
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float m4[4] = {h[4 * v] / cnt, h[4 * v + 1] / cnt, h[4 * v + 2] / cnt, h[4 * v + 3] / cnt};
                    av[v] = (int)pack_codes4(m4, a.pool_mult);
                }
            }
#pragma unroll
            for (int j = 0; j < NB; ++j)
                acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, on ? bv[j] : v4i{0, 0, 0, 0}, acc[j], 0, 0, 0);
        }
        // y = (acc * a_scale) * w_scale[n] + bias[n] (gemm_i8_k's EPI_BIAS), through LDS into the row layout
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int n = 16 * j + r;
            const float ws = a.w_scale[n], bs = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float y = (float)acc[j][i] * a.a_scale;
                y = y * ws;
                if (a.bias) y = y + bs;
                tl[(4 * gq + i) * LDW + n] = y;
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's tile writes are in LDS
        __builtin_amdgcn_wave_barrier();
        float y[NB][4];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const float4 v = *(const float4*)(tl + r * LDW + 16 * j + 4 * gq);
            y[j][0] = v.x;
            y[j][1] = v.y;
            y[j][2] = v.z;
            y[j][3] = v.w;
            if (row_ok) *(float4*)(a.y_out + o * CN + 16 * j + 4 * gq) = v;
        }
        __builtin_amdgcn_wave_barrier();  // every lane has read the tile before the next trip writes it
        if (!a.gamma) continue;
        ln_silu_quad<NB, false>(y, a.gamma, a.beta, 1e-6f, gq);
        uint32_t pk[NB];
        silu_codes_packed<NB>(y, a.ln_mult, pk);
        if (row_ok) {
#pragma unroll
            for (int j = 0; j < NB; ++j) *(uint32_t*)(a.codes + o * CN + 16 * j + 4 * gq) = pk[j];
        }
    }
}

static int launch_pool_linear_ln(const PoolLinArgs& a, int64_t cap, hipStream_t s) {
    if (cap == 0) return PMG_OK;
    PMG_REQUIRE(a.Ck % 16 == 0 && a.Ck > 0, "pool linear input width must be a multiple of 16");
    const dim3 grid(row_grid(cap * 4));  // 64 coarse rows (256 threads) per block, grid-stride
    switch (a.Cn) {
        case 16: hipLaunchKernelGGL(pool_linear_ln_k<1>, grid, dim3(256), 0, s, a); break;
        case 32: hipLaunchKernelGGL(pool_linear_ln_k<2>, grid, dim3(256), 0, s, a); break;
        case 48: hipLaunchKernelGGL(pool_linear_ln_k<3>, grid, dim3(256), 0, s, a); break;
        case 64: hipLaunchKernelGGL(pool_linear_ln_k<4>, grid, dim3(256), 0, s, a); break;
        case 96: hipLaunchKernelGGL(pool_linear_ln_k<6>, grid, dim3(256), 0, s, a); break;
        case 128: hipLaunchKernelGGL(pool_linear_ln_k<8>, grid, dim3(256), 0, s, a); break;
        case 192: hipLaunchKernelGGL(pool_linear_ln_k<12>, grid, dim3(256), 0, s, a); break;
        case 256: hipLaunchKernelGGL(pool_linear_ln_k<16>, grid, dim3(256), 0, s, a); break;
        default: return fail(PMG_E_INVALID, "unsupported level width " + std::to_string(a.Cn));
    }
    return check_launch("pool_linear_ln_k");
}

// NearestUp as one kernel (int8): for each fine voxel i, the codes of its parent's coarse row (quant_rows_k's
// arithmetic) times the up linear (gemm_i8_k's EPI_BIAS), plus the skip row (rows_ln_k's UP gather: lin[parent] +
// skip), written as the fine fp32 row, then the next block's LayerNorm -> SiLU -> int8 codes when the level has a
// block. The linear runs per fine voxel instead of once per coarse voxel (a parent has 1.7-4 children on Model A):
// the MFMA work is small, and the coarse linear's fp32 rows are neither written nor read back.
struct UpLinArgs {
    const float* cur;       // coarse level [cap][Cs] fp32
    int Cs, Ct;
    const int32_t* parent;  // fine voxel -> coarse row
    const int64_t* count;   // fine voxel count (device)
    float in_mult;          // the up linear's input quantisation
    const int8_t* w;        // [Ct][Cs]
    float a_scale;
    const float* w_scale;   // [Ct]
    const float* bias;      // [Ct] or NULL
    const float* skip;      // fine [cap][Ct] fp32 (the encoder side's row)
    float* y_out;           // fine [cap][Ct] fp32
    const float* gamma;     // next block's LayerNorm, or NULL (no codes)
    const float* beta;
    float ln_mult;
    int8_t* codes;          // fine [cap][Ct]
};

template <int NB>
__global__ __launch_bounds__(256) void up_linear_ln_k(UpLinArgs a) {
    constexpr int CT = 16 * NB;
    constexpr int LDW = CT + 4;  // LDS tile row stride (floats)
    __shared__ float tile[4][16 * LDW];
    const int64_t rows = *a.count;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r = lane & 15, gq = lane >> 4;
    const int nchunk = a.Cs >> 4;  // 16-channel chunks of a coarse row
    const int rowb = a.Cs;         // bytes per weight row
    float* tl = tile[wv];
    for (int64_t mb = blockIdx.x; mb * 64 < rows; mb += gridDim.x) {
        const int64_t m0 = (mb * 4 + wv) * 16;
        if (m0 >= rows) break;
        const int64_t i = m0 + r;
        const bool row_ok = i < rows;
        const int64_t par = row_ok ? (int64_t)a.parent[i] : 0;
        v4i acc[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[j] = v4i{0, 0, 0, 0};
        for (int q0 = 0; q0 < nchunk; q0 += 4) {
            const int ch = q0 + gq;  // this lane group's 16-channel chunk
            const bool on = ch < nchunk;
            const int qc = on ? ch : nchunk - 1;
            v4i bv[NB];
#pragma unroll
            for (int j = 0; j < NB; ++j) bv[j] = *(const v4i*)(a.w + (int64_t)(16 * j + r) * rowb + qc * 16);
            const float* src = a.cur + par * a.Cs + 16 * qc;
            float4 f[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) f[v] = *(const float4*)(src + 4 * v);
            v4i av;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float h[4] = {f[v].x, f[v].y, f[v].z, f[v].w};
                av[v] = (int)pack_codes4(h, a.in_mult);
            }
            if (!(on && row_ok)) av = v4i{0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < NB; ++j)
                acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, on ? bv[j] : v4i{0, 0, 0, 0}, acc[j], 0, 0, 0);
        }
        // lin = (acc * a_scale) * w_scale[n] + bias[n] (gemm_i8_k's EPI_BIAS), through LDS into the row layout
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int n = 16 * j + r;
            const float ws = a.w_scale[n], bs = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float y = (float)acc[j][q] * a.a_scale;
                y = y * ws;
                if (a.bias) y = y + bs;
                tl[(4 * gq + q) * LDW + n] = y;
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's tile writes are in LDS
        __builtin_amdgcn_wave_barrier();
        const int64_t io = row_ok ? i : 0;
        float y[NB][4];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const float4 v = *(const float4*)(tl + r * LDW + 16 * j + 4 * gq);
            const float4 k = *(const float4*)(a.skip + io * CT + 16 * j + 4 * gq);
            y[j][0] = v.x + k.x;
            y[j][1] = v.y + k.y;
            y[j][2] = v.z + k.z;
            y[j][3] = v.w + k.w;
            if (row_ok) *(float4*)(a.y_out + i * CT + 16 * j + 4 * gq) = make_float4(y[j][0], y[j][1], y[j][2], y[j][3]);
        }
        __builtin_amdgcn_wave_barrier();  // every lane has read the tile before the next trip writes it
        if (!a.gamma) continue;
        ln_silu_quad<NB, false>(y, a.gamma, a.beta, 1e-6f, gq);
        uint32_t pk[NB];
        silu_codes_packed<NB>(y, a.ln_mult, pk);
        if (row_ok) {
#pragma unroll
            for (int j = 0; j < NB; ++j) *(uint32_t*)(a.codes + i * CT + 16 * j + 4 * gq) = pk[j];
        }
    }
}

static int launch_up_linear_ln(const UpLinArgs& a, int64_t cap, hipStream_t s) {
    if (cap == 0) return PMG_OK;
    PMG_REQUIRE(a.Cs % 16 == 0 && a.Cs > 0, "up linear input width must be a multiple of 16");
    const dim3 grid(row_grid(cap * 4));  // 64 fine rows (256 threads) per block, grid-stride
    switch (a.Ct) {
        case 16: hipLaunchKernelGGL(up_linear_ln_k<1>, grid, dim3(256), 0, s, a); break;
        case 32: hipLaunchKernelGGL(up_linear_ln_k<2>, grid, dim3(256), 0, s, a); break;
        case 48: hipLaunchKernelGGL(up_linear_ln_k<3>, grid, dim3(256), 0, s, a); break;
        case 64: hipLaunchKernelGGL(up_linear_ln_k<4>, grid, dim3(256), 0, s, a); break;
        case 96: hipLaunchKernelGGL(up_linear_ln_k<6>, grid, dim3(256), 0, s, a); break;
        case 128: hipLaunchKernelGGL(up_linear_ln_k<8>, grid, dim3(256), 0, s, a); break;
        case 192: hipLaunchKernelGGL(up_linear_ln_k<12>, grid, dim3(256), 0, s, a); break;
        case 256: hipLaunchKernelGGL(up_linear_ln_k<16>, grid, dim3(256), 0, s, a); break;
        default: return fail(PMG_E_INVALID, "unsupported level width " + std::to_string(a.Ct));
    }
    return check_launch("up_linear_ln_k");
}

// PoolDown and NearestUp (int8) with the output channels split over the block's four waves, for level widths of 64,
// 128, 192 and 256 (Cn = 16 NB, NB % 4 == 0). A block takes RG groups of 16 rows at a time:
//   1. the linear's input codes -- the pooled children's mean (PoolDown: the children read from the coarse voxel's
//      child record, all of them requested at once, summed from 0 in child row order) or the parent's row (NearestUp),
//      quantised -- of each (row group, 64-channel trip) pair, formed by one wave and kept in LDS as the MFMA's A
//      operand (lane (r, g): row r, 16 codes of chunk 4 trip + g);
//   2. wave w multiplies them by its quarter of the weight rows (its B operands, loaded once per block), the
//      result (gemm_i8_k's EPI_BIAS arithmetic) goes to an LDS tile of whole rows;
//   3. each wave takes a quarter of the rows in the row layout of the LayerNorm (lane (r, g): row r, channels
//      16 j + 4 g + i; the quad-order sums of ln_silu_quad): (the skip row added,) the fp32 row written, then the
//      next block's LayerNorm -> SiLU -> int8 codes.
// The same arithmetic as pool_linear_ln_k / up_linear_ln_k, operation for operation. At the coarse levels (a few
// thousand rows) a block of one row group puts four waves on 16 rows where those kernels had one wave reading every
// weight row and walking the children one dependent load at a time.
template <bool UP, int NB, int RG, int KT>
struct RowLin4 {
    static constexpr int CN = 16 * NB, NBW = NB / 4, LDW = CN + 4, R = 16 * RG;
};

// Step 2 and 3's shared part: acc -> fp32 (a_scale, w_scale, bias) into the tile.
template <int NB, int RG, int LDW>
__device__ inline void lin4_tile(float* tile, const v4i (&acc)[RG][NB / 4], float a_scale, const float* w_scale,
                                 const float* bias, int wv, int r, int gq) {
#pragma unroll
    for (int j = 0; j < NB / 4; ++j) {
        const int n = 16 * ((NB / 4) * wv + j) + r;
        const float ws = w_scale[n], bs = bias ? bias[n] : 0.0f;
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float y = (float)acc[rg][j][i] * a_scale;
                y = y * ws;
                if (bias) y = y + bs;
                tile[(16 * rg + 4 * gq + i) * LDW + n] = y;
            }
    }
}

template <bool UP, int NB, int RG, int KT, class Args>
__global__ __launch_bounds__(256) void rowlin4_k(Args a) {
    typedef RowLin4<UP, NB, RG, KT> G;
    constexpr int CN = G::CN, NBW = G::NBW, LDW = G::LDW, R = G::R;
    __shared__ float tile[R * LDW];
    __shared__ v4i s_a[RG][KT][64];
    const int64_t rows = *a.count;
    if ((int64_t)blockIdx.x * R >= rows) return;  // before the weight loads: most of the grid has no rows
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int r = lane & 15, gq = lane >> 4;
    int Kin;
    if constexpr (UP) Kin = a.Cs;
    else Kin = a.Ck;
    const int nchunk = Kin >> 4;  // 16-channel chunks of an input row
    // this wave's B operands: W[16 (NBW wv + j) + r][chunk 4 t + g], every trip
    v4i bw[KT][NBW];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
        const int ch = 4 * t + gq;
#pragma unroll
        for (int j = 0; j < NBW; ++j)
            bw[t][j] = ch < nchunk ? *(const v4i*)(a.w + (int64_t)(16 * (NBW * wv + j) + r) * Kin + 16 * ch)
                                   : v4i{0, 0, 0, 0};
    }
    // step 3's rows: wave w takes rows [w R/4, (w + 1) R/4); lanes with r >= R/4 repeat a row and store nothing
    constexpr int RW = R / 4;
    const int lr = wv * RW + (r % RW);
    const bool lact = r < RW;
    for (int64_t mb = blockIdx.x; mb * R < rows; mb += gridDim.x) {
        const int64_t m0 = mb * R;
        // ---- 1. input codes of (row group, trip) tasks
        for (int task = wv; task < RG * KT; task += 4) {
            const int rg = RG == 1 ? 0 : task % RG, t = RG == 1 ? task : task / RG;
            const int64_t o = m0 + 16 * rg + r;
            const bool row_ok = o < rows;
            const int ch = 4 * t + gq;
            const bool on = row_ok && ch < nchunk;
            v4i av = v4i{0, 0, 0, 0};
            if constexpr (UP) {
                const int64_t par = row_ok ? (int64_t)a.parent[o] : 0;
                const float* src = a.cur + par * a.Cs + 16 * (ch < nchunk ? ch : nchunk - 1);
                float4 f[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) f[v] = *(const float4*)(src + 4 * v);
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float h[4] = {f[v].x, f[v].y, f[v].z, f[v].w};
                    av[v] = (int)pack_codes4(h, a.in_mult);
                }
                if (!on) av = v4i{0, 0, 0, 0};
            } else {
                const int4 ci = a.child[row_ok ? o : 0];
                const int32_t cr[4] = {ci.x, ci.y, ci.z, ci.w};
                int head[4], nc[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    head[q] = cr[q] & 0x3fffffff;
                    nc[q] = (int)((uint32_t)cr[q] >> 30);
                }
                if (on) {
                    // the children's 16 channels, two child columns' worth requested at a time, added in child
                    // row order
                    float h[16];
#pragma unroll
                    for (int e = 0; e < 16; ++e) h[e] = 0.0f;
#pragma unroll
                    for (int qp = 0; qp < 4; qp += 2) {
                        float4 f[2][2][4];
#pragma unroll
                        for (int q = 0; q < 2; ++q)
#pragma unroll
                            for (int i = 0; i < 2; ++i) {
                                const int cq = qp + q;
                                const float* src = a.x + (int64_t)(i < nc[cq] ? head[cq] + i : 0) * a.Ck + 16 * ch;
#pragma unroll
                                for (int v = 0; v < 4; ++v) f[q][i][v] = *(const float4*)(src + 4 * v);
                            }
#pragma unroll
                        for (int q = 0; q < 2; ++q)
#pragma unroll
                            for (int i = 0; i < 2; ++i)
                                if (i < nc[qp + q]) {
#pragma unroll
                                    for (int v = 0; v < 4; ++v) {
                                        h[4 * v + 0] = h[4 * v + 0] + f[q][i][v].x;
                                        h[4 * v + 1] = h[4 * v + 1] + f[q][i][v].y;
                                        h[4 * v + 2] = h[4 * v + 2] + f[q][i][v].z;
                                        h[4 * v + 3] = h[4 * v + 3] + f[q][i][v].w;
                                    }
                                }
                    }
                    const float cnt = (float)(nc[0] + nc[1] + nc[2] + nc[3]);
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float m4[4] = {h[4 * v] / cnt, h[4 * v + 1] / cnt, h[4 * v + 2] / cnt,
                                             h[4 * v + 3] / cnt};
                        av[v] = (int)pack_codes4(m4, a.pool_mult);
                    }
                }
            }
            s_a[rg][t][lane] = av;
        }
        const int64_t o3 = m0 + lr;
        const bool ok3 = lact && o3 < rows;
        __syncthreads();
        // ---- 2. this wave's quarter of the output channels
        v4i acc[RG][NBW];
#pragma unroll
        for (int rg = 0; rg < RG; ++rg)
#pragma unroll
            for (int j = 0; j < NBW; ++j) acc[rg][j] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < KT; ++t)
#pragma unroll
            for (int rg = 0; rg < RG; ++rg) {
                const v4i av = s_a[rg][t][lane];
#pragma unroll
                for (int j = 0; j < NBW; ++j)
                    acc[rg][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bw[t][j], acc[rg][j], 0, 0, 0);
            }
        lin4_tile<NB, RG, LDW>(tile, acc, a.a_scale, a.w_scale, a.bias, wv, r, gq);
        __syncthreads();
        // ---- 3. whole rows: (skip,) the fp32 row, LayerNorm codes
        float y[NB][4];
        float4 sk[UP ? NB : 1];
        if constexpr (UP) {  // the skip rows (NearestUp)
            const int64_t io = o3 < rows ? o3 : 0;
#pragma unroll
            for (int j = 0; j < NB; ++j) sk[j] = *(const float4*)(a.skip + io * CN + 16 * j + 4 * gq);
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const float4 v = *(const float4*)(tile + lr * LDW + 16 * j + 4 * gq);
            if constexpr (UP) {
                y[j][0] = v.x + sk[j].x;
                y[j][1] = v.y + sk[j].y;
                y[j][2] = v.z + sk[j].z;
                y[j][3] = v.w + sk[j].w;
            } else {
                y[j][0] = v.x;
                y[j][1] = v.y;
                y[j][2] = v.z;
                y[j][3] = v.w;
            }
            if (ok3) *(float4*)(a.y_out + o3 * CN + 16 * j + 4 * gq) = make_float4(y[j][0], y[j][1], y[j][2], y[j][3]);
        }
        if (a.gamma) {
            ln_silu_quad<NB, false>(y, a.gamma, a.beta, 1e-6f, gq);
            uint32_t pk[NB];
            silu_codes_packed<NB>(y, a.ln_mult, pk);
            if (ok3) {
#pragma unroll
                for (int j = 0; j < NB; ++j) *(uint32_t*)(a.codes + o3 * CN + 16 * j + 4 * gq) = pk[j];
            }
        }
        __syncthreads();  // the tile and the input codes are rewritten by the next trip
    }
}

// Row groups per block of rowlin4_k on level k: one (16-row blocks) when the level is expected to hold at most 4096
// rows -- a surface keeps about 2 cap / 4^k voxels on level k -- so that its few rows still spread over the CUs (at
// 16 NB = 256 channels the LayerNorm's registers leave one block per CU); else four (64-row blocks: the weight
// operands of a block are reused over four row tiles and every lane of the LayerNorm phase holds a row). Measured on
// the A-shape U-Net (levels 1-4: 183582, 48758, 11016, 2567 rows): PoolDown into level 4 20 us with one row group,
// 29 us with four; every other PoolDown / NearestUp faster with four.
static bool rowlin4_rg4(int64_t cap, int k) { return (2 * cap >> (2 * k)) > 4096; }

// Launch of rowlin4_k when it takes the widths (Cout a multiple of 64 up to 256, Cin up to 256); returns -1 when it
// does not (the caller launches the one-wave-per-16-rows kernel). rg4: four row groups per block (levels with many
// rows), else one.
template <bool UP, class Args>
static int launch_rowlin4(const Args& a, int Cin, int Cout, bool rg4, int64_t cap, hipStream_t s) {
    if (Cout % 64 != 0 || Cout > 256 || Cin % 16 != 0 || Cin > 256) return -1;
    const int KT = (Cin / 16 + 3) / 4, NB = Cout / 16;
    const int R = rg4 ? 64 : 16;
    int64_t blocks = (cap + R - 1) / R;
    if (blocks > kRowBlocksMax) blocks = kRowBlocksMax;
    const dim3 grid((unsigned)blocks);
#define PMG_RL4(NBV, RGV, KTV) \
    if (NB == NBV && (rg4 ? 4 : 1) == RGV && KT == KTV) { \
        hipLaunchKernelGGL((rowlin4_k<UP, NBV, RGV, KTV, Args>), grid, dim3(256), 0, s, a); \
        return check_launch(UP ? "rowlin4_k (up)" : "rowlin4_k (pool)"); \
    }
#define PMG_RL4_KT(NBV, RGV) PMG_RL4(NBV, RGV, 1) PMG_RL4(NBV, RGV, 2) PMG_RL4(NBV, RGV, 3) PMG_RL4(NBV, RGV, 4)
    PMG_RL4_KT(4, 1) PMG_RL4_KT(4, 4) PMG_RL4_KT(8, 1) PMG_RL4_KT(8, 4)
    PMG_RL4_KT(12, 1) PMG_RL4_KT(12, 4) PMG_RL4_KT(16, 1) PMG_RL4_KT(16, 4)
#undef PMG_RL4_KT
#undef PMG_RL4
    return -1;
}

static int launch_gemm(const GemmArgs& g, int epi, bool f16, hipStream_t s, bool narrow = false) {
    PMG_REQUIRE(g.K % 16 == 0 && g.N % 16 == 0 && g.K > 0 && g.N > 0, "GEMM sizes must be multiples of 16");
    if (g.rows_cap == 0) return PMG_OK;
    const int b = g.N / 16;
    const int nb = narrow ? 1 : (b % 4 == 0 ? 4 : (b % 2 == 0 ? 2 : 1));
    const unsigned gy = (unsigned)(g.N / (16 * nb));
    int64_t gx = (g.rows_cap + 63) / 64;
    const int64_t gx_max = kRowBlocksMax / gy > 0 ? kRowBlocksMax / gy : 1;  // device-sized rows: grid-stride
    if (g.rows_dev && gx > gx_max) gx = gx_max;
    const dim3 grid((unsigned)gx, gy);
#define PMG_GEMM_CASE(NBV)                                                                                \
    if (nb == NBV) {                                                                                      \
        if (f16) {                                                                                        \
            if (epi == PMG_EPI_Q)                                                                         \
                hipLaunchKernelGGL((gemm_i8_k<NBV, PMG_EPI_Q, _Float16>), grid, dim3(256), 0, s, g);      \
            else                                                                                          \
                hipLaunchKernelGGL((gemm_i8_k<NBV, PMG_EPI_BIAS, _Float16>), grid, dim3(256), 0, s, g);   \
        } else if (epi == PMG_EPI_Q) {                                                                    \
            hipLaunchKernelGGL((gemm_i8_k<NBV, PMG_EPI_Q>), grid, dim3(256), 0, s, g);                    \
        } else {                                                                                          \
            hipLaunchKernelGGL((gemm_i8_k<NBV, PMG_EPI_BIAS>), grid, dim3(256), 0, s, g);                 \
        }                                                                                                 \
    }
    PMG_GEMM_CASE(4)
    PMG_GEMM_CASE(2)
    PMG_GEMM_CASE(1)
#undef PMG_GEMM_CASE
    return check_launch("gemm_i8_k");
}

#define PMG_LN_SWITCH(C, BODY)                                                                  \
    switch (C) {                                                                                \
        case 16: { constexpr int CC = 16; BODY; break; }                                       \
        case 32: { constexpr int CC = 32; BODY; break; }                                       \
        case 48: { constexpr int CC = 48; BODY; break; }                                       \
        case 64: { constexpr int CC = 64; BODY; break; }                                       \
        case 96: { constexpr int CC = 96; BODY; break; }                                       \
        case 128: { constexpr int CC = 128; BODY; break; }                                     \
        case 192: { constexpr int CC = 192; BODY; break; }                                     \
        case 256: { constexpr int CC = 256; BODY; break; }                                     \
        case 512: { constexpr int CC = 512; BODY; break; }                                     \
        default: return fail(PMG_E_INVALID, "unsupported level width " + std::to_string(C));   \
    }

// Level widths: int8 16 .. 256 (the deployed refiners); the fp16 teacher also 512 (the stock refiner's deepest
// level, train.py:124), on the generic convolution. Level 0: the map-free convolutions' widths.
static bool unet_width(int C, int prec) {
    return C == 16 || C == 32 || C == 48 || C == 64 || C == 96 || C == 128 || C == 192 || C == 256 ||
           (prec == PMG_PREC_FP16 && C == 512);
}
static bool col_width(int C, int prec) {
    return C == 16 || C == 32 || C == 48 || C == 64 || (prec == PMG_PREC_INT8 && C == 128);
}

static int launch_rows_ln(bool up, int C, const float* x, const int32_t* parent, const float* skip,
                          const int64_t* count, int64_t cap, const float* gamma, const float* beta, float mult,
                          float* y_out, void* codes, bool f16, hipStream_t s) {
    if (cap == 0) return PMG_OK;
    const dim3 grid(row_grid(cap * 4));  // 64 rows (256 threads) per block, grid-stride
    if (f16) {
        _Float16* c16 = (_Float16*)codes;
        if (up) {
            PMG_LN_SWITCH(C, hipLaunchKernelGGL((rows_ln_k<CC, true, _Float16>), grid, dim3(256), 0, s, x, parent,
                                                skip, count, gamma, beta, 1e-6f, mult, y_out, c16));
        } else {
            PMG_LN_SWITCH(C, hipLaunchKernelGGL((rows_ln_k<CC, false, _Float16>), grid, dim3(256), 0, s, x, parent,
                                                skip, count, gamma, beta, 1e-6f, mult, y_out, c16));
        }
    } else {
        int8_t* c8 = (int8_t*)codes;
        if (C > 256) return fail(PMG_E_INVALID, "int8 level widths end at 256");
        if (up) {
            PMG_LN_SWITCH(C, hipLaunchKernelGGL((rows_ln_k<CC, true, int8_t>), grid, dim3(256), 0, s, x, parent,
                                                skip, count, gamma, beta, 1e-6f, mult, y_out, c8));
        } else {
            PMG_LN_SWITCH(C, hipLaunchKernelGGL((rows_ln_k<CC, false, int8_t>), grid, dim3(256), 0, s, x, parent,
                                                skip, count, gamma, beta, 1e-6f, mult, y_out, c8));
        }
    }
    return check_launch("rows_ln_k");
}

}  // namespace pmg

using namespace pmg;

// ---------------------------------------------------------------------------------------------------------------
// The U-Net context: one arena holding every level's structure and activations at the level-0 capacity.
struct pmg_unet {
    pmg_unet_config cfg{};
    int L = 0;
    int64_t cap = 0;              // level-0 voxels = B * H * W, the capacity of every level
    int Hk[kMaxLevels], Wk[kMaxLevels];
    int64_t ncols[kMaxLevels];    // B * Hk * Wk
    int R = 0, Cc = 0;            // encoder token grid
    int64_t T = 0;                // tokens B * R * Cc
    int Cmax = 0;

    void* arena = nullptr;
    size_t arena_bytes = 0;
    int64_t* counts = nullptr;    // [L] voxels per level (device)
    int32_t* zq0 = nullptr;       // level-0 keys [cap]
    int32_t* zmin = nullptr;      // [B] (and zmax [B])
    int4* coords0 = nullptr;      // level-0 coordinates when not given
    int4* coords[kMaxLevels] = {};      // [cap] (level 0: the caller's or coords0)
    int32_t* off[kMaxLevels] = {};      // column CSR [ncols + 1] (level 0: NULL)
    int32_t* parent[kMaxLevels] = {};   // level k -> k + 1 [cap]
    int4* child[kMaxLevels] = {};       // level k + 1 -> its children on level k [cap] (pool_emit_k)
    int32_t* nmap_t[kMaxLevels] = {};   // [27][cap] (levels >= 1)
    uint32_t* tmask[kMaxLevels] = {};   // [cap / 16 + 1]
    float* xd[kMaxLevels] = {};         // down-stage stream = skip [cap][C_k]
    float* xu[kMaxLevels] = {};         // up-stage stream [cap][C_k] (k < L - 1)
    float* xb = nullptr;                // bottleneck stream [cap][C_L]
    int32_t* scan_excl = nullptr;       // [max ncols]: a column's first row within its block of 256 columns
    int32_t* scan_tiles = nullptr;      // [max ncols / 256 + 1]: each block's voxel total
    // activations entering a convolution or a linear: int8 codes, or fp16 (the teacher)
    void* q1 = nullptr;                 // [cap][Cmax]
    void* q2 = nullptr;
    void* codes = nullptr;              // linear inputs [cap][max(2 C_L, Cmax)]
    void* codes2 = nullptr;             // fuse_proj.2 input [cap][C_L]
    float* lin = nullptr;               // NearestUp linear output [cap][Cmax]
    void* enc_codes = nullptr;          // [T][enc_channels]
    float* enc_tok = nullptr;           // [T][C_L]
    int32_t* part = nullptr;            // tap-split partial sums of the coarsest level's convolutions
    int64_t part_bytes = 0;

    // pmg_unet_step: its own workspace (the prompt / anchor fit, the final fit, the fits' (s, t)), allocated by
    // pmg_unet_step_prepare
    bool step_ready = false;
    pmg_unet_step_config scfg{};
    void* step_arena = nullptr;
    void* fit_ws[2] = {nullptr, nullptr};  // prompt (and anchor) fit, final fit
    size_t fit_ws_bytes[2] = {0, 0};
    float* st_scratch = nullptr;           // [3][B][2]: prompt, final, anchor (s, t)

    bool have_weights = false;
    const float* in_w = nullptr;
    const float* in_b = nullptr;
    const float* pr_w = nullptr;
    const float* pr_b = nullptr;
    const float* out_w = nullptr;
    const float* out_b = nullptr;
    std::vector<pmg_block_weights> down[kMaxLevels], dec[kMaxLevels], bott;
    std::vector<pmg_linear_weights> pool, up;
    pmg_linear_weights enc{}, fuse0{}, fuse2{};

    // the level structure is built on a side stream beside the level-0 layers (a parallel branch of the captured
    // graph): fork after the level-0 coordinates, join before each level's first use
    hipStream_t side = nullptr;
    hipEvent_t ev_fork = nullptr;
    hipEvent_t ev_level[kMaxLevels] = {};
    hipEvent_t ev_enc = nullptr;  // the encoder tokens (also made on the side stream)

    GraphCache graphs;
};

static size_t ualign(size_t v) { return (v + 255) & ~(size_t)255; }

// Where the network's last convolution (a level-0 block) puts out_proj: the module's (M, 1) output `delta`
// (sparse_unet.py:258), or -- the refine step -- logz + delta into the point map points_out (v3.py:359), scaled by the
// output gate when gate_lidar is set (v3.py:565-569).
struct UnetOut {
    float* delta = nullptr;
    const float* points = nullptr;
    float* points_out = nullptr;
    const float* gate_lidar = nullptr;
    const float* gate_conf = nullptr;
    int gate_dh = 0, gate_dw = 0;
    float gate_floor = 0.0f, gate_scale = 0.0f;
};

// One residual block on level k (flex_sparse_blocks.py:70-75) whose conv1 input codes are in u->q1 and whose stream
// is x (updated in place). After conv2: the next block's LayerNorm codes (level 0: fused RLN epilogue; else the row
// kernel), nothing, or (last level-0 block of the network) out_proj into `rout`.
static int enqueue_block(pmg_unet* u, int k, const pmg_block_weights& bk, const pmg_block_weights* next, float* x,
                         const UnetOut* rout, hipStream_t s) {
    const int C = u->cfg.channels[k];
    const bool f16 = u->cfg.precision == PMG_PREC_FP16;
    const int prec = f16 ? PMG_PREC_FP16 : PMG_PREC_INT8;
    if (k == 0) {
        ColConvArgs a1{};
        a1.x = u->q1;
        a1.zq = u->zq0;
        a1.w = bk.w1;
        a1.M = u->cap;
        a1.H = u->cfg.H;
        a1.W = u->cfg.W;
        a1.a_scale = bk.a1_scale;
        a1.w_scale = bk.w1_scale;
        a1.bias = bk.b1;
        a1.out_mult = bk.q2_mult;
        a1.out = u->q2;
        if (int e = launch_conv_col(prec, a1, C, PMG_EPI_Q, s)) return e;
        ColConvArgs a2{};
        a2.x = u->q2;
        a2.zq = u->zq0;
        a2.w = bk.w2;
        a2.M = u->cap;
        a2.H = u->cfg.H;
        a2.W = u->cfg.W;
        a2.a_scale = bk.a2_scale;
        a2.w_scale = bk.w2_scale;
        a2.bias = bk.b2;
        a2.skip = x;
        a2.out = x;
        if (next) {
            a2.ln_gamma = next->ln_gamma;
            a2.ln_beta = next->ln_beta;
            a2.ln_eps = 1e-6f;
            a2.next_mult = next->q1_mult;
            a2.next_q = u->q1;
            return launch_conv_col(prec, a2, C, PMG_EPI_RLN, s);
        }
        if (rout) {
            a2.out_w = u->out_w;
            a2.out_b = u->out_b;
            if (rout->delta) {
                a2.out = rout->delta;
            } else {
                a2.points = rout->points;
                a2.points_out = rout->points_out;
                a2.gate_lidar = rout->gate_lidar;
                a2.gate_conf = rout->gate_conf;
                a2.gate_dh = rout->gate_dh;
                a2.gate_dw = rout->gate_dw;
                a2.gate_floor = rout->gate_floor;
                a2.gate_scale = rout->gate_scale;
            }
            return launch_conv_col(prec, a2, C, PMG_EPI_ROUT, s);
        }
        return launch_conv_col(prec, a2, C, PMG_EPI_R, s);
    }
    DevConv c1{};
    c1.x = (const int8_t*)u->q1;
    c1.nmap_t = u->nmap_t[k];
    c1.tile_mask = u->tmask[k];
    c1.cap = u->cap;
    c1.m_dev = u->counts + k;
    c1.Ci = C;
    c1.Co = C;
    c1.w = (const int8_t*)bk.w1;
    c1.epilogue = f16 ? PMG_EPI_SILU : PMG_EPI_Q;
    c1.a_scale = bk.a1_scale;
    c1.w_scale = bk.w1_scale;
    c1.bias = bk.b1;
    c1.out_mult = bk.q2_mult;
    c1.out = u->q2;
    // the tap split (a second launch) only at the coarsest level: the capacity does not bound a level's rows, and
    // at the finer levels, with too many rows to split, that launch would only cost its dispatch
    if (k == u->L - 1 && k > 0 && !f16) {
        c1.part = u->part;
        c1.part_bytes = u->part_bytes;
    }
    auto conv = [&](const DevConv& d) { return f16 ? launch_conv_f16_dev(d, s) : launch_conv_i8_dev(d, s); };
    if (int e = conv(c1)) return e;
    DevConv c2 = c1;
    c2.x = (const int8_t*)u->q2;
    c2.w = (const int8_t*)bk.w2;
    c2.epilogue = PMG_EPI_R;
    c2.a_scale = bk.a2_scale;
    c2.w_scale = bk.w2_scale;
    c2.bias = bk.b2;
    c2.skip = x;
    c2.out = x;
    if (int e = conv(c2)) return e;
    if (next)
        return launch_rows_ln(false, C, x, nullptr, nullptr, u->counts + k, u->cap, next->ln_gamma, next->ln_beta,
                              next->q1_mult, nullptr, u->q1, f16, s);
    return PMG_OK;
}

// A stage of blocks on level k over stream x, whose first block's input codes are already in q1.
static int enqueue_stage(pmg_unet* u, int k, const std::vector<pmg_block_weights>& st, float* x, const UnetOut* rout,
                         hipStream_t s) {
    for (size_t j = 0; j < st.size(); ++j) {
        const pmg_block_weights* next = j + 1 < st.size() ? &st[j + 1] : nullptr;
        if (int e = enqueue_block(u, k, st[j], next, x, next ? nullptr : rout, s)) return e;
    }
    return PMG_OK;
}

static int ln_codes(pmg_unet* u, int k, const float* x, const pmg_block_weights& b, hipStream_t s) {
    return launch_rows_ln(false, u->cfg.channels[k], x, nullptr, nullptr, u->counts + k, u->cap, b.ln_gamma,
                          b.ln_beta, b.q1_mult, nullptr, u->q1, u->cfg.precision == PMG_PREC_FP16, s);
}

static int linear(pmg_unet* u, const void* a, const int64_t* rows_dev, int64_t rows_cap, int K,
                  const pmg_linear_weights& lw, int N, int epi, float out_mult, void* out, const float* planar,
                  hipStream_t s, bool narrow = false) {
    GemmArgs g{a, lw.w, rows_cap, rows_dev, K, N, lw.a_scale, lw.w_scale, lw.bias, out_mult, out, planar,
               (int64_t)u->R * u->Cc};
    return launch_gemm(g, epi, u->cfg.precision == PMG_PREC_FP16, s, narrow);
}

// The level structure (levels 1 .. L-1) from the level-0 coordinates; with `done`, level k + 1's event is recorded
// after its kernels.
static int enqueue_structure(pmg_unet* u, hipStream_t s, hipEvent_t* done = nullptr) {
    for (int k = 0; k + 1 < u->L; ++k) {
        PoolGeom g{u->coords[k], u->off[k], u->cfg.B, u->Hk[k], u->Wk[k], u->Hk[k + 1], u->Wk[k + 1]};
        const int64_t nc = u->ncols[k + 1];
        const unsigned gb = (unsigned)((nc + 255) / 256);
        hipLaunchKernelGGL(pool_count_k, dim3(gb), dim3(256), 0, s, g, nc, u->scan_excl, u->scan_tiles);
        if (int e = check_launch("pool_count_k")) return e;
        hipLaunchKernelGGL(pool_emit_k, dim3(gb), dim3(256), 0, s, g, nc, u->scan_excl, u->scan_tiles,
                           u->counts + k + 1, u->coords[k + 1], u->off[k + 1], u->parent[k], u->child[k]);
        if (int e = check_launch("pool_emit_k")) return e;
        hipLaunchKernelGGL(nmap_level_k, dim3((unsigned)((u->cap + 255) / 256)), dim3(256), 0, s, u->coords[k + 1],
                           u->off[k + 1], u->counts + k + 1, u->Hk[k + 1], u->Wk[k + 1], u->cap, u->nmap_t[k + 1],
                           u->tmask[k + 1]);
        if (int e = check_launch("nmap_level_k")) return e;
        if (done) PMG_CHECK_HIP(hipEventRecord(done[k + 1], s));
    }
    return PMG_OK;
}

// The prompt features of the refine step, computed per voxel in the input stage from the LiDAR in the affine frame of
// the prompt fit's (s, t) (v3.py:548-555, 362-383).
struct UnetPrompt {
    const float* lidar = nullptr;
    const float* conf = nullptr;
    int dh = 0, dw = 0;
    const float* st = nullptr;
    int soft_gate = 0;
};

// Sparse3DUNet.forward (sparse_unet.py:176-258) on level-0 voxels; out_proj goes to `rout`. The prompt features are
// the given `prompt` [M][2], or computed from `lp` (the refine step), or absent.
static int enqueue_unet(pmg_unet* u, const float* feats, const int32_t* coords, const float* prompt,
                        const UnetPrompt* lp, const float* enc_feat, const float* enc_bias, const UnetOut& rout,
                        hipStream_t s) {
    const pmg_unet_config& c = u->cfg;
    const int L = u->L;
    const int64_t cap = u->cap;
    // level 0: keys and coordinates (the caller's, or _voxelize's from the log depth)
    if (coords) {
        hipLaunchKernelGGL(copy_coords_k, dim3((unsigned)((cap + 255) / 256)), dim3(256), 0, s, (const int4*)coords,
                           cap, u->coords0);
        if (int e = check_launch("copy_coords_k")) return e;
    } else {
        if (int e = pmg_voxelize(feats + 2, 3, c.B, c.H, c.W, c.depth_resolution, u->zq0, u->zmin, u->zmin + c.B, s))
            return e;
        hipLaunchKernelGGL(level0_coords_k, dim3((unsigned)((cap + 255) / 256)), dim3(256), 0, s, u->zq0, u->zmin,
                           c.H, c.W, cap, u->coords0);
        if (int e = check_launch("level0_coords_k")) return e;
    }
    u->coords[0] = u->coords0;
    const int32_t* zkeys = (const int32_t*)u->coords0 + 3;
    // input_proj (+ prompt_proj), the level-0 keys, and the first block's codes (sparse_unet.py:189-192)
    const pmg_block_weights* first = !u->down[0].empty() ? &u->down[0][0] : nullptr;
    InputStage in{};
    in.points = feats;
    in.B = c.B;
    in.H = c.H;
    in.W = c.W;
    in.C = c.channels[0];
    in.dh = c.H;
    in.dw = c.W;
    in.in_w = u->in_w;
    in.in_b = u->in_b;
    in.pr_w = u->pr_w;
    in.pr_b = u->pr_b;
    in.x_out = u->xd[0];
    in.gamma = first ? first->ln_gamma : u->in_b;  // without a level-0 block the codes are not read
    in.beta = first ? first->ln_beta : u->in_b;
    in.eps = 1e-6f;
    in.out_mult = first ? first->q1_mult : 1.0f;
    in.q_out = u->q1;
    in.resolution = c.depth_resolution;
    in.zq_out = u->zq0;
    in.prompt_in = prompt;
    in.use_prompt = prompt != nullptr;
    if (lp && lp->st) {
        in.lidar = lp->lidar;
        in.conf = lp->conf;
        in.dh = lp->dh;
        in.dw = lp->dw;
        in.st = lp->st;
        in.soft_gate = lp->soft_gate;
        in.use_prompt = 1;
    }
    in.zkeys = zkeys;
    in.zkey_stride = 4;
    const bool f16 = c.precision == PMG_PREC_FP16;
    // The level structure on a side stream, concurrent with the input stage and the level-0 blocks. The input
    // stage is enqueued right after the fork, before the side stream's work: a graph replay keeps the first
    // successor of a node on that node's queue, and the input stage heads the critical path (enqueued after the
    // structure, it started ~40 us after the level-0 coordinates it waits for). Measured on one box, three
    // alternating runs each: forward 1.150-1.165 -> 1.145-1.150 ms. Building level 1's structure on this stream
    // instead (1.164-1.166 ms), or levels 1 and 2.. on two side streams (1.144-1.146 ms), did not pay.
    PMG_CHECK_HIP(hipEventRecord(u->ev_fork, s));
    if (int e = launch_input_stage(in, f16, s)) return e;
    PMG_CHECK_HIP(hipStreamWaitEvent(u->side, u->ev_fork, 0));
    if (int e = enqueue_structure(u, u->side, u->ev_level)) return e;
    // then, on the same side stream, the encoder conditioning's tokens: the encoder feature quantised and
    // transposed, times encoder_fuse (+ the planar bias map) per token (sparse_unet.py:160-174, 227-232)
    {
        const int CL = c.channels[L - 1];
        const dim3 grid((unsigned)(((int64_t)u->R * u->Cc + 63) / 64), (unsigned)((c.enc_channels + 63) / 64),
                        (unsigned)c.B);
        if (f16)
            hipLaunchKernelGGL(enc_quant_k<_Float16>, grid, dim3(256), 0, u->side, enc_feat, c.enc_channels,
                               (int64_t)u->R * u->Cc, 1.0f, (_Float16*)u->enc_codes);
        else
            hipLaunchKernelGGL(enc_quant_k<int8_t>, grid, dim3(256), 0, u->side, enc_feat, c.enc_channels,
                               (int64_t)u->R * u->Cc, u->enc.q_mult, (int8_t*)u->enc_codes);
        if (int e = check_launch("enc_quant_k")) return e;
        // the encoder tokens and the deepest level are a few thousand rows with long K: one 16-column block per
        // wave gives the GEMM four times the waves (Model A: encoder_fuse 20 -> 13 us, fuse_proj 30 -> 28 us)
        if (int e = linear(u, u->enc_codes, nullptr, u->T, c.enc_channels, u->enc, CL, PMG_EPI_BIAS, 0.0f,
                           u->enc_tok, enc_bias, u->side, true))
            return e;
        PMG_CHECK_HIP(hipEventRecord(u->ev_enc, u->side));
    }

    // down stages and PoolDown (sparse_unet.py:223-231; flex_sparse_blocks.py:85-90)
    for (int k = 0; k < L; ++k) {
        if (int e = enqueue_stage(u, k, u->down[k], u->xd[k], nullptr, s)) return e;
        if (k + 1 == L) break;
        PMG_CHECK_HIP(hipStreamWaitEvent(s, u->ev_level[k + 1], 0));  // level k + 1's structure is built
        const int Ck = c.channels[k], Cn = c.channels[k + 1];
        PoolGeom g{u->coords[k], u->off[k], c.B, u->Hk[k], u->Wk[k], u->Hk[k + 1], u->Wk[k + 1]};
        const pmg_block_weights* nb = !u->down[k + 1].empty() ? &u->down[k + 1][0] : nullptr;
        if (!f16) {  // pool mean + linear + the next block's LayerNorm codes in one kernel
            const pmg_linear_weights& lw = u->pool[k];
            PoolLinArgs pa{u->xd[k], Ck, Cn, g, u->coords[k + 1], u->child[k], u->counts + k + 1, lw.q_mult,
                           (const int8_t*)lw.w, lw.a_scale, lw.w_scale, lw.bias, u->xd[k + 1],
                           nb ? nb->ln_gamma : nullptr, nb ? nb->ln_beta : nullptr, nb ? nb->q1_mult : 1.0f,
                           (int8_t*)u->q1};
            const int rc = launch_rowlin4<false>(pa, Ck, Cn, rowlin4_rg4(cap, k + 1), cap, s);
            if (rc == -1) {
                if (int e = launch_pool_linear_ln(pa, cap, s)) return e;
            } else if (rc) {
                return rc;
            }
            continue;
        }
        // fp16 (the teacher): mean pool to fp16 codes, the fp16 GEMM, then the next block's LayerNorm
        hipLaunchKernelGGL(pool_quant_k<_Float16>, dim3(row_grid(cap * (Ck / 4))), dim3(256), 0, s, u->xd[k], Ck, g,
                           u->coords[k + 1], u->counts + k + 1, 1.0f, (_Float16*)u->codes);
        if (int e = check_launch("pool_quant_k")) return e;
        if (int e = linear(u, u->codes, u->counts + k + 1, cap, Ck, u->pool[k], Cn, PMG_EPI_BIAS, 0.0f, u->xd[k + 1],
                           nullptr, s))
            return e;
        if (nb)
            if (int e = ln_codes(u, k + 1, u->xd[k + 1], *nb, s)) return e;
    }

    // encoder conditioning and fuse_proj at the deepest level (sparse_unet.py:233-240)
    const int top = L - 1, CL = c.channels[top];
    {
        // the encoder tokens (enc_tok) were made on the side stream
        PMG_CHECK_HIP(hipStreamWaitEvent(s, u->ev_enc, 0));
        const bool narrow_top = top >= 2;
        if (f16)
            hipLaunchKernelGGL(concat_quant_k<_Float16>, dim3(row_grid(cap * (CL / 2))), dim3(256), 0, s,
                               u->xd[top], u->enc_tok, u->coords[top], u->counts + top, CL, u->R, u->Cc, 1.0f,
                               (_Float16*)u->codes);
        else
            hipLaunchKernelGGL(concat_quant_k<int8_t>, dim3(row_grid(cap * (CL / 2))), dim3(256), 0, s,
                               u->xd[top], u->enc_tok, u->coords[top], u->counts + top, CL, u->R, u->Cc,
                               u->fuse0.q_mult, (int8_t*)u->codes);
        if (int e = check_launch("concat_quant_k")) return e;
        if (int e = linear(u, u->codes, u->counts + top, cap, 2 * CL, u->fuse0, CL, PMG_EPI_Q, u->fuse2.q_mult,
                           u->codes2, nullptr, s, narrow_top))
            return e;
        if (int e = linear(u, u->codes2, u->counts + top, cap, CL, u->fuse2, CL, PMG_EPI_BIAS, 0.0f, u->xb, nullptr,
                           s, narrow_top))
            return e;
    }
    // bottleneck (sparse_unet.py:244-247)
    if (!u->bott.empty()) {
        if (int e = ln_codes(u, top, u->xb, u->bott[0], s)) return e;
        if (int e = enqueue_stage(u, top, u->bott, u->xb, nullptr, s)) return e;
    }
    // NearestUp + skip + up stages (sparse_unet.py:249-256; flex_sparse_blocks.py:99-105)
    float* cur = u->xb;
    for (int i = 0; i + 1 < L; ++i) {
        const int t = L - 2 - i;
        const int Cs = c.channels[t + 1], Ct = c.channels[t];
        const pmg_block_weights* fb = !u->dec[i].empty() ? &u->dec[i][0] : nullptr;
        if (!f16) {  // parent codes + linear + skip + the next block's LayerNorm codes in one kernel, per fine voxel
            const pmg_linear_weights& lw = u->up[i];
            UpLinArgs ua{cur, Cs, Ct, u->parent[t], u->counts + t, lw.q_mult, (const int8_t*)lw.w, lw.a_scale,
                         lw.w_scale, lw.bias, u->xd[t], u->xu[t], fb ? fb->ln_gamma : nullptr,
                         fb ? fb->ln_beta : nullptr, fb ? fb->q1_mult : 1.0f, (int8_t*)u->q1};
            const int rc = launch_rowlin4<true>(ua, Cs, Ct, rowlin4_rg4(cap, t), cap, s);
            if (rc == -1) {
                if (int e = launch_up_linear_ln(ua, cap, s)) return e;
            } else if (rc) {
                return rc;
            }
        } else {  // fp16 (the teacher): quantise, the fp16 GEMM at the coarse level, then the gather + LayerNorm
            hipLaunchKernelGGL(quant_rows_k<_Float16>, dim3(row_grid(cap * Cs / 4)), dim3(256), 0, s, cur, Cs,
                               u->counts + t + 1, 1.0f, (_Float16*)u->codes);
            if (int e = check_launch("quant_rows_k")) return e;
            if (int e = linear(u, u->codes, u->counts + t + 1, cap, Cs, u->up[i], Ct, PMG_EPI_BIAS, 0.0f, u->lin,
                               nullptr, s))
                return e;
            if (int e = launch_rows_ln(true, Ct, u->lin, u->parent[t], u->xd[t], u->counts + t, cap,
                                       fb ? fb->ln_gamma : nullptr, fb ? fb->ln_beta : nullptr,
                                       fb ? fb->q1_mult : 1.0f, u->xu[t], u->q1, f16, s))
                return e;
        }
        if (int e = enqueue_stage(u, t, u->dec[i], u->xu[t], t == 0 ? &rout : nullptr, s)) return e;
        cur = u->xu[t];
    }
    return PMG_OK;
}

// One refine-loop step with the multi-level refiner (v3.py:547-576, the device engine's order Refiner.swift:224-292):
// prompt fit -> (residual, gate) prompt features -> _voxelize -> structure -> Sparse3DUNet -> logz + delta (output
// gate) -> elastic anchor -> final metric fit -> post_depth. points_out may alias points.
static int enqueue_unet_step(pmg_unet* u, const float* points, float* points_out, const float* lidar,
                             const float* conf, const float* enc_feat, const float* enc_bias, float* st_prompt,
                             float* st_final, float* depth, hipStream_t s) {
    const pmg_unet_config& c = u->cfg;
    const pmg_unet_step_config& q = u->scfg;
    const int B = c.B;
    float* const st_p = st_prompt ? st_prompt : u->st_scratch;
    float* const st_f = st_final ? st_final : u->st_scratch + 2 * B;
    float* const st_a = u->st_scratch + 4 * B;
    auto prompt_fit = [&](const float* pts, float* st) {
        FitLaunch f{};
        f.mode = 1;
        f.logz = pts + 2;
        f.stride = 3;
        f.lidar = lidar;
        f.conf = conf;
        f.B = B;
        f.H = c.H;
        f.W = c.W;
        f.dh = q.dh;
        f.dw = q.dw;
        f.N = (int64_t)c.H * c.W;
        f.iters = q.fit_iters;
        f.trim = q.fit_trim;
        f.min_points = q.fit_min_points;
        f.st = st;
        f.info = nullptr;
        f.workspace = u->fit_ws[0];
        f.workspace_bytes = u->fit_ws_bytes[0];
        return launch_fit(f, s);
    };
    UnetPrompt lp{};
    if (q.use_prompt) {
        if (int e = prompt_fit(points, st_p)) return e;
        lp.lidar = lidar;
        lp.conf = conf;
        lp.dh = q.dh;
        lp.dw = q.dw;
        lp.st = st_p;
        lp.soft_gate = q.soft_gate;
    }
    UnetOut rout{};
    rout.points = points;
    rout.points_out = points_out;
    if (q.output_gate) {
        rout.gate_lidar = lidar;
        rout.gate_conf = conf;
        rout.gate_dh = q.dh;
        rout.gate_dw = q.dw;
        rout.gate_floor = q.output_gate_floor;  // floor + (1.0 - floor) * u with both constants rounded to fp32
        rout.gate_scale = (float)(1.0 - (double)q.output_gate_floor);
    }
    if (int e = enqueue_unet(u, points, nullptr, nullptr, q.use_prompt ? &lp : nullptr, enc_feat, enc_bias, rout, s))
        return e;
    if (q.anchor > 0.0f) {  // v3.py:570-573: re-fit on the refined depth, then the pull toward the LiDAR
        if (int e = prompt_fit(points_out, st_a)) return e;
        if (int e = launch_anchor(points_out, B, c.H, c.W, lidar, conf, q.dh, q.dw, st_a, q.anchor, s)) return e;
    }
    if (q.final_fit) {  // v3.py:768-778
        FinalFit f{};
        f.logz = points_out + 2;
        f.stride = 3;
        f.lidar = lidar;
        f.conf = conf;
        f.mask_binary = nullptr;
        f.B = B;
        f.H = c.H;
        f.W = c.W;
        f.dh = q.dh;
        f.dw = q.dw;
        f.iters = q.fit_iters;
        f.trim = q.fit_trim;
        f.min_points = q.fit_min_points;
        f.st = st_f;
        f.info = nullptr;
        f.workspace = u->fit_ws[1];
        f.workspace_bytes = u->fit_ws_bytes[1];
        if (int e = launch_final_fit(f, s)) return e;
        if (depth)  // MetricFit.metal:200-211 (v3.py:776)
            if (int e = pmg_post_depth(points_out + 2, 3, nullptr, B, c.H, c.W, st_f, depth, s)) return e;
    }
    return PMG_OK;
}

extern "C" {

pmg_unet* pmg_unet_create(const pmg_unet_config* cfg) {
    if (!cfg) {
        set_error("pmg_unet_create: null config");
        return nullptr;
    }
    const pmg_unet_config& c = *cfg;
    const int L = c.levels;
    std::string why;
    if (L < 2 || L > kMaxLevels) why = "levels must be in [2, 8] (sparse_unet.py:52)";
    else if (c.B < 1 || c.H < 1 || c.W < 1 || (int64_t)c.B * c.H * c.W > INT_MAX / 32)
        why = "bad point-map size";
    else if (c.precision != PMG_PREC_INT8 && c.precision != PMG_PREC_FP16) why = "precision must be int8 or fp16";
    else if (c.enc_channels < 16 || c.enc_channels % 16 != 0) why = "enc_channels must be a positive multiple of 16";
    else if (c.bottleneck_blocks < 0) why = "bottleneck_blocks must be >= 0";
    else {
        const int ds = 1 << (L - 1);
        if (c.H % ds != 0 || c.W % ds != 0)
            why = "H and W must be multiples of the encoder downsampling 2^(levels-1) (sparse_unet.py:187)";
        if (!col_width(c.channels[0], c.precision))
            why = c.precision == PMG_PREC_FP16 ? "fp16 level-0 width must be 16, 32, 48 or 64"
                                               : "level-0 width must be 16, 32, 48, 64 or 128";
        for (int k = 0; k < L && why.empty(); ++k) {
            if (!unet_width(c.channels[k], c.precision))
                why = c.precision == PMG_PREC_FP16 ? "fp16 level widths must be 16, 32, 48, 64, 96, 128, 192, 256 or 512"
                                                   : "level widths must be 16, 32, 48, 64, 96, 128, 192 or 256";
            if (c.enc_blocks[k] < 0 || c.enc_blocks[k] > 16) why = "enc_blocks must be in [0, 16]";
            if (k + 1 < L && (c.dec_blocks[k] < 0 || c.dec_blocks[k] > 16)) why = "dec_blocks must be in [0, 16]";
        }
        if (why.empty() && c.dec_blocks[L - 2] < 1)
            why = "the last up stage (level 0) needs a block: out_proj runs in its last convolution's epilogue";
    }
    if (!why.empty()) {
        set_error("pmg_unet_create: " + why);
        return nullptr;
    }
    pmg_unet* u = new pmg_unet();
    u->cfg = c;
    u->L = L;
    u->cap = (int64_t)c.B * c.H * c.W;
    u->Hk[0] = c.H;
    u->Wk[0] = c.W;
    for (int k = 1; k < L; ++k) {
        u->Hk[k] = (u->Hk[k - 1] + 1) / 2;
        u->Wk[k] = (u->Wk[k - 1] + 1) / 2;
    }
    int64_t maxcols = 1;
    for (int k = 0; k < L; ++k) {
        u->ncols[k] = (int64_t)c.B * u->Hk[k] * u->Wk[k];
        if (k > 0 && u->ncols[k] > maxcols) maxcols = u->ncols[k];
        if (c.channels[k] > u->Cmax) u->Cmax = c.channels[k];
    }
    u->R = u->Hk[L - 1];
    u->Cc = u->Wk[L - 1];
    u->T = (int64_t)c.B * u->R * u->Cc;
    const int CL = c.channels[L - 1];
    const int64_t cap = u->cap;
    size_t off = 0;
    std::vector<std::pair<void**, size_t>> plan;
    auto take = [&](void** p, size_t bytes) { plan.push_back({p, bytes}); };
    take((void**)&u->counts, sizeof(int64_t) * kMaxLevels);
    take((void**)&u->zq0, 4 * cap);
    take((void**)&u->zmin, 8 * c.B);
    take((void**)&u->coords0, 16 * cap);
    for (int k = 0; k < L; ++k) {
        if (k > 0) {
            take((void**)&u->coords[k], 16 * cap);
            take((void**)&u->off[k], 4 * (u->ncols[k] + 1));
            take((void**)&u->nmap_t[k], (size_t)27 * 4 * cap);
            take((void**)&u->tmask[k], 4 * (cap / 16 + 1));
        }
        if (k + 1 < L) {
            take((void**)&u->parent[k], 4 * cap);
            take((void**)&u->child[k], 16 * cap);
            take((void**)&u->xu[k], (size_t)4 * cap * c.channels[k]);
        }
        take((void**)&u->xd[k], (size_t)4 * cap * c.channels[k]);
    }
    take((void**)&u->xb, (size_t)4 * cap * CL);
    take((void**)&u->scan_excl, 4 * maxcols);
    take((void**)&u->scan_tiles, 4 * (maxcols / 256 + 2));
    const size_t elt = c.precision == PMG_PREC_FP16 ? 2 : 1;
    take((void**)&u->q1, elt * cap * u->Cmax);
    take((void**)&u->q2, elt * cap * u->Cmax);
    take((void**)&u->codes, elt * cap * (2 * CL > u->Cmax ? 2 * CL : u->Cmax));
    take((void**)&u->codes2, elt * cap * CL);
    take((void**)&u->lin, (size_t)4 * cap * u->Cmax);
    take((void**)&u->enc_codes, elt * u->T * c.enc_channels);
    take((void**)&u->enc_tok, (size_t)4 * u->T * CL);
    if (L > 1 && c.precision != PMG_PREC_FP16) u->part_bytes = conv_split_bytes(c.channels[L - 1]);
    if (u->part_bytes > 0) take((void**)&u->part, (size_t)u->part_bytes);
    for (auto& p : plan) off += ualign(p.second);
    u->arena_bytes = off;
    if (hipMalloc(&u->arena, u->arena_bytes) != hipSuccess) {
        set_error("pmg_unet_create: hipMalloc of " + std::to_string(u->arena_bytes) + " bytes failed");
        delete u;
        return nullptr;
    }
    if (hipMemset(u->arena, 0, u->arena_bytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        set_error("pmg_unet_create: clearing the workspace failed");
        (void)hipFree(u->arena);
        delete u;
        return nullptr;
    }
    uint8_t* a = (uint8_t*)u->arena;
    off = 0;
    for (auto& p : plan) {
        *p.first = a + off;
        off += ualign(p.second);
    }
    // level 0 holds cap voxels: its count is known, every other is written by the structure kernels
    if (hipMemcpy(u->counts, &u->cap, sizeof(int64_t), hipMemcpyHostToDevice) != hipSuccess) {
        set_error("pmg_unet_create: initialising the level counts failed");
        (void)hipFree(u->arena);
        delete u;
        return nullptr;
    }
    bool ok = hipStreamCreateWithFlags(&u->side, hipStreamNonBlocking) == hipSuccess &&
              hipEventCreateWithFlags(&u->ev_fork, hipEventDisableTiming) == hipSuccess &&
              hipEventCreateWithFlags(&u->ev_enc, hipEventDisableTiming) == hipSuccess;
    for (int k = 1; k < L && ok; ++k) ok = hipEventCreateWithFlags(&u->ev_level[k], hipEventDisableTiming) == hipSuccess;
    if (!ok) {
        set_error("pmg_unet_create: creating the structure stream or its events failed");
        pmg_unet_destroy(u);
        return nullptr;
    }
    return u;
}

void pmg_unet_destroy(pmg_unet* u) {
    if (!u) return;
    u->graphs.clear();
    if (u->side) (void)hipStreamSynchronize(u->side);
    for (int k = 0; k < kMaxLevels; ++k)
        if (u->ev_level[k]) (void)hipEventDestroy(u->ev_level[k]);
    if (u->ev_fork) (void)hipEventDestroy(u->ev_fork);
    if (u->ev_enc) (void)hipEventDestroy(u->ev_enc);
    if (u->side) (void)hipStreamDestroy(u->side);
    if (u->step_arena) (void)hipFree(u->step_arena);
    if (u->arena) (void)hipFree(u->arena);
    delete u;
}

size_t pmg_unet_workspace_bytes(const pmg_unet* u) { return u ? u->arena_bytes : 0; }

int pmg_unet_set_weights(pmg_unet* u, const pmg_unet_weights* w) {
    PMG_REQUIRE(u && w, "null argument");
    const pmg_unet_config& c = u->cfg;
    const int L = u->L;
    int nb = 0;
    for (int k = 0; k < L; ++k) nb += c.enc_blocks[k];
    nb += c.bottleneck_blocks;
    for (int k = 0; k + 1 < L; ++k) nb += c.dec_blocks[k];
    PMG_REQUIRE(w->n_blocks == nb && w->blocks, "block count mismatch: expected " + std::to_string(nb));
    PMG_REQUIRE(w->n_linears == 2 * (L - 1) + 3 && w->linears, "linear count mismatch: expected " +
                                                                 std::to_string(2 * (L - 1) + 3));
    PMG_REQUIRE(w->in_w && w->in_b && w->out_w && w->out_b, "missing projection weights");
    PMG_REQUIRE((w->pr_w == nullptr) == (w->pr_b == nullptr), "prompt_proj needs weight and bias");
    const bool i8 = c.precision == PMG_PREC_INT8;
    for (int i = 0; i < nb; ++i) {
        const pmg_block_weights& b = w->blocks[i];
        PMG_REQUIRE(b.ln_gamma && b.ln_beta && b.w1 && b.b1 && b.w2 && b.b2 && (!i8 || (b.w1_scale && b.w2_scale)),
                    "missing block weights");
        PMG_REQUIRE(aligned16(b.w1) && aligned16(b.w2), "conv weights must be 16-byte aligned");
        PMG_REQUIRE(!i8 || (b.a1_scale > 0.0f && b.a2_scale > 0.0f && b.q1_mult > 0.0f && b.q2_mult > 0.0f),
                    "int8 blocks need positive activation scales");
    }
    for (int i = 0; i < w->n_linears; ++i) {
        const pmg_linear_weights& l = w->linears[i];
        PMG_REQUIRE(l.w && (!i8 || l.w_scale) && l.bias && aligned16(l.w), "missing or misaligned linear weights");
        PMG_REQUIRE(!i8 || (l.a_scale > 0.0f && l.q_mult > 0.0f), "linears need positive activation scales");
    }
    u->in_w = w->in_w;
    u->in_b = w->in_b;
    u->pr_w = w->pr_w;
    u->pr_b = w->pr_b;
    u->out_w = w->out_w;
    u->out_b = w->out_b;
    int q = 0;
    for (int k = 0; k < L; ++k) u->down[k].assign(w->blocks + q, w->blocks + q + c.enc_blocks[k]), q += c.enc_blocks[k];
    u->bott.assign(w->blocks + q, w->blocks + q + c.bottleneck_blocks);
    q += c.bottleneck_blocks;
    for (int i = 0; i + 1 < L; ++i) u->dec[i].assign(w->blocks + q, w->blocks + q + c.dec_blocks[i]), q += c.dec_blocks[i];
    u->pool.assign(w->linears, w->linears + (L - 1));
    u->enc = w->linears[L - 1];
    u->fuse0 = w->linears[L];
    u->fuse2 = w->linears[L + 1];
    u->up.assign(w->linears + L + 2, w->linears + 2 * L + 1);
    u->have_weights = true;
    u->graphs.clear();
    return PMG_OK;
}

int pmg_unet_forward(pmg_unet* u, const float* feats, const int32_t* coords, const float* prompt_feats,
                     const float* encoder_feature, const float* encoder_bias_map, float* out, void* stream) {
    PMG_REQUIRE(u && u->have_weights, "weights not set");
    PMG_REQUIRE(feats && encoder_feature && out, "null buffer");
    PMG_REQUIRE(!prompt_feats || u->pr_w, "prompt_feats given but the refiner has no prompt_proj");
    PMG_REQUIRE(!coords || aligned16(coords), "coords must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    const void* const key[kGraphKey] = {(const void*)3, feats, coords, prompt_feats, encoder_feature, encoder_bias_map,
                                        out, stream};
    UnetOut rout{};
    rout.delta = out;
    return u->graphs.run(key, s, u->cfg.use_graph != 0, [&] {
        return enqueue_unet(u, feats, coords, prompt_feats, nullptr, encoder_feature, encoder_bias_map, rout, s);
    });
}

int pmg_unet_step_prepare(pmg_unet* u, const pmg_unet_step_config* sc) {
    PMG_REQUIRE(u && sc, "null argument");
    const pmg_unet_step_config& q = *sc;
    const pmg_unet_config& c = u->cfg;
    PMG_REQUIRE(q.dh >= 1 && q.dw >= 1, "bad LiDAR size");
    PMG_REQUIRE(q.fit_iters >= 0 && q.fit_iters <= 64 && q.fit_min_points >= 1 && q.fit_trim >= 0.0f &&
                    q.fit_trim < 1.0f,
                "bad fit parameters");
    PMG_REQUIRE(q.output_gate_floor >= 0.0f && q.output_gate_floor <= 1.0f, "output_gate_floor must be in [0, 1]");
    PMG_REQUIRE(q.anchor >= 0.0f && q.anchor <= 1.0f, "anchor must be in [0, 1]");
    PMG_REQUIRE(!(q.use_prompt || q.anchor > 0.0f) || (int64_t)c.H * c.W <= kFitMaxElements,
                "H*W exceeds the metric fit's 2^21 elements (use_prompt / anchor)");
    PMG_REQUIRE(!q.final_fit || (int64_t)q.dh * q.dw <= kFitMaxElements,
                "dh*dw exceeds the metric fit's 2^21 elements (final_fit)");
    u->graphs.clear();  // (synchronises) captured steps use the old workspace
    if (u->step_arena) {
        (void)hipFree(u->step_arena);
        u->step_arena = nullptr;
    }
    u->step_ready = false;
    u->fit_ws_bytes[0] = ualign(fit_workspace_bytes((int64_t)c.H * c.W, q.fit_iters));
    u->fit_ws_bytes[1] = q.final_fit ? ualign(final_fit_workspace_bytes(c.B, q.dh, q.dw, q.fit_iters)) : 256;
    const size_t st_bytes = ualign(6 * sizeof(float) * (size_t)c.B);
    const size_t bytes = u->fit_ws_bytes[0] + u->fit_ws_bytes[1] + st_bytes;
    if (hipMalloc(&u->step_arena, bytes) != hipSuccess) {
        u->step_arena = nullptr;
        return fail(PMG_E_HIP, "pmg_unet_step_prepare: hipMalloc of " + std::to_string(bytes) + " bytes failed");
    }
    PMG_CHECK_HIP(hipMemset(u->step_arena, 0, bytes));  // the fits' workspaces start zero-filled
    PMG_CHECK_HIP(hipDeviceSynchronize());
    uint8_t* a = (uint8_t*)u->step_arena;
    u->fit_ws[0] = a;
    u->fit_ws[1] = a + u->fit_ws_bytes[0];
    u->st_scratch = (float*)(a + u->fit_ws_bytes[0] + u->fit_ws_bytes[1]);
    u->scfg = q;
    u->step_ready = true;
    return PMG_OK;
}

int pmg_unet_step(pmg_unet* u, const float* points, float* points_out, const float* lidar, const float* conf,
                  const float* encoder_feature, const float* encoder_bias_map, float* st_prompt, float* st_final,
                  float* depth, void* stream) {
    PMG_REQUIRE(u && u->have_weights, "weights not set");
    PMG_REQUIRE(u->step_ready, "pmg_unet_step_prepare has not run");
    PMG_REQUIRE(points && points_out && lidar && conf && encoder_feature, "null buffer");
    PMG_REQUIRE(!u->scfg.use_prompt || u->pr_w, "use_prompt needs prompt_proj weights");
    PMG_REQUIRE(!depth || u->scfg.final_fit, "post_depth (depth) needs final_fit");
    hipStream_t s = (hipStream_t)stream;
    const void* const key[kGraphKey] = {(const void*)4, points, points_out, lidar, conf, encoder_feature,
                                        encoder_bias_map, st_prompt, st_final, depth, stream};
    return u->graphs.run(key, s, u->cfg.use_graph != 0, [&] {
        return enqueue_unet_step(u, points, points_out, lidar, conf, encoder_feature, encoder_bias_map, st_prompt,
                                 st_final, depth, s);
    });
}

int pmg_unet_check(pmg_unet* u, void* stream) {
    PMG_REQUIRE(u, "null context");
    PMG_CHECK_HIP(hipStreamSynchronize((hipStream_t)stream));
    if (!u->step_ready) return PMG_OK;
    unsigned seen[2] = {0, 0};
    const bool has[2] = {u->fit_ws_bytes[0] > kFitErrSeenOffset, u->fit_ws_bytes[1] > kFitErrSeenOffset};
    for (int k = 0; k < 2; ++k)
        if (has[k])
            PMG_CHECK_HIP(hipMemcpy(&seen[k], (uint8_t*)u->fit_ws[k] + kFitErrSeenOffset, sizeof(unsigned),
                                    hipMemcpyDeviceToHost));
    if (seen[0] || seen[1]) {
        for (int k = 0; k < 2; ++k)
            if (has[k]) PMG_CHECK_HIP(hipMemset((uint8_t*)u->fit_ws[k] + kFitErrSeenOffset, 0, sizeof(unsigned)));
        PMG_CHECK_HIP(hipDeviceSynchronize());
        return fail(PMG_E_DEVICE, "pmg_unet_check: a device-wide wait in the metric fit expired (" +
                                      std::to_string(seen[0] + seen[1]) + " launches)");
    }
    return PMG_OK;
}

const void* pmg_unet_buffer(pmg_unet* u, int id, int level) {
    if (!u || level < 0 || level >= u->L) return nullptr;
    switch (id) {
        case PMG_UNET_COUNTS: return u->counts;
        case PMG_UNET_COORDS: return u->coords[level];
        case PMG_UNET_PARENT: return level + 1 < u->L ? u->parent[level] : nullptr;
        case PMG_UNET_NMAP: return level > 0 ? u->nmap_t[level] : nullptr;
        case PMG_UNET_TILE_MASK: return level > 0 ? u->tmask[level] : nullptr;
        case PMG_UNET_DOWN: return u->xd[level];
        case PMG_UNET_UP: return level + 1 < u->L ? u->xu[level] : u->xb;
        case PMG_UNET_ENC_TOKENS: return u->enc_tok;
        case PMG_UNET_COL_OFFSETS: return level > 0 ? u->off[level] : nullptr;
        case PMG_UNET_STEP_ST: return u->step_ready ? u->st_scratch : nullptr;
        default: return nullptr;
    }
}

int64_t pmg_unet_capacity(const pmg_unet* u) { return u ? u->cap : 0; }

}  // extern "C"
