// Voxelisation and submanifold neighbour maps.
//
// Level 0 of the refiner has exactly one voxel per pixel (MoGeModel._voxelize, moge/model/v3.py:305-344), so its
// 27-neighbour map is a 3x3 image stencil plus a depth predicate (_core.py:269-295): one thread per voxel reads
// nine z values and writes its 27 map entries, coalesced across the wave in the tap-major layout the
// convolutions read. Generic coordinates (the 1M-voxel microbench, levels >= 1) go through an open-addressing
// hash over the reference's linearised keys (_core.py:89-94) with 64-bit compare-and-swap insertion.
//
// Every map kernel also emits the per-16-row tile tap mask the convolutions branch on: bit v set iff any row of
// the tile has tap v. It is reduced across each 16-lane group with shuffles and stored by the group's first lane,
// so no atomics and no separate pass are needed.
#include <climits>

#include "pmg_common.h"

namespace pmg {

// ------------------------------------------------------------------------------------------------------------
// Voxelisation: zq = rint(logz * res), per-batch min/max.  v3.py:332-335.
__global__ __launch_bounds__(256) void voxelize_k(const float* __restrict__ logz, int64_t stride, int HW,
                                                  float res, int32_t* __restrict__ zq, int32_t* zmin,
                                                  int32_t* zmax) {
    const int b = blockIdx.y;
    const int p = blockIdx.x * 256 + threadIdx.x;
    int mn = INT_MAX, mx = INT_MIN;
    if (p < HW) {
        const int64_t o = (int64_t)b * HW + p;
        const float v = logz[o * stride] * res;
        const int q = (int)rne(v);
        zq[o] = q;
        mn = q;
        mx = q;
    }
    mn = wave_min_i32(mn);
    mx = wave_max_i32(mx);
    __shared__ int smn[4], smx[4];
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        smn[w] = mn;
        smx[w] = mx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; ++k) {
            mn = smn[k] < mn ? smn[k] : mn;
            mx = smx[k] > mx ? smx[k] : mx;
        }
        atomicMin(&zmin[b], mn);
        atomicMax(&zmax[b], mx);
    }
}

// OR of a 27-bit row mask over the 16 rows of a tile; the tile's first lane stores it.
__device__ inline void store_tile_mask(uint32_t rmask, int64_t o, int64_t M, uint32_t* tile_mask) {
    if (!tile_mask) return;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) rmask |= __shfl_xor(rmask, off, 16);
    if ((o & 15) == 0 && o < M) tile_mask[o >> 4] = rmask;
}

// ------------------------------------------------------------------------------------------------------------
// Column stencil map. _core.py:269-295; tap order _core.py:65-82.
__global__ __launch_bounds__(256) void nmap_column_k(const int32_t* __restrict__ zq, const int32_t* __restrict__ zmin,
                                                     int H, int W, int64_t M, int32_t* __restrict__ nmap_t,
                                                     int32_t* __restrict__ nmap_rows, uint32_t* tile_mask,
                                                     int32_t* __restrict__ coords) {
    const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
    uint32_t rmask = 0;
    if (o < M) {
        const int64_t HW = (int64_t)H * W;
        const int b = (int)(o / HW);
        const int p = (int)(o - (int64_t)b * HW);
        const int i = p / W;
        const int j = p - i * W;
        const int64_t zc = zq[o];
#pragma unroll
        for (int di = -1; di <= 1; ++di) {
#pragma unroll
            for (int dj = -1; dj <= 1; ++dj) {
                const int v0 = (di + 1) * 9 + (dj + 1) * 3;
                int h0 = -1, h1 = -1, h2 = -1;
                const int ni = i + di, nj = j + dj;
                if (ni >= 0 && ni < H && nj >= 0 && nj < W) {
                    const int64_t nn = o + (int64_t)di * W + dj;
                    const int64_t dz = (int64_t)zq[nn] - zc;
                    if (dz == -1) h0 = (int)nn;
                    if (dz == 0) h1 = (int)nn;
                    if (dz == 1) h2 = (int)nn;
                }
                if (nmap_t) {
                    nmap_t[(int64_t)(v0 + 0) * M + o] = h0;
                    nmap_t[(int64_t)(v0 + 1) * M + o] = h1;
                    nmap_t[(int64_t)(v0 + 2) * M + o] = h2;
                }
                if (nmap_rows) {
                    nmap_rows[o * 27 + v0 + 0] = h0;
                    nmap_rows[o * 27 + v0 + 1] = h1;
                    nmap_rows[o * 27 + v0 + 2] = h2;
                }
                rmask |= (h0 >= 0 ? 1u : 0u) << v0;
                rmask |= (h1 >= 0 ? 1u : 0u) << (v0 + 1);
                rmask |= (h2 >= 0 ? 1u : 0u) << (v0 + 2);
            }
        }
        if (coords) {
            int4 c;
            c.x = b;
            c.y = i;
            c.z = j;
            c.w = (int)(zc - zmin[b]);
            reinterpret_cast<int4*>(coords)[o] = c;
        }
    }
    store_tile_mask(rmask, o, M, tile_mask);
}

// ------------------------------------------------------------------------------------------------------------
// Open-addressing hash over linearised keys. Keys are 64-bit, EMPTY = all ones (a linearised in-bounds key is
// never negative). Linear probing; the table has at least 4x as many slots as keys. Duplicate coordinates keep
// the smallest row index (atomicMin), which makes the map independent of insertion order.
constexpr uint64_t kEmpty = ~0ull;

__device__ inline uint64_t mix64(uint64_t k) {
    k ^= k >> 33;
    k *= 0xff51afd7ed558ccdull;
    k ^= k >> 33;
    k *= 0xc4ceb9fe1a85ec53ull;
    k ^= k >> 33;
    return k;
}

struct Shape4 {
    int64_t s0, s1, s2, s3;
};

// _linearise (_core.py:89-94): ((b*S1 + x)*S2 + y)*S3 + z.
__device__ inline int64_t linearise(int b, int x, int y, int z, const Shape4& S) {
    return (((int64_t)b * S.s1 + x) * S.s2 + y) * S.s3 + z;
}

__global__ __launch_bounds__(256) void hash_clear_k(uint64_t* keys, int32_t* vals, int64_t cap) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < cap) {
        keys[i] = kEmpty;
        vals[i] = INT_MAX;
    }
}

__global__ __launch_bounds__(256) void hash_insert_k(const int4* __restrict__ coords, int64_t M, Shape4 S,
                                                     uint64_t* keys, int32_t* vals, uint64_t cap_mask) {
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (m >= M) return;
    const int4 c = coords[m];
    const uint64_t key = (uint64_t)linearise(c.x, c.y, c.z, c.w, S);
    uint64_t slot = mix64(key) & cap_mask;
    for (uint64_t probe = 0; probe <= cap_mask; ++probe) {
        const uint64_t prev = atomicCAS((unsigned long long*)&keys[slot], (unsigned long long)kEmpty,
                                        (unsigned long long)key);
        if (prev == kEmpty || prev == key) {
            atomicMin(&vals[slot], (int)m);
            return;
        }
        slot = (slot + 1) & cap_mask;
    }
}

__device__ inline int hash_lookup(const uint64_t* __restrict__ keys, const int32_t* __restrict__ vals,
                                  uint64_t cap_mask, uint64_t key) {
    uint64_t slot = mix64(key) & cap_mask;
    for (uint64_t probe = 0; probe <= cap_mask; ++probe) {
        const uint64_t k = keys[slot];
        if (k == key) return vals[slot];
        if (k == kEmpty) return -1;
        slot = (slot + 1) & cap_mask;
    }
    return -1;
}

// _SortedIndex.lookup (_core.py:114-124): out-of-bounds queries never hit.
__global__ __launch_bounds__(256) void hash_query_k(const int4* __restrict__ coords, int64_t M, Shape4 S,
                                                    const uint64_t* __restrict__ keys,
                                                    const int32_t* __restrict__ vals, uint64_t cap_mask,
                                                    int32_t* __restrict__ nmap_t, int32_t* __restrict__ nmap_rows,
                                                    uint32_t* tile_mask) {
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    uint32_t rmask = 0;
    if (m < M) {
        const int4 c = coords[m];
        const bool bok = c.x >= 0 && c.x < S.s0;
        for (int v = 0; v < 27; ++v) {
            const int dx = v / 9 - 1, dy = (v / 3) % 3 - 1, dz = v % 3 - 1;
            const int x = c.y + dx, y = c.z + dy, z = c.w + dz;
            int hit = -1;
            if (bok && x >= 0 && x < S.s1 && y >= 0 && y < S.s2 && z >= 0 && z < S.s3)
                hit = hash_lookup(keys, vals, cap_mask, (uint64_t)linearise(c.x, x, y, z, S));
            if (nmap_t) nmap_t[(int64_t)v * M + m] = hit;
            if (nmap_rows) nmap_rows[m * 27 + v] = hit;
            rmask |= (hit >= 0 ? 1u : 0u) << v;
        }
    }
    store_tile_mask(rmask, m, M, tile_mask);
}

// ------------------------------------------------------------------------------------------------------------
// Row-major (M, 27) -> tap-major [27][M] plus tile masks.
__global__ __launch_bounds__(256) void nmap_from_rows_k(const int32_t* __restrict__ rows, int64_t M,
                                                        int32_t* __restrict__ nmap_t, uint32_t* tile_mask) {
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    uint32_t rmask = 0;
    if (m < M) {
        for (int v = 0; v < 27; ++v) {
            const int h = rows[m * 27 + v];
            if (nmap_t) nmap_t[(int64_t)v * M + m] = h;
            rmask |= (h >= 0 ? 1u : 0u) << v;
        }
    }
    store_tile_mask(rmask, m, M, tile_mask);
}

// ------------------------------------------------------------------------------------------------------------
// Compacted kernel maps: per tap, ascending output rows with a neighbour (the reference's nonzero()).
// Pass 1: per 256-row block and tap, the number of valid rows (wave ballots).
__global__ __launch_bounds__(256) void kmap_count_k(const int32_t* __restrict__ nmap_t, int64_t M, int nblk,
                                                    int32_t* __restrict__ counts) {
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    __shared__ int part[27][4];
    const int w = threadIdx.x >> 6;
    for (int v = 0; v < 27; ++v) {
        const bool ok = m < M && nmap_t[(int64_t)v * M + m] >= 0;
        const uint64_t bal = __ballot(ok);
        if ((threadIdx.x & 63) == 0) part[v][w] = __popcll(bal);
    }
    __syncthreads();
    if (threadIdx.x < 27) {
        const int v = threadIdx.x;
        counts[(int64_t)v * nblk + blockIdx.x] = part[v][0] + part[v][1] + part[v][2] + part[v][3];
    }
}

// Pass 2: one block per tap, exclusive scan of its nblk block counts in place; totals[v] = the tap's count.
__global__ __launch_bounds__(1024) void kmap_scan_k(int32_t* counts, int nblk, int64_t* totals) {
    const int v = blockIdx.x;
    int32_t* c = counts + (int64_t)v * nblk;
    const int per = (nblk + 1023) / 1024;
    const int lo = threadIdx.x * per;
    const int hi = min(lo + per, nblk);
    int64_t s = 0;
    for (int i = lo; i < hi; ++i) s += c[i];
    __shared__ int64_t sc[1024];
    sc[threadIdx.x] = s;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
        const int64_t add = threadIdx.x >= off ? sc[threadIdx.x - off] : 0;
        __syncthreads();
        sc[threadIdx.x] += add;
        __syncthreads();
    }
    int64_t run = sc[threadIdx.x] - s;  // exclusive
    for (int i = lo; i < hi; ++i) {
        const int32_t t = c[i];
        c[i] = (int32_t)run;
        run += t;
    }
    if (threadIdx.x == 1023) totals[v] = sc[1023];
}

// Pass 3: offsets[0..27] = exclusive scan of the totals.
__global__ void kmap_offsets_k(const int64_t* totals, int64_t* offsets) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    int64_t run = 0;
    for (int v = 0; v < 27; ++v) {
        offsets[v] = run;
        run += totals[v];
    }
    offsets[27] = run;
}

// Pass 4: each valid (row, tap) writes its pair at offsets[v] + block offset + wave prefix + lane prefix.
__global__ __launch_bounds__(256) void kmap_write_k(const int32_t* __restrict__ nmap_t, int64_t M, int nblk,
                                                    const int32_t* __restrict__ counts,
                                                    const int64_t* __restrict__ offsets, int32_t* out_rows,
                                                    int32_t* in_rows, int64_t capacity) {
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    __shared__ int wcnt[27][4];
    const int w = threadIdx.x >> 6;
    int hv[27];
    uint64_t bal[27];
    for (int v = 0; v < 27; ++v) {
        hv[v] = m < M ? nmap_t[(int64_t)v * M + m] : -1;
        bal[v] = __ballot(hv[v] >= 0);
        if ((threadIdx.x & 63) == 0) wcnt[v][w] = __popcll(bal[v]);
    }
    __syncthreads();
    for (int v = 0; v < 27; ++v) {
        if (hv[v] < 0) continue;
        int before = 0;
        for (int k = 0; k < w; ++k) before += wcnt[v][k];
        const unsigned below = __builtin_amdgcn_mbcnt_hi((unsigned)(bal[v] >> 32),
                                                         __builtin_amdgcn_mbcnt_lo((unsigned)bal[v], 0u));
        const int64_t pos = offsets[v] + counts[(int64_t)v * nblk + blockIdx.x] + before + below;
        if (pos < capacity) {
            out_rows[pos] = (int32_t)m;
            in_rows[pos] = hv[v];
        }
    }
}

}  // namespace pmg

using namespace pmg;

extern "C" {

int pmg_voxelize(const float* logz, int64_t stride, int B, int H, int W, float resolution, int32_t* zq,
                 int32_t* zmin, int32_t* zmax, void* stream) {
    PMG_REQUIRE(logz && zq && zmin && zmax, "null buffer");
    PMG_REQUIRE(B > 0 && H > 0 && W > 0 && stride >= 1, "bad shape");
    PMG_REQUIRE((int64_t)H * W <= INT_MAX && (int64_t)B * H * W <= INT_MAX, "map too large");
    PMG_REQUIRE(B <= 65535, "batch too large");
    hipStream_t s = (hipStream_t)stream;
    fill_u32(zmin, 0x7fffffffu, B, s);
    fill_u32(zmax, 0x80000000u, B, s);
    const int HW = H * W;
    dim3 grid((HW + 255) / 256, B);
    hipLaunchKernelGGL(voxelize_k, grid, dim3(256), 0, s, logz, stride, HW, resolution, zq, zmin, zmax);
    return check_launch("voxelize_k");
}

int pmg_nmap_column(const int32_t* zq, const int32_t* zmin, int B, int H, int W, int32_t* nmap_t,
                    int32_t* nmap_rows, uint32_t* tile_mask, int32_t* coords, void* stream) {
    PMG_REQUIRE(zq, "null zq");
    PMG_REQUIRE(!coords || zmin, "coords need zmin");
    PMG_REQUIRE(B > 0 && H > 0 && W > 0, "bad shape");
    const int64_t M = (int64_t)B * H * W;
    PMG_REQUIRE(M <= INT_MAX, "too many voxels for int32 indices");
    PMG_REQUIRE(!coords || aligned16(coords), "coords must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(nmap_column_k, dim3((unsigned)((M + 255) / 256)), dim3(256), 0, s, zq, zmin, H, W, M,
                       nmap_t, nmap_rows, tile_mask, coords);
    return check_launch("nmap_column_k");
}

static int64_t hash_capacity(int64_t M) {
    int64_t cap = 1024;
    while (cap < 4 * M) cap <<= 1;
    return cap;
}

size_t pmg_hash_workspace_bytes(int64_t M) {
    if (M < 0) return 0;
    const int64_t cap = hash_capacity(M);
    return (size_t)cap * (sizeof(uint64_t) + sizeof(int32_t)) + 256;
}

int pmg_nmap_hash(const int32_t* coords, int64_t M, const int64_t* shape, int32_t* nmap_t, int32_t* nmap_rows,
                  uint32_t* tile_mask, void* workspace, size_t workspace_bytes, void* stream) {
    PMG_REQUIRE(coords && shape, "null argument");
    PMG_REQUIRE(M >= 0 && M <= INT_MAX, "bad voxel count");
    PMG_REQUIRE(aligned16(coords), "coords must be 16-byte aligned");
    for (int d = 0; d < 4; ++d) PMG_REQUIRE(shape[d] > 0 && shape[d] <= INT_MAX, "bad sparse shape");
    // The linearised key must fit in 63 bits so that no key equals the EMPTY marker.
    const double span = (double)shape[0] * (double)shape[1] * (double)shape[2] * (double)shape[3];
    PMG_REQUIRE(span < 9.0e18, "sparse shape too large for 64-bit keys");
    PMG_REQUIRE(workspace && workspace_bytes >= pmg_hash_workspace_bytes(M), "workspace too small");
    if (M == 0) return PMG_OK;
    hipStream_t s = (hipStream_t)stream;
    const int64_t cap = hash_capacity(M);
    uint64_t* keys = (uint64_t*)workspace;
    int32_t* vals = (int32_t*)(keys + cap);
    Shape4 S{shape[0], shape[1], shape[2], shape[3]};
    hipLaunchKernelGGL(hash_clear_k, dim3((unsigned)((cap + 255) / 256)), dim3(256), 0, s, keys, vals, cap);
    if (int e = check_launch("hash_clear_k")) return e;
    const dim3 g((unsigned)((M + 255) / 256));
    hipLaunchKernelGGL(hash_insert_k, g, dim3(256), 0, s, (const int4*)coords, M, S, keys, vals,
                       (uint64_t)(cap - 1));
    if (int e = check_launch("hash_insert_k")) return e;
    hipLaunchKernelGGL(hash_query_k, g, dim3(256), 0, s, (const int4*)coords, M, S, (const uint64_t*)keys,
                       (const int32_t*)vals, (uint64_t)(cap - 1), nmap_t, nmap_rows, tile_mask);
    return check_launch("hash_query_k");
}

int pmg_nmap_from_rows(const int32_t* nmap_rows, int64_t M, int32_t* nmap_t, uint32_t* tile_mask, void* stream) {
    PMG_REQUIRE(nmap_rows, "null map");
    PMG_REQUIRE(M >= 0 && M <= INT_MAX, "bad voxel count");
    if (M == 0) return PMG_OK;
    hipLaunchKernelGGL(nmap_from_rows_k, dim3((unsigned)((M + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       nmap_rows, M, nmap_t, tile_mask);
    return check_launch("nmap_from_rows_k");
}

size_t pmg_kmap_workspace_bytes(int64_t M) {
    const int64_t nblk = (M + 255) / 256;
    return (size_t)(27 * nblk) * sizeof(int32_t) + 32 * sizeof(int64_t) + 256;
}

int pmg_kmap_compact(const int32_t* nmap_t, int64_t M, int64_t* offsets, int32_t* out_rows, int32_t* in_rows,
                     int64_t capacity, void* workspace, size_t workspace_bytes, void* stream) {
    PMG_REQUIRE(nmap_t && offsets, "null argument");
    PMG_REQUIRE(M >= 0 && M <= INT_MAX, "bad voxel count");
    PMG_REQUIRE(capacity >= 0 && (capacity == 0 || (out_rows && in_rows)), "bad output");
    PMG_REQUIRE(workspace && workspace_bytes >= pmg_kmap_workspace_bytes(M), "workspace too small");
    hipStream_t s = (hipStream_t)stream;
    if (M == 0) {
        fill_u32(offsets, 0u, 2 * 28, s);
        return check_launch("fill");
    }
    const int nblk = (int)((M + 255) / 256);
    int64_t* totals = (int64_t*)workspace;
    int32_t* counts = (int32_t*)(totals + 32);
    hipLaunchKernelGGL(kmap_count_k, dim3(nblk), dim3(256), 0, s, nmap_t, M, nblk, counts);
    if (int e = check_launch("kmap_count_k")) return e;
    hipLaunchKernelGGL(kmap_scan_k, dim3(27), dim3(1024), 0, s, counts, nblk, totals);
    if (int e = check_launch("kmap_scan_k")) return e;
    hipLaunchKernelGGL(kmap_offsets_k, dim3(1), dim3(64), 0, s, (const int64_t*)totals, offsets);
    if (int e = check_launch("kmap_offsets_k")) return e;
    hipLaunchKernelGGL(kmap_write_k, dim3(nblk), dim3(256), 0, s, nmap_t, M, nblk, (const int32_t*)counts,
                       (const int64_t*)offsets, out_rows, in_rows, capacity);
    if (int e = check_launch("kmap_write_k")) return e;
    int64_t total = 0;
    PMG_CHECK_HIP(hipMemcpyAsync(&total, offsets + 27, sizeof(int64_t), hipMemcpyDeviceToHost, s));
    PMG_CHECK_HIP(hipStreamSynchronize(s));
    if (total > capacity)
        return fail(PMG_E_OVERFLOW, "pmg_kmap_compact: " + std::to_string(total) + " pairs exceed capacity " +
                                        std::to_string(capacity));
    return PMG_OK;
}

}  // extern "C"
