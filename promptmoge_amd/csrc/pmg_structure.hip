// Voxelisation and submanifold neighbour maps.
//
// Level 0 of the refiner has exactly one voxel per pixel (MoGeModel._voxelize, moge/model/v3.py:305-344), so its
// 27-neighbour map is a 3x3 image stencil plus a depth predicate (_core.py:269-295): one thread per voxel reads
// nine z values and writes its 27 map entries, coalesced across the wave in the tap-major layout the
// convolutions read. Generic coordinates (the 1M-voxel microbench, levels >= 1) go through an open-addressing
// hash of 4x4x4 bricks keyed by the reference's linearisation (_core.py:89-94) on the brick grid.
//
// Every map kernel also emits the per-16-row tile tap mask the convolutions branch on: bit v set iff any row of
// the tile has tap v. It is reduced across each 16-lane group with shuffles and stored by the group's first lane,
// so no atomics and no separate pass are needed.
#include <climits>

#include "pmg_common.h"

namespace pmg {

// ------------------------------------------------------------------------------------------------------------
// Voxelisation: zq = rint(logz * res), per-batch min/max.  v3.py:332-335. Grid-stride over a capped grid
// (kVoxBlocks per batch item), so that few blocks meet at the per-batch min/max atomics: one block per 256 pixels
// serialised 2400 same-address atomics at 480 x 640 (30 us).
constexpr int kVoxBlocks = 64;
// The per-batch-item key range before voxelize_k's atomics: zmin = INT_MAX, zmax = INT_MIN (one launch for both).
__global__ __launch_bounds__(256) void minmax_init_k(int32_t* zmin, int32_t* zmax, int B) {
    const int b = blockIdx.x * 256 + threadIdx.x;
    if (b < B) {
        zmin[b] = INT_MAX;
        zmax[b] = INT_MIN;
    }
}
__global__ __launch_bounds__(256) void voxelize_k(const float* __restrict__ logz, int64_t stride, int HW,
                                                  float res, int32_t* __restrict__ zq, int32_t* zmin,
                                                  int32_t* zmax) {
    const int b = blockIdx.y;
    int mn = INT_MAX, mx = INT_MIN;
#pragma unroll 4
    for (int p = blockIdx.x * 256 + threadIdx.x; p < HW; p += gridDim.x * 256) {
        const int64_t o = (int64_t)b * HW + p;
        const float v = logz[o * stride] * res;
        const int q = (int)rne(v);
        zq[o] = q;
        mn = q < mn ? q : mn;
        mx = q > mx ? q : mx;
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
// Generic coordinates: an open-addressing hash of 4x4x4 bricks. A bucket is one brick of the sparse grid: a
// key and 64 row indices, one per cell. The 27 neighbours of a voxel
// fall in at most 2x2x2 bricks (one per axis unless the voxel sits on a brick face), so a query resolves <= 8
// buckets with independent loads and then reads its 27 cells from them; neighbouring voxels share those buckets,
// which keeps the query's traffic in L1/L2 instead of one random 128-byte line per tap. Keys are the linearised
// brick coordinates (the reference's _linearise, _core.py:89-94, on the brick grid); EMPTY = all ones. Cells
// hold -1 until a voxel writes its row index. Coordinates must be unique, as in a sparse tensor; for a duplicated
// coordinate the map names one of its rows.
constexpr uint64_t kEmpty = ~0ull;
constexpr int kBrickLog = 2;  // 4 cells per axis

// Home bucket of a brick key: the key folded to 32 bits, Fibonacci-hashed (one 32-bit multiply; consecutive
// bricks land far apart), top bits taken. cap = 2^cap_log2 buckets.
__device__ inline uint64_t brick_home(uint64_t k, int cap_log2) {
    const uint32_t f = (uint32_t)k ^ (uint32_t)(k >> 32) * 0x85ebca6bu;
    return (uint64_t)((f * 0x9e3779b1u) >> (32 - cap_log2));
}

struct Shape4 {
    int64_t s0, s1, s2, s3;
};

struct BrickTable {
    uint64_t* head;  // [cap] brick key of each bucket
    int32_t* vals;   // [cap][64] row index of each cell, -1 if empty
    uint64_t cap_mask;
    int cap_log2;
    Shape4 S;   // sparse shape (b, x, y, z)
    Shape4 Sb;  // brick grid: (b, ceil(x/4), ceil(y/4), ceil(z/4))
};

__device__ inline uint64_t brick_key(int b, int bx, int by, int bz, const Shape4& Sb) {
    return (((uint64_t)b * Sb.s1 + bx) * Sb.s2 + by) * Sb.s3 + bz;
}

__device__ inline int brick_cell(int x, int y, int z) { return ((x & 3) << 4) | ((y & 3) << 2) | (z & 3); }

__device__ inline bool in_shape(int b, int x, int y, int z, const Shape4& S) {
    return b >= 0 && b < S.s0 && x >= 0 && x < S.s1 && y >= 0 && y < S.s2 && z >= 0 && z < S.s3;
}

// Workgroups are dispatched round-robin over the 8 XCDs (block b runs on XCD b mod 8). Remapping block b to chunk
// xcd_chunk(b) gives each XCD one contiguous range of chunks, so voxels that share buckets also share an L2.
__device__ inline int64_t xcd_chunk(int64_t b, int64_t n) {
    const int64_t x = b & 7, j = b >> 3, q = n >> 3, r = n & 7;
    return x < r ? x * (q + 1) + j : r * (q + 1) + (x - r) * q + j;
}

__global__ __launch_bounds__(256) void brick_clear_k(uint64_t* head, int64_t cap) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < cap) head[i] = kEmpty;
}

// Finds or claims the bucket of brick key `bk`; `fresh` tells whether this call claimed it (its cells are then
// still to be emptied). Keys only ever change from EMPTY to a brick, so a plain (possibly stale) read that shows a
// key is final, and a stale EMPTY only costs a compare-and-swap that then reports the key. The table has more
// buckets than there can be bricks, so the probe ends within cap steps.
__device__ inline uint32_t brick_claim(const BrickTable& T, uint64_t bk, bool& fresh) {
    uint64_t slot = brick_home(bk, T.cap_log2);
    fresh = false;
    for (uint64_t probe = 0; probe <= T.cap_mask; ++probe) {
        const uint64_t t = T.head[slot];
        if (t == bk) return (uint32_t)slot;
        if (t == kEmpty) {
            const unsigned long long prev =
                atomicCAS((unsigned long long*)&T.head[slot], (unsigned long long)kEmpty, (unsigned long long)bk);
            if (prev == kEmpty) {
                fresh = true;
                return (uint32_t)slot;
            }
            if (prev == bk) return (uint32_t)slot;
        }
        slot = (slot + 1) & T.cap_mask;
    }
    return 0xffffffffu;  // unreachable: the table never fills
}

__device__ inline uint64_t shfl_up_u64(uint64_t v, int off) {
    const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)v, off, 64);
    const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)(v >> 32), off, 64);
    return ((uint64_t)hi << 32) | lo;
}

// Lane index of the first lane of this lane's run: runs are maximal spans of consecutive lanes with head == false
// after a head lane (a max-scan of the head lanes' indices).
__device__ inline int run_start(bool head, int lane) {
    int h = head ? lane : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int t = __shfl_up(h, off, 64);
        if (lane >= off) h = t > h ? t : h;
    }
    return h;
}

// Insertion, pass 1: every brick that holds a voxel gets a bucket with empty cells. Consecutive lanes of a wave in
// the same brick form a run; the run's first lane claims (all runs in parallel; two runs of one brick find the
// same bucket) and the run takes its slot. slot_of[m] = the voxel's bucket.
__global__ __launch_bounds__(256) void brick_claim_k(const int4* __restrict__ coords, int64_t M, BrickTable T,
                                                     uint32_t* __restrict__ slot_of) {
    const int64_t m = xcd_chunk(blockIdx.x, gridDim.x) * 256 + threadIdx.x;
    const int lane = threadIdx.x & 63;
    bool valid = false;
    uint64_t bk = 0;
    if (m < M) {
        const int4 c = coords[m];
        valid = in_shape(c.x, c.y, c.z, c.w, T.S);
        if (valid) bk = brick_key(c.x, c.y >> kBrickLog, c.z >> kBrickLog, c.w >> kBrickLog, T.Sb);
    }
    const bool prev_valid = __shfl_up((int)valid, 1, 64) != 0;
    const uint64_t prev_bk = shfl_up_u64(bk, 1);
    const bool head = valid && (lane == 0 || !prev_valid || prev_bk != bk);
    uint32_t slot = 0xffffffffu;
    bool fresh = false;
    if (head) slot = brick_claim(T, bk, fresh);
    // the wave empties the cells of the buckets it claimed, one coalesced 256-byte store per bucket
    uint64_t todo = __ballot(fresh);
    while (todo) {
        const int l = __builtin_ctzll(todo);
        const uint32_t fs = (uint32_t)__builtin_amdgcn_readlane((int)slot, l);
        T.vals[(uint64_t)fs * 64 + lane] = -1;
        todo &= todo - 1;
    }
    slot = (uint32_t)__shfl((int)slot, run_start(head, lane), 64);
    if (m < M) slot_of[m] = valid ? slot : 0xffffffffu;
}

// Insertion, pass 2 (every bucket claimed and emptied): each voxel writes its row index into its cell.
__global__ __launch_bounds__(256) void brick_store_k(const int4* __restrict__ coords, int64_t M, BrickTable T,
                                                     const uint32_t* __restrict__ slot_of) {
    const int64_t m = xcd_chunk(blockIdx.x, gridDim.x) * 256 + threadIdx.x;
    if (m >= M) return;
    const uint32_t slot = slot_of[m];
    if (slot == 0xffffffffu) return;
    const int4 c = coords[m];
    T.vals[(uint64_t)slot * 64 + brick_cell(c.y, c.z, c.w)] = (int32_t)m;
}

// The bucket of brick key bk, or -1 if the brick holds no voxel; `first` is the key read at the home slot.
__device__ inline int32_t brick_probe(const BrickTable& T, uint64_t bk, uint64_t home, uint64_t first) {
    uint64_t slot = home;
    uint64_t h = first;
    for (uint64_t probe = 0; probe <= T.cap_mask; ++probe) {
        if (h == bk) return (int32_t)slot;
        if (h == kEmpty) break;
        slot = (slot + 1) & T.cap_mask;
        h = T.head[slot];
    }
    return -1;
}

// Query: the 27 neighbours of every voxel (_SortedIndex.lookup semantics, _core.py:114-124: out-of-bounds
// neighbours never hit). Per axis the offsets -1, 0, +1 stay in the voxel's own brick except on a brick face,
// where one of them enters the next brick in direction e = -1 or +1; bucket k = (kx, ky, kz) is the brick with
// the extra step on the axes whose bit is set. The <= 8 buckets are resolved first (every home-slot header loaded
// before any is compared), then each tap picks its bucket through a mux tree shared across taps (x, then y,
// then z) and all 27 cell loads are issued together.
__global__ __launch_bounds__(256) void brick_query_k(const int4* __restrict__ coords, int64_t M, BrickTable T,
                                                     int32_t* __restrict__ nmap_t, int32_t* __restrict__ nmap_rows,
                                                     uint32_t* tile_mask, uint32_t* __restrict__ row_mask) {
    const int64_t m = xcd_chunk(blockIdx.x, gridDim.x) * 256 + threadIdx.x;
    uint32_t rmask = 0;
    if (m < M) {
        const int4 c = coords[m];
        const int p[3] = {c.y, c.z, c.w};
        const int ext[3] = {(int)T.S.s1, (int)T.S.s2, (int)T.S.s3};
        const int bext[3] = {(int)T.Sb.s1, (int)T.Sb.s2, (int)T.Sb.s3};
        const int64_t stride[3] = {T.Sb.s2 * T.Sb.s3, T.Sb.s3, 1};
        const bool bok = c.x >= 0 && c.x < T.S.s0;
        int b0[3], e[3], cp[3][3];
        bool okd[3][3], sel[3][3], eok[3];
#pragma unroll
        for (int a = 0; a < 3; ++a) {
            b0[a] = p[a] >> kBrickLog;
            const int r = p[a] & 3;
            e[a] = r == 0 ? -1 : (r == 3 ? 1 : 0);
            eok[a] = e[a] != 0 && b0[a] + e[a] >= 0 && b0[a] + e[a] < bext[a];
#pragma unroll
            for (int di = 0; di < 3; ++di) {
                const int q = p[a] + di - 1;
                okd[a][di] = q >= 0 && q < ext[a];
                sel[a][di] = (di == 0 && r == 0) || (di == 2 && r == 3);
                cp[a][di] = (q & 3) << (4 - 2 * a);
            }
        }
        const bool own = bok && b0[0] < bext[0] && b0[1] < bext[1] && b0[2] < bext[2] && b0[0] >= 0 &&
                         b0[1] >= 0 && b0[2] >= 0;
        const uint64_t key0 = own ? brick_key(c.x, b0[0], b0[1], b0[2], T.Sb) : 0;
        uint64_t key[8], home[8], first[8];
        bool want[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            bool ok = own;
            int64_t kk = (int64_t)key0;
#pragma unroll
            for (int a = 0; a < 3; ++a)
                if ((k >> (2 - a)) & 1) {
                    ok = ok && eok[a];
                    kk += e[a] * stride[a];
                }
            want[k] = ok;
            key[k] = ok ? (uint64_t)kk : 0;
            home[k] = brick_home(key[k], T.cap_log2);
            first[k] = T.head[home[k]];  // unconditional: all 8 loads are issued before any compare
        }
        int32_t slot[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            slot[k] = -1;
            if (want[k]) slot[k] = brick_probe(T, key[k], home[k], first[k]);
        }
        // Cell loads are unconditional (taps out of bounds or in an absent brick read cell 0 of bucket 0 and are
        // discarded), so no load sits under a branch and all 27 are in flight together.
        uint64_t idx[27];
        uint32_t okbits = 0;
#pragma unroll
        for (int dx = 0; dx < 3; ++dx) {
            int32_t sx[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) sx[j] = sel[0][dx] ? slot[4 + j] : slot[j];
#pragma unroll
            for (int dy = 0; dy < 3; ++dy) {
                int32_t sy[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) sy[j] = sel[1][dy] ? sx[2 + j] : sx[j];
#pragma unroll
                for (int dz = 0; dz < 3; ++dz) {
                    const int v = dx * 9 + dy * 3 + dz;
                    const int32_t sl = sel[2][dz] ? sy[1] : sy[0];
                    const int cell = cp[0][dx] | cp[1][dy] | cp[2][dz];
                    const bool ok = okd[0][dx] && okd[1][dy] && okd[2][dz] && sl >= 0;
                    idx[v] = ok ? (uint64_t)sl * 64 + cell : 0;
                    okbits |= (ok ? 1u : 0u) << v;
                }
            }
        }
        int hit[27];
#pragma unroll
        for (int v = 0; v < 27; ++v) hit[v] = T.vals[idx[v]];
#pragma unroll
        for (int v = 0; v < 27; ++v) {
            hit[v] = ((okbits >> v) & 1u) ? hit[v] : -1;
            rmask |= (hit[v] >= 0 ? 1u : 0u) << v;
        }
        if (nmap_t) {
#pragma unroll
            for (int v = 0; v < 27; ++v) nmap_t[(int64_t)v * M + m] = hit[v];
        }
        if (nmap_rows) {
#pragma unroll
            for (int v = 0; v < 27; ++v) nmap_rows[m * 27 + v] = hit[v];
        }
        if (row_mask) row_mask[m] = rmask;
    }
    store_tile_mask(rmask, m, M, tile_mask);
}

// ------------------------------------------------------------------------------------------------------------
// Generic map for coordinates in increasing _linearise order (_core.py:89-94): the order of _SortedIndex's sorted
// keys (_core.py:105-124), and the order voxelisation and pool caches produce. The voxels of a (b, x, y) column are
// then one contiguous run in increasing z, so a dense table over the B * X * Y columns holds each run's [start, end)
// and a neighbour is found in its column's run: no hashing, no atomics, no probing. The table is never cleared:
// sorted_heads_k rewrites the entry of every column this set holds, and an entry is trusted only if it names a row
// range of this set whose first row lies in that column, which no stale entry of an absent column can.

__device__ inline uint64_t lin_key_u(const int4& c, const Shape4& S) {
    return (((uint64_t)(uint32_t)c.x * (uint64_t)S.s1 + (uint32_t)c.y) * (uint64_t)S.s2 + (uint32_t)c.z) *
               (uint64_t)S.s3 + (uint32_t)c.w;
}

// Each row checks that it lies inside the shape and follows the previous row in _linearise order (else the status
// word gets bit 0: the map is then not valid); the first and last rows of a column's run write its table entry.
// Columns are numbered (b X + x) Y + y < 2^31.
__global__ __launch_bounds__(256) void sorted_heads_k(const int4* __restrict__ coords, int64_t M, Shape4 S,
                                                      int2* __restrict__ cols, uint32_t* __restrict__ status) {
    const int64_t m = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (m >= M) return;
    const int4 c = coords[m];
    const int4 pv = coords[m > 0 ? m - 1 : 0];
    const int4 nx = coords[m + 1 < M ? m + 1 : m];
    const bool inside = in_shape(c.x, c.y, c.z, c.w, S);
    const bool bad = !inside || (m > 0 && !(lin_key_u(pv, S) < lin_key_u(c, S)));
    if (bad) {
        __hip_atomic_fetch_or(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    const bool first = m == 0 || pv.x != c.x || pv.y != c.y || pv.z != c.z;
    const bool last = m + 1 == M || nx.x != c.x || nx.y != c.y || nx.z != c.z;
    int32_t* e = (int32_t*)&cols[((uint32_t)c.x * (uint32_t)S.s1 + (uint32_t)c.y) * (uint32_t)S.s2 + (uint32_t)c.z];
    if (first) e[0] = (int32_t)m;
    if (last) e[1] = (int32_t)(m + 1);
}

// Query (_SortedIndex.lookup semantics, _core.py:114-124): the 9 neighbouring columns' entries are loaded together
// and validated by their first rows; in each run the lower bound of z - 1 (the first row itself, or a binary search
// in lock step over the columns that start lower, bounded by the row z - 1 would have without gaps), then the rows
// holding z - 1, z, z + 1 among the next three, each placed by its z. Same outputs as brick_query_k.
__global__ __launch_bounds__(256) void sorted_query_k(const int4* __restrict__ coords, int64_t M, Shape4 S,
                                                      const int2* __restrict__ cols, int32_t* __restrict__ nmap_t,
                                                      int32_t* __restrict__ nmap_rows, uint32_t* tile_mask,
                                                      uint32_t* __restrict__ row_mask) {
    const int64_t m = xcd_chunk(blockIdx.x, gridDim.x) * 256 + threadIdx.x;
    uint32_t rmask = 0;
    if (m < M) {
        const int4 c = coords[m];
        const int zlo = c.w - 1;
        const int X = (int)S.s1, Y = (int)S.s2;
        const uint32_t cb = (uint32_t)c.x * (uint32_t)X;
        int2 r[9];
        bool in[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            const int x = c.y + k / 3 - 1, y = c.z + k % 3 - 1;
            in[k] = x >= 0 && x < X && y >= 0 && y < Y;
            r[k] = cols[in[k] ? (cb + (uint32_t)x) * (uint32_t)Y + (uint32_t)y : 0u];  // the 9 loads together
        }
        int4 h[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            in[k] = in[k] && r[k].x >= 0 && r[k].x < r[k].y && (int64_t)r[k].y <= M;
            h[k] = coords[in[k] ? r[k].x : 0];
        }
        // lo: the first row of the run with z >= z - 1 (searched over [lo, hi) when the run starts lower)
        int32_t lo[9], hi[9];
        bool srch = false;
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            const int x = c.y + k / 3 - 1, y = c.z + k % 3 - 1;
            in[k] = in[k] && h[k].x == c.x && h[k].y == x && h[k].z == y;
            // z rises by at least 1 per row, so the row start + (z - 1 - z_first) + 1 already lies above z - 1
            const bool below = in[k] && h[k].w < zlo;
            const int64_t cap = (int64_t)r[k].x + ((int64_t)zlo - h[k].w) + 1;
            lo[k] = below ? r[k].x + 1 : r[k].x;
            hi[k] = below ? (int32_t)(cap < r[k].y ? cap : r[k].y) : r[k].x;
            srch = srch || hi[k] > lo[k];
        }
        while (srch) {  // every search range halves per trip
            int zm[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) zm[k] = coords[hi[k] > lo[k] ? lo[k] + (hi[k] - lo[k]) / 2 : 0].w;
            srch = false;
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                if (hi[k] > lo[k]) {
                    const int32_t mid = lo[k] + (hi[k] - lo[k]) / 2;
                    if (zm[k] < zlo) lo[k] = mid + 1;
                    else hi[k] = mid;
                    srch = srch || hi[k] > lo[k];
                }
            }
        }
        // rows lo, lo + 1, lo + 2 hold the run's z values from z - 1 up, in order: each is placed by its z
        int hit[27];
#pragma unroll
        for (int v = 0; v < 27; ++v) hit[v] = -1;
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            int zf[3];
#pragma unroll
            for (int j = 0; j < 3; ++j) zf[j] = coords[in[k] && lo[k] + j < r[k].y ? lo[k] + j : 0].w;
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                const int dz = zf[j] - zlo;
                const bool ok = in[k] && lo[k] + j < r[k].y;
#pragma unroll
                for (int d = 0; d < 3; ++d)
                    if (ok && dz == d) hit[3 * k + d] = lo[k] + j;
            }
        }
#pragma unroll
        for (int v = 0; v < 27; ++v) rmask |= (hit[v] >= 0 ? 1u : 0u) << v;
        if (nmap_t) {
            int32_t* o = nmap_t + m;
#pragma unroll
            for (int v = 0; v < 27; ++v) o[(int64_t)v * M] = hit[v];
        }
        if (nmap_rows) {
#pragma unroll
            for (int v = 0; v < 27; ++v) nmap_rows[m * 27 + v] = hit[v];
        }
        if (row_mask) row_mask[m] = rmask;
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
    hipLaunchKernelGGL(minmax_init_k, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, s, zmin, zmax, B);
    if (int e = check_launch("minmax_init_k")) return e;
    const int HW = H * W;
    const int nb = (HW + 255) / 256;
    dim3 grid(nb < kVoxBlocks ? nb : kVoxBlocks, B);
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

static size_t align_up_sz(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Buckets: a power of two above 1.5x the most bricks M voxels can occupy (load factor < 2/3).
static int64_t hash_capacity(int64_t bricks) {
    int64_t cap = 1024;
    while (cap < bricks + bricks / 2) cap <<= 1;
    return cap;
}

static size_t hash_bytes(int64_t cap, int64_t M) {
    return align_up_sz((size_t)cap * sizeof(uint64_t), 256) + align_up_sz((size_t)cap * 64 * sizeof(int32_t), 256) +
           (size_t)M * sizeof(uint32_t);
}

size_t pmg_hash_workspace_bytes(int64_t M) {
    if (M < 0) return 0;
    return hash_bytes(hash_capacity(M), M);
}

int pmg_nmap_hash(const int32_t* coords, int64_t M, const int64_t* shape, int32_t* nmap_t, int32_t* nmap_rows,
                  uint32_t* tile_mask, uint32_t* row_mask, void* workspace, size_t workspace_bytes, void* stream) {
    PMG_REQUIRE(coords && shape, "null argument");
    PMG_REQUIRE(M >= 0 && M <= INT_MAX, "bad voxel count");
    PMG_REQUIRE(aligned16(coords), "coords must be 16-byte aligned");
    for (int d = 0; d < 4; ++d) PMG_REQUIRE(shape[d] > 0 && shape[d] <= INT_MAX, "bad sparse shape");
    // Brick keys must fit in 63 bits so that no key equals the EMPTY marker.
    const Shape4 Sb{shape[0], (shape[1] + 3) / 4, (shape[2] + 3) / 4, (shape[3] + 3) / 4};
    const double span = (double)Sb.s0 * (double)Sb.s1 * (double)Sb.s2 * (double)Sb.s3;
    PMG_REQUIRE(span < 9.0e18, "sparse shape too large for 64-bit keys");
    PMG_REQUIRE(workspace && workspace_bytes >= pmg_hash_workspace_bytes(M), "workspace too small");
    PMG_REQUIRE(M < ((int64_t)1 << 30), "at most 2^30 voxels (32-bit bucket hashing)");
    if (M == 0) return PMG_OK;
    hipStream_t s = (hipStream_t)stream;
    const int64_t bricks = span < (double)M ? (int64_t)span : M;
    const int64_t cap = hash_capacity(bricks);
    BrickTable T;
    T.head = (uint64_t*)workspace;
    T.vals = (int32_t*)((char*)workspace + align_up_sz((size_t)cap * sizeof(uint64_t), 256));
    uint32_t* slot_of = (uint32_t*)((char*)T.vals + align_up_sz((size_t)cap * 64 * sizeof(int32_t), 256));
    T.cap_mask = (uint64_t)(cap - 1);
    T.cap_log2 = 0;
    while (((int64_t)1 << T.cap_log2) < cap) ++T.cap_log2;
    T.S = Shape4{shape[0], shape[1], shape[2], shape[3]};
    T.Sb = Sb;
    hipLaunchKernelGGL(brick_clear_k, dim3((unsigned)((cap + 255) / 256)), dim3(256), 0, s, T.head, cap);
    if (int e = check_launch("brick_clear_k")) return e;
    const dim3 g((unsigned)((M + 255) / 256));
    hipLaunchKernelGGL(brick_claim_k, g, dim3(256), 0, s, (const int4*)coords, M, T, slot_of);
    if (int e = check_launch("brick_claim_k")) return e;
    hipLaunchKernelGGL(brick_store_k, g, dim3(256), 0, s, (const int4*)coords, M, T, (const uint32_t*)slot_of);
    if (int e = check_launch("brick_store_k")) return e;
    hipLaunchKernelGGL(brick_query_k, g, dim3(256), 0, s, (const int4*)coords, M, T, nmap_t, nmap_rows, tile_mask,
                       row_mask);
    return check_launch("brick_query_k");
}

size_t pmg_sorted_workspace_bytes(const int64_t* shape) {
    if (!shape) return 0;
    for (int d = 0; d < 3; ++d)
        if (shape[d] <= 0) return 0;
    const double cols = (double)shape[0] * (double)shape[1] * (double)shape[2];
    if (cols > (double)((int64_t)1 << 31)) return 0;
    return 256 + (size_t)cols * sizeof(int2);
}

int pmg_nmap_sorted(const int32_t* coords, int64_t M, const int64_t* shape, int32_t* nmap_t, int32_t* nmap_rows,
                    uint32_t* tile_mask, uint32_t* row_mask, void* workspace, size_t workspace_bytes, void* stream) {
    PMG_REQUIRE(coords && shape, "null argument");
    PMG_REQUIRE(M >= 0 && M < ((int64_t)1 << 31) - 1, "bad voxel count");
    PMG_REQUIRE(aligned16(coords), "coords must be 16-byte aligned");
    for (int d = 0; d < 4; ++d) PMG_REQUIRE(shape[d] > 0 && shape[d] <= INT_MAX, "bad sparse shape");
    const double span = (double)shape[0] * (double)shape[1] * (double)shape[2] * (double)shape[3];
    PMG_REQUIRE(span < 1.8e19, "sparse shape too large for 64-bit keys");
    const size_t need = pmg_sorted_workspace_bytes(shape);
    PMG_REQUIRE(need > 0, "more than 2^31 (b, x, y) columns");
    PMG_REQUIRE(workspace && workspace_bytes >= need && aligned16(workspace), "workspace too small");
    if (M == 0) return PMG_OK;
    hipStream_t s = (hipStream_t)stream;
    const Shape4 S{shape[0], shape[1], shape[2], shape[3]};
    uint32_t* status = (uint32_t*)workspace;
    int2* cols = (int2*)((char*)workspace + 256);
    const dim3 g((unsigned)((M + 255) / 256));
    hipLaunchKernelGGL(sorted_heads_k, g, dim3(256), 0, s, (const int4*)coords, M, S, cols, status);
    if (int e = check_launch("sorted_heads_k")) return e;
    hipLaunchKernelGGL(sorted_query_k, g, dim3(256), 0, s, (const int4*)coords, M, S, (const int2*)cols, nmap_t,
                       nmap_rows, tile_mask, row_mask);
    return check_launch("sorted_query_k");
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
