// Sparse pooling and nearest upsampling of the multi-level refiner: build_pool_cache, sparse_pool and
// sparse_upsample (promptmoge/_fallback/flex_gemm/_core.py:339-505) on the GPU.
//
// Pool cache (perfect partition: kernel == stride, padding 0). Every input voxel's parent key is its coordinates
// divided by the stride, linearised on the output grid as _linearise does (_core.py:89-94). The output voxels are
// the distinct parent keys in increasing order (torch.unique(sorted=True)); `parent` maps every input voxel to
// its output row; `seg_indices` is the stable argsort of `parent` (the input rows grouped by output row, each
// group in input order) and `seg_offsets` the group boundaries. All of it comes from one stable LSD radix sort of
// (key, input row) pairs over the key's significant bits (8 bits per pass, three kernels per pass as below),
// after which a flag marks each first occurrence of a key and an exclusive scan of the flags numbers the
// output rows. The number of output rows is written to device memory (the caller reads it once, as the
// reference's int(...) does).
//
// Radix pass, over tiles of 2048 keys: pool_hist_k counts the tile's digits (LDS atomics), pool_scan_k (one
// block) turns the digit-major counts into each (digit, tile)'s output base, pool_scatter_k places the keys of
// each tile in 8 rounds of 256: a key's rank among equal digits of its round comes from 9 wave ballots plus the
// counts of the lower waves, so the pass is stable and deterministic.
//
// sparse_pool: one thread per (output row, 4 channels) sums its group's rows in seg_indices order -- input order,
// the order of the reference's index_add_ -- in fp32 and divides by the group size ('mean'). sparse_upsample:
// out[i] = feats[parent[i]], a row gather.
#include <climits>

#include "pmg_common.h"
#include "pmg_internal.h"

namespace pmg {

constexpr int kPoolThreads = 256;
constexpr int kPoolRounds = 8;
constexpr int kPoolTile = kPoolThreads * kPoolRounds;  // 2048 keys per tile

struct PoolGeom {
    int64_t in[4];   // B, X, Y, Z of the input grid
    int64_t out[4];  // B, X', Y', Z' of the output grid
    int s[3];        // stride per spatial dimension
};

__global__ __launch_bounds__(256) void pool_keys_k(const int4* __restrict__ coords, int64_t M, PoolGeom pg,
                                                   uint64_t* __restrict__ keys,
                                                   unsigned long long* __restrict__ counts) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= M) return;
    const int4 c = coords[i];
    const bool in = c.x >= 0 && c.x < pg.in[0] && c.y >= 0 && c.y < pg.in[1] && c.z >= 0 && c.z < pg.in[2] &&
                    c.w >= 0 && c.w < pg.in[3];
    uint64_t key = ~0ull;  // an out-of-grid voxel sorts last; the caller rejects the cache
    if (in) {
        const int64_t x = c.y / pg.s[0], y = c.z / pg.s[1], z = c.w / pg.s[2];
        key = (uint64_t)(((c.x * pg.out[1] + x) * pg.out[2] + y) * pg.out[3] + z);
    } else {
        atomicAdd(&counts[1], 1ull);
    }
    keys[i] = key;
}

__global__ __launch_bounds__(kPoolThreads) void pool_hist_k(const uint64_t* __restrict__ keys, int64_t M, int shift,
                                                            int ntile, uint32_t* __restrict__ hist) {
    __shared__ uint32_t h[256];
    h[threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kPoolTile;
    for (int k = 0; k < kPoolRounds; ++k) {
        const int64_t i = base + k * kPoolThreads + threadIdx.x;
        if (i < M) atomicAdd(&h[(keys[i] >> shift) & 0xffu], 1u);
    }
    __syncthreads();
    hist[(int64_t)threadIdx.x * ntile + blockIdx.x] = h[threadIdx.x];
}

// One block of 1024 threads: exclusive scan of n counts in place; the total goes to *total if given.
// Exclusive scan of v[0, n) in place (and its total), one block: chunks of 8192 values are loaded coalesced into
// LDS (all loads in flight at once), each thread scans 8 consecutive values, the 1024 thread sums are scanned by
// wave shuffles and the 16 wave totals, and the chunk is stored back coalesced with the running carry.
__global__ __launch_bounds__(1024) void pool_scan_k(uint32_t* v, int n, unsigned long long* total) {
    constexpr int PER = 8, CH = 1024 * PER;
    __shared__ uint32_t s_v[CH];
    __shared__ uint32_t part[16];
    const int t = threadIdx.x;
    uint32_t carry = 0u;
    for (int base = 0; base < n; base += CH) {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = base + k * 1024 + t;
            s_v[k * 1024 + t] = i < n ? v[i] : 0u;
        }
        __syncthreads();
        uint32_t loc[PER], sum = 0u;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            loc[k] = sum;
            sum += s_v[t * PER + k];
        }
        // inclusive scan of the thread sums: within each wave by shuffles, then the 16 wave totals
        uint32_t inc = sum;
        const int lane = t & 63, wv = t >> 6;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t y = __shfl_up(inc, off, 64);
            if (lane >= off) inc += y;
        }
        if (lane == 63) part[wv] = inc;
        __syncthreads();
        uint32_t wbase = 0u;
        for (int q = 0; q < wv; ++q) wbase += part[q];
        uint32_t ctot = 0u;
        for (int q = 0; q < 16; ++q) ctot += part[q];
        const uint32_t before = carry + wbase + inc - sum;
#pragma unroll
        for (int k = 0; k < PER; ++k) s_v[t * PER + k] = before + loc[k];
        carry += ctot;
        __syncthreads();
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = base + k * 1024 + t;
            if (i < n) v[i] = s_v[k * 1024 + t];
        }
        __syncthreads();  // the next chunk overwrites s_v and part
    }
    if (total && t == 0) total[0] = carry;
}

// Large scans run on a grid: pool_scan_chunk_k scans each 8192-value chunk in place (local exclusive values) and
// writes its total to ctot[chunk]; the totals are scanned by pool_scan_k; pool_scan_add_k adds them back.
__global__ __launch_bounds__(1024) void pool_scan_chunk_k(uint32_t* v, int n, uint32_t* ctot) {
    constexpr int PER = 8, CH = 1024 * PER;
    __shared__ uint32_t s_v[CH];
    __shared__ uint32_t part[16];
    const int t = threadIdx.x, base = blockIdx.x * CH;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = base + k * 1024 + t;
        s_v[k * 1024 + t] = i < n ? v[i] : 0u;
    }
    __syncthreads();
    uint32_t loc[PER], sum = 0u;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        loc[k] = sum;
        sum += s_v[t * PER + k];
    }
    uint32_t inc = sum;
    const int lane = t & 63, wv = t >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(inc, off, 64);
        if (lane >= off) inc += y;
    }
    if (lane == 63) part[wv] = inc;
    __syncthreads();
    uint32_t wbase = 0u, ctot_ = 0u;
    for (int q = 0; q < 16; ++q) {
        wbase += q < wv ? part[q] : 0u;
        ctot_ += part[q];
    }
    const uint32_t before = wbase + inc - sum;
#pragma unroll
    for (int k = 0; k < PER; ++k) s_v[t * PER + k] = before + loc[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = base + k * 1024 + t;
        if (i < n) v[i] = s_v[k * 1024 + t];
    }
    if (t == 0) ctot[blockIdx.x] = ctot_;
}

__global__ __launch_bounds__(1024) void pool_scan_add_k(uint32_t* v, int n, const uint32_t* ctot) {
    constexpr int CH = 1024 * 8;
    const uint32_t add = ctot[blockIdx.x];
    for (int k = 0; k < 8; ++k) {
        const int i = blockIdx.x * CH + k * 1024 + threadIdx.x;
        if (i < n) v[i] += add;
    }
}

// Exclusive scan of v[0, n) (and its total): one block for up to one chunk, else the three-kernel grid scan.
static int pool_scan(uint32_t* v, int n, unsigned long long* total, uint32_t* ctot, hipStream_t s) {
    constexpr int CH = 1024 * 8;
    if (n <= CH) {
        hipLaunchKernelGGL(pool_scan_k, dim3(1), dim3(1024), 0, s, v, n, total);
        return check_launch("pool_scan_k");
    }
    const int nc = (n + CH - 1) / CH;
    hipLaunchKernelGGL(pool_scan_chunk_k, dim3(nc), dim3(1024), 0, s, v, n, ctot);
    if (int e = check_launch("pool_scan_chunk_k")) return e;
    hipLaunchKernelGGL(pool_scan_k, dim3(1), dim3(1024), 0, s, ctot, nc, total);
    if (int e = check_launch("pool_scan_k")) return e;
    hipLaunchKernelGGL(pool_scan_add_k, dim3(nc), dim3(1024), 0, s, v, n, (const uint32_t*)ctot);
    return check_launch("pool_scan_add_k");
}

// vals_in == nullptr: the value of key i is i (the first pass).
__global__ __launch_bounds__(kPoolThreads) void pool_scatter_k(const uint64_t* __restrict__ keys_in,
                                                               const int32_t* __restrict__ vals_in, int64_t M,
                                                               int shift, int ntile, const uint32_t* __restrict__ off,
                                                               uint64_t* __restrict__ keys_out,
                                                               int32_t* __restrict__ vals_out) {
    constexpr int NW = kPoolThreads / 64;
    __shared__ uint32_t run[256];      // keys of each digit this tile has placed
    __shared__ uint32_t cnt[NW][256];  // this round's count of each digit per wave
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    run[tid] = off[(int64_t)tid * ntile + blockIdx.x];
    const uint64_t below = (1ull << lane) - 1ull;
    const int64_t base = (int64_t)blockIdx.x * kPoolTile;
    for (int k = 0; k < kPoolRounds; ++k) {
        const int64_t i = base + k * kPoolThreads + tid;
        const bool ok = i < M;
        const uint64_t key = ok ? keys_in[i] : 0ull;
        const int32_t val = ok ? (vals_in ? vals_in[i] : (int32_t)i) : 0;
        const uint32_t d = ok ? (uint32_t)((key >> shift) & 0xffu) : 256u;  // 256 matches no real digit
        uint64_t peers = __ballot(ok);
#pragma unroll
        for (int b = 0; b < 9; ++b) {
            const uint64_t bb = __ballot((d >> b) & 1u);
            peers &= ((d >> b) & 1u) ? bb : ~bb;
        }
        for (int e = lane; e < 256; e += 64) cnt[w][e] = 0;
        __syncthreads();
        const uint32_t rank = (uint32_t)__popcll(peers & below);
        if (ok && rank == 0) cnt[w][d] = (uint32_t)__popcll(peers);
        __syncthreads();
        if (ok) {
            uint32_t pos = run[d] + rank;
            for (int q = 0; q < w; ++q) pos += cnt[q][d];
            keys_out[pos] = key;
            vals_out[pos] = val;
        }
        __syncthreads();
        uint32_t add = 0;
#pragma unroll
        for (int q = 0; q < NW; ++q) add += cnt[q][tid];
        run[tid] += add;
        __syncthreads();  // the next round clears cnt[] and reads run[]
    }
}

__device__ inline bool pool_first(const uint64_t* sk, int64_t i) { return i == 0 || sk[i] != sk[i - 1]; }

// Number of first occurrences in each tile of the sorted keys.
__global__ __launch_bounds__(kPoolThreads) void pool_count_k(const uint64_t* __restrict__ sk, int64_t M,
                                                             uint32_t* __restrict__ tile_cnt) {
    __shared__ uint32_t part[kPoolThreads / 64];
    const int64_t base = (int64_t)blockIdx.x * kPoolTile;
    uint32_t c = 0;
    for (int k = 0; k < kPoolRounds; ++k) {
        const int64_t i = base + k * kPoolThreads + threadIdx.x;
        c += (i < M && pool_first(sk, i)) ? 1u : 0u;
    }
    c = wave_incl_scan_u32(c);
    if ((threadIdx.x & 63) == 63) part[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int q = 0; q < kPoolThreads / 64; ++q) t += part[q];
        tile_cnt[blockIdx.x] = t;
    }
}

// Output row numbers: parent, seg_offsets, out_coords (decoded from the key).
__global__ __launch_bounds__(kPoolThreads) void pool_emit_k(const uint64_t* __restrict__ sk,
                                                            const int32_t* __restrict__ order, int64_t M,
                                                            const uint32_t* __restrict__ tile_base, PoolGeom pg,
                                                            const unsigned long long* __restrict__ counts,
                                                            int32_t* __restrict__ parent,
                                                            int64_t* __restrict__ seg_offsets,
                                                            int4* __restrict__ out_coords) {
    constexpr int NW = kPoolThreads / 64;
    __shared__ uint32_t part[NW];
    __shared__ uint32_t s_run;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    if (tid == 0) s_run = tile_base[blockIdx.x];
    const uint64_t below = (1ull << lane) - 1ull;
    const int64_t base = (int64_t)blockIdx.x * kPoolTile;
    for (int k = 0; k < kPoolRounds; ++k) {
        const int64_t i = base + k * kPoolThreads + tid;
        const bool ok = i < M;
        const bool f = ok && pool_first(sk, i);
        const uint64_t fb = __ballot(f);
        if (lane == 0) part[w] = (uint32_t)__popcll(fb);
        __syncthreads();
        uint32_t before = s_run;
        for (int q = 0; q < w; ++q) before += part[q];
        // rank = output rows started at or before i, minus one
        const uint32_t rank = before + (uint32_t)__popcll(fb & below) + (f ? 1u : 0u) - 1u;
        if (ok) {
            parent[order[i]] = (int32_t)rank;
            if (f) {
                seg_offsets[rank] = i;
                uint64_t key = sk[i];
                int4 c;
                c.w = (int)(key % (uint64_t)pg.out[3]);
                key /= (uint64_t)pg.out[3];
                c.z = (int)(key % (uint64_t)pg.out[2]);
                key /= (uint64_t)pg.out[2];
                c.y = (int)(key % (uint64_t)pg.out[1]);
                c.x = (int)(key / (uint64_t)pg.out[1]);
                out_coords[rank] = c;
            }
            if (i == M - 1) seg_offsets[counts[0]] = M;
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t t = 0;
            for (int q = 0; q < NW; ++q) t += part[q];
            s_run += t;
        }
        __syncthreads();
    }
}

// out[r][c0..c0+3] = sum (mean) of feats[seg_indices[k]][c0..c0+3], k in [seg_offsets[r], seg_offsets[r+1]), in
// that order; one thread per (row, 4 channels).
__global__ __launch_bounds__(256) void pool_reduce_k(const float* __restrict__ feats, int C,
                                                     const int32_t* __restrict__ seg_indices,
                                                     const int64_t* __restrict__ seg_offsets, int64_t num_out,
                                                     int mean, float* __restrict__ out) {
    const int q4 = C / 4;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= num_out * q4) return;
    const int64_t r = t / q4;
    const int c0 = (int)(t - r * q4) * 4;
    const int64_t lo = seg_offsets[r], hi = seg_offsets[r + 1];
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    for (int64_t k = lo; k < hi; ++k) {
        const float4 v = *(const float4*)(feats + (int64_t)seg_indices[k] * C + c0);
        a0 = a0 + v.x;
        a1 = a1 + v.y;
        a2 = a2 + v.z;
        a3 = a3 + v.w;
    }
    if (mean) {
        const int64_t n = hi - lo;
        const float d = (float)(n > 1 ? n : 1);
        a0 = a0 / d;
        a1 = a1 / d;
        a2 = a2 / d;
        a3 = a3 / d;
    }
    *(float4*)(out + r * C + c0) = make_float4(a0, a1, a2, a3);
}

// out[i] = feats[parent[i]] for rows of row_bytes (a multiple of 16): one thread per 16 bytes.
__global__ __launch_bounds__(256) void upsample_k(const v4i* __restrict__ feats, const int32_t* __restrict__ parent,
                                                  int64_t rows_out, int64_t row_v4, v4i* __restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= rows_out * row_v4) return;
    const int64_t i = t / row_v4, e = t - i * row_v4;
    out[t] = feats[(int64_t)parent[i] * row_v4 + e];
}

static size_t pool_align(size_t x) { return (x + 255) & ~(size_t)255; }

static int64_t pool_tiles(int64_t M) { return (M + kPoolTile - 1) / kPoolTile; }

size_t radix_sort_workspace_bytes(int64_t M) {
    const size_t n = (size_t)(M > 0 ? M : 1);
    const size_t nt = (size_t)pool_tiles(M > 0 ? M : 1);
    return 2 * pool_align(n * 8) + 2 * pool_align(n * 4) + pool_align(256 * nt * 4) + pool_align(nt * 4) +
           pool_align((256 * nt / 8192 + 2) * 4);
}

RadixBufs radix_bufs(void* workspace, int64_t M) {
    const size_t n = (size_t)(M > 0 ? M : 1);
    const size_t nt = (size_t)pool_tiles(M > 0 ? M : 1);
    char* p = (char*)workspace;
    RadixBufs r;
    r.keys[0] = (uint64_t*)p;
    r.keys[1] = (uint64_t*)(p + pool_align(n * 8));
    p += 2 * pool_align(n * 8);
    r.vals[0] = (int32_t*)p;
    r.vals[1] = (int32_t*)(p + pool_align(n * 4));
    p += 2 * pool_align(n * 4);
    r.hist = (uint32_t*)p;
    p += pool_align(256 * nt * 4);
    r.tcnt = (uint32_t*)p;
    p += pool_align(nt * 4);
    r.ctot = (uint32_t*)p;
    return r;
}

int radix_sort_pairs(RadixBufs& r, int64_t M, int bits, int32_t* vals_final, hipStream_t s) {
    const int nt = (int)pool_tiles(M);
    const int npass = (bits + 7) / 8;
    int cur = 0;
    for (int pass = 0; pass < npass; ++pass) {
        const int shift = 8 * pass;
        const uint64_t* kin = r.keys[cur];
        const int32_t* vin = pass == 0 ? nullptr : r.vals[cur];
        uint64_t* kout = r.keys[cur ^ 1];
        int32_t* vout = pass == npass - 1 ? vals_final : r.vals[cur ^ 1];
        hipLaunchKernelGGL(pool_hist_k, dim3(nt), dim3(kPoolThreads), 0, s, kin, M, shift, nt, r.hist);
        if (int e = check_launch("pool_hist_k")) return e;
        if (int e = pool_scan(r.hist, 256 * nt, nullptr, r.ctot, s)) return e;
        hipLaunchKernelGGL(pool_scatter_k, dim3(nt), dim3(kPoolThreads), 0, s, kin, vin, M, shift, nt,
                           (const uint32_t*)r.hist, kout, vout);
        if (int e = check_launch("pool_scatter_k")) return e;
        cur ^= 1;
    }
    r.sorted = cur;
    return PMG_OK;
}

}  // namespace pmg

using namespace pmg;

extern "C" {

size_t pmg_pool_cache_workspace_bytes(int64_t M) { return M < 0 ? 0 : radix_sort_workspace_bytes(M); }

int pmg_pool_cache(const int32_t* coords, int64_t M, const int64_t* sparse_shape, const int32_t* stride,
                   const int64_t* out_sparse_shape, int32_t* out_coords, int32_t* parent, int32_t* seg_indices,
                   int64_t* seg_offsets, int64_t* counts, void* workspace, size_t workspace_bytes, void* stream) {
    PMG_REQUIRE(coords && sparse_shape && stride && out_sparse_shape && out_coords && parent && seg_indices &&
                    seg_offsets && counts && workspace,
                "null buffer");
    PMG_REQUIRE(M >= 0 && M < ((int64_t)1 << 31), "bad voxel count");
    PMG_REQUIRE(pool_tiles(M) * 256 <= INT_MAX, "too many voxels");
    PMG_REQUIRE(workspace_bytes >= pmg_pool_cache_workspace_bytes(M), "workspace too small");
    PMG_REQUIRE(aligned16(coords) && aligned16(out_coords), "coords must be 16-byte aligned");
    PoolGeom pg;
    uint64_t total = 1;
    for (int d = 0; d < 4; ++d) {
        PMG_REQUIRE(sparse_shape[d] > 0 && out_sparse_shape[d] > 0, "bad sparse shape");
        pg.in[d] = sparse_shape[d];
        pg.out[d] = out_sparse_shape[d];
        PMG_REQUIRE(total <= (uint64_t)INT64_MAX / (uint64_t)pg.out[d], "output grid too large");
        total *= (uint64_t)pg.out[d];
    }
    PMG_REQUIRE(pg.out[0] == pg.in[0], "the batch dimension is not pooled");
    for (int d = 0; d < 3; ++d) {
        PMG_REQUIRE(stride[d] >= 1, "bad stride");
        pg.s[d] = stride[d];
        // every pooled coordinate must fit the output grid
        PMG_REQUIRE((pg.in[d + 1] - 1) / stride[d] < pg.out[d + 1], "output grid smaller than the pooled input");
    }
    hipStream_t s = (hipStream_t)stream;
    fill_u32(counts, 0u, 4, s);  // counts[0] = output rows, counts[1] = voxels outside the input grid
    if (int e = check_launch("fill_u32")) return e;
    if (M == 0) {
        fill_u32(seg_offsets, 0u, 2, s);
        return check_launch("fill_u32");
    }
    const int nt = (int)pool_tiles(M);
    RadixBufs rb = radix_bufs(workspace, M);
    uint32_t* tcnt = rb.tcnt;
    uint32_t* ctot = rb.ctot;

    const unsigned g256 = (unsigned)((M + 255) / 256);
    hipLaunchKernelGGL(pool_keys_k, dim3(g256), dim3(256), 0, s, (const int4*)coords, M, pg, rb.keys[0],
                       (unsigned long long*)counts);
    if (int e = check_launch("pool_keys_k")) return e;
    // stable LSD radix sort of (key, row) over the significant bits of the output-grid keys
    const int bits = total > 1 ? 64 - __builtin_clzll(total - 1) : 1;
    if (int e = radix_sort_pairs(rb, M, bits, seg_indices, s)) return e;
    const uint64_t* sk = rb.keys[rb.sorted];
    hipLaunchKernelGGL(pool_count_k, dim3(nt), dim3(kPoolThreads), 0, s, sk, M, tcnt);
    if (int e = check_launch("pool_count_k")) return e;
    if (int e = pool_scan(tcnt, nt, (unsigned long long*)counts, ctot, s)) return e;
    hipLaunchKernelGGL(pool_emit_k, dim3(nt), dim3(kPoolThreads), 0, s, sk, (const int32_t*)seg_indices, M,
                       (const uint32_t*)tcnt, pg, (const unsigned long long*)counts, parent, seg_offsets,
                       (int4*)out_coords);
    return check_launch("pool_emit_k");
}

int pmg_sparse_pool(const float* feats, int64_t M, int C, const int32_t* seg_indices, const int64_t* seg_offsets,
                    int64_t num_out, int reduce, float* out, void* stream) {
    PMG_REQUIRE(feats && seg_indices && seg_offsets && out, "null buffer");
    PMG_REQUIRE(M >= 0 && num_out >= 0 && num_out <= M, "bad row counts");
    PMG_REQUIRE(C > 0 && C % 4 == 0, "C must be a positive multiple of 4");
    PMG_REQUIRE(reduce == 0 || reduce == 1, "reduce must be 0 (sum) or 1 (mean)");
    PMG_REQUIRE(aligned16(feats) && aligned16(out), "feats and out must be 16-byte aligned");
    if (num_out == 0) return PMG_OK;
    const int64_t threads = num_out * (C / 4);
    PMG_REQUIRE((threads + 255) / 256 <= INT_MAX, "too large");
    hipLaunchKernelGGL(pool_reduce_k, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       feats, C, seg_indices, seg_offsets, num_out, reduce, out);
    return check_launch("pool_reduce_k");
}

int pmg_sparse_upsample(const void* feats, int64_t row_bytes, const int32_t* parent, int64_t rows_out, void* out,
                        void* stream) {
    PMG_REQUIRE(feats && parent && out, "null buffer");
    PMG_REQUIRE(rows_out >= 0, "bad row count");
    PMG_REQUIRE(row_bytes > 0 && row_bytes % 16 == 0, "row_bytes must be a positive multiple of 16");
    PMG_REQUIRE(aligned16(feats) && aligned16(out), "feats and out must be 16-byte aligned");
    if (rows_out == 0) return PMG_OK;
    const int64_t threads = rows_out * (row_bytes / 16);
    PMG_REQUIRE((threads + 255) / 256 <= INT_MAX, "too large");
    hipLaunchKernelGGL(upsample_k, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const v4i*)feats, parent, rows_out, row_bytes / 16, (v4i*)out);
    return check_launch("upsample_k");
}

}  // extern "C"
