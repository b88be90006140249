// Row order for the generic-map convolution: rows sorted by their tap mask.
//
// The block-tiled convolution stages one tap's weights per block and multiplies every row of a 512-row chunk by
// them; a tap that only some rows of the chunk have still costs its full MFMA work for the chunk. In the
// caller's row order (e.g. lexicographic coordinates of surfaces) 16 consecutive rows together use ~25 of the 27
// taps while each row uses ~13. Processing the rows sorted by their 27-bit tap mask -- here by its top 16 bits
// (taps 11..26), which keeps rows of one surface orientation together -- brings the tiles back to about the
// per-row tap count. The order changes no result: each output row is computed from its own map row alone.
//
// The sort is a stable LSD radix sort with two 8-bit digits, three kernels per digit:
//   order_hist_k     per-block digit counts (LDS atomics; counts do not depend on order);
//   order_scan_k     one block: exclusive scan of the counts in digit-major order -> each (digit, block) base;
//   order_scatter_k  per block, 16 rounds of 256 keys in input order; within a round the rank of a key among
//                    equal digits comes from 9 wave ballots (the lanes whose digit matches on every bit) and
//                    the per-wave counts of the lower waves, so the scatter is stable and deterministic.
// Keys carry the full mask through the passes, so the per-tile union of the sorted masks is a contiguous OR.
#include <climits>

#include "pmg_common.h"

namespace pmg {

constexpr int kOrdThreads = 256;
constexpr int kOrdRounds = 16;
constexpr int kOrdTile = kOrdThreads * kOrdRounds;  // keys per block
constexpr int kOrdShift = 11;                      // the sort key is mask >> 11 (taps 11..26)

__device__ inline uint32_t ord_digit(uint32_t key, int pass) { return (key >> (kOrdShift + 8 * pass)) & 0xffu; }

__global__ __launch_bounds__(kOrdThreads) void order_hist_k(const uint32_t* __restrict__ keys, int64_t M, int pass,
                                                            int nblk, uint32_t* __restrict__ hist) {
    __shared__ uint32_t h[256];
    h[threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kOrdTile;
    for (int k = 0; k < kOrdRounds; ++k) {
        const int64_t i = base + k * kOrdThreads + threadIdx.x;
        if (i < M) atomicAdd(&h[ord_digit(keys[i], pass)], 1u);
    }
    __syncthreads();
    hist[(int64_t)threadIdx.x * nblk + blockIdx.x] = h[threadIdx.x];
}

// One block of 1024 threads: exclusive scan of n = 256 * nblk counts in place.
__global__ __launch_bounds__(1024) void order_scan_k(uint32_t* hist, int n) {
    __shared__ uint32_t part[1024];
    const int per = (n + 1023) / 1024;
    const int lo = threadIdx.x * per, hi = min(lo + per, n);
    uint32_t s = 0;
    for (int i = lo; i < hi; ++i) s += hist[i];
    part[threadIdx.x] = s;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
        const uint32_t add = threadIdx.x >= off ? part[threadIdx.x - off] : 0u;
        __syncthreads();
        part[threadIdx.x] += add;
        __syncthreads();
    }
    uint32_t run = part[threadIdx.x] - s;
    for (int i = lo; i < hi; ++i) {
        const uint32_t t = hist[i];
        hist[i] = run;
        run += t;
    }
}

// vals_in == nullptr: the value of key i is i (the first pass).
__global__ __launch_bounds__(kOrdThreads) void order_scatter_k(const uint32_t* __restrict__ keys_in,
                                                               const int32_t* __restrict__ vals_in, int64_t M,
                                                               int pass, int nblk, const uint32_t* __restrict__ off,
                                                               uint32_t* __restrict__ keys_out,
                                                               int32_t* __restrict__ vals_out) {
    constexpr int NW = kOrdThreads / 64;
    __shared__ uint32_t run[256];     // keys of each digit already placed by this block
    __shared__ uint32_t cnt[NW][256]; // this round's count of each digit per wave
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    run[tid] = off[(int64_t)tid * nblk + blockIdx.x];
    const uint64_t below = (1ull << lane) - 1ull;
    const int64_t base = (int64_t)blockIdx.x * kOrdTile;
    for (int k = 0; k < kOrdRounds; ++k) {
        const int64_t i = base + k * kOrdThreads + tid;
        const bool ok = i < M;
        const uint32_t key = ok ? keys_in[i] : 0u;
        const int32_t val = ok ? (vals_in ? vals_in[i] : (int32_t)i) : 0;
        const uint32_t d = ok ? ord_digit(key, pass) : 256u;  // 256: matches no real digit
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

// order_tile_mask[t] = OR of the sorted masks t*16 .. t*16+15.
__global__ __launch_bounds__(256) void order_tiles_k(const uint32_t* __restrict__ keys, int64_t M,
                                                     uint32_t* __restrict__ tile_mask) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    uint32_t m = i < M ? keys[i] : 0u;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) m |= (uint32_t)__shfl_xor((int)m, off, 16);
    if ((i & 15) == 0 && i < M) tile_mask[i >> 4] = m;
}

static size_t ord_align(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace pmg

using namespace pmg;

extern "C" {

size_t pmg_row_order_workspace_bytes(int64_t M) {
    if (M < 0) return 0;
    const int64_t nblk = (M + kOrdTile - 1) / kOrdTile;
    return 2 * ord_align((size_t)M * 4) + ord_align((size_t)M * 4) + ord_align((size_t)256 * nblk * 4);
}

int pmg_row_order(const uint32_t* row_mask, int64_t M, int32_t* order, uint32_t* order_tile_mask, void* workspace,
                  size_t workspace_bytes, void* stream) {
    PMG_REQUIRE(row_mask && order && order_tile_mask && workspace, "null buffer");
    PMG_REQUIRE(M >= 0 && M < ((int64_t)1 << 31), "bad voxel count");
    PMG_REQUIRE(workspace_bytes >= pmg_row_order_workspace_bytes(M), "workspace too small");
    if (M == 0) return PMG_OK;
    hipStream_t s = (hipStream_t)stream;
    const int nblk = (int)((M + kOrdTile - 1) / kOrdTile);
    PMG_REQUIRE((int64_t)256 * nblk <= INT_MAX, "too many voxels");
    char* p = (char*)workspace;
    uint32_t* k1 = (uint32_t*)p;
    uint32_t* k2 = (uint32_t*)(p + ord_align((size_t)M * 4));
    int32_t* v1 = (int32_t*)(p + 2 * ord_align((size_t)M * 4));
    uint32_t* hist = (uint32_t*)(p + 3 * ord_align((size_t)M * 4));
    // pass 0: row_mask -> (k1, v1); pass 1: (k1, v1) -> (k2, order)
    for (int pass = 0; pass < 2; ++pass) {
        const uint32_t* kin = pass == 0 ? row_mask : k1;
        const int32_t* vin = pass == 0 ? nullptr : v1;
        uint32_t* kout = pass == 0 ? k1 : k2;
        int32_t* vout = pass == 0 ? v1 : order;
        hipLaunchKernelGGL(order_hist_k, dim3(nblk), dim3(kOrdThreads), 0, s, kin, M, pass, nblk, hist);
        if (int e = check_launch("order_hist_k")) return e;
        hipLaunchKernelGGL(order_scan_k, dim3(1), dim3(1024), 0, s, hist, 256 * nblk);
        if (int e = check_launch("order_scan_k")) return e;
        hipLaunchKernelGGL(order_scatter_k, dim3(nblk), dim3(kOrdThreads), 0, s, kin, vin, M, pass, nblk,
                           (const uint32_t*)hist, kout, vout);
        if (int e = check_launch("order_scatter_k")) return e;
    }
    hipLaunchKernelGGL(order_tiles_k, dim3((unsigned)((M + 255) / 256)), dim3(256), 0, s, (const uint32_t*)k2, M,
                       order_tile_mask);
    return check_launch("order_tiles_k");
}

}  // extern "C"
