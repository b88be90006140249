// Row order for the generic-map convolution: rows sorted by their tap mask within windows of consecutive rows.
//
// The block-tiled convolution multiplies every 16-row tile by the weights of each tap any of its rows has. In the
// caller's row order (e.g. lexicographic coordinates of surfaces) 16 consecutive rows together use ~25 of the 27
// taps while each row uses ~13. Sorting the rows of each window of 4096 consecutive rows by their tap mask -- by
// its top 16 bits (taps 11..26), which keeps rows of one surface orientation together -- brings a tile's taps down
// to ~17, while the window keeps the rows (and the neighbours they gather) spatially local. A global sort gets the
// tiles to ~13.5 taps but scatters every chunk's neighbours over the whole volume. The order changes no result:
// each output row is computed from its own map row alone.
//
// One block per window, entirely in LDS: a stable LSD radix sort with two 8-bit digits. Per digit: a histogram
// (LDS atomics; counts do not depend on order), an exclusive scan of the 256 counts, and 16 rounds of 256 keys in
// window order, where the rank of a key among equal digits comes from 9 wave ballots (the lanes whose digit
// matches on every bit) plus the counts of the lower waves -- so the sort is stable and deterministic. The keys
// keep the full mask, so the per-tile union of the sorted masks is a contiguous OR.
#include <climits>

#include "pmg_common.h"

namespace pmg {

constexpr int kOrdThreads = 256;
constexpr int kOrdRounds = 16;
constexpr int kOrdWindow = kOrdThreads * kOrdRounds;  // 4096 rows per window (one block)
constexpr int kOrdShift = 11;                         // the sort key is mask >> 11 (taps 11..26)

__global__ __launch_bounds__(kOrdThreads) void order_window_k(const uint32_t* __restrict__ row_mask, int64_t M,
                                                              int32_t* __restrict__ order,
                                                              uint32_t* __restrict__ tile_mask) {
    constexpr int NW = kOrdThreads / 64;
    __shared__ uint32_t s_key[2][kOrdWindow];
    __shared__ int32_t s_val[2][kOrdWindow];
    __shared__ uint32_t s_run[256];
    __shared__ uint32_t s_cnt[NW][256];
    __shared__ uint32_t s_tmp[256];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t base = (int64_t)blockIdx.x * kOrdWindow;
    const int n = (int)(M - base < kOrdWindow ? M - base : kOrdWindow);
    for (int i = tid; i < kOrdWindow; i += kOrdThreads) {
        s_key[0][i] = i < n ? row_mask[base + i] : 0u;
        s_val[0][i] = (int32_t)(base + i);
    }
    const uint64_t below = (1ull << lane) - 1ull;
    for (int pass = 0; pass < 2; ++pass) {
        const int src = pass & 1, dst = src ^ 1;
        const int sh = kOrdShift + 8 * pass;
        // digit counts, then their exclusive scan (Hillis-Steele over the 256 digits, one per thread)
        s_run[tid] = 0;
        __syncthreads();
        for (int i = tid; i < n; i += kOrdThreads) atomicAdd(&s_run[(s_key[src][i] >> sh) & 0xffu], 1u);
        __syncthreads();
        const uint32_t c = s_run[tid];
        s_tmp[tid] = c;
        __syncthreads();
        for (int off = 1; off < 256; off <<= 1) {
            const uint32_t add = tid >= off ? s_tmp[tid - off] : 0u;
            __syncthreads();
            s_tmp[tid] += add;
            __syncthreads();
        }
        s_run[tid] = s_tmp[tid] - c;  // start of digit tid
        __syncthreads();
        for (int k = 0; k < kOrdRounds; ++k) {
            const int i = k * kOrdThreads + tid;
            const bool ok = i < n;
            const uint32_t key = s_key[src][i];
            const int32_t val = s_val[src][i];
            const uint32_t d = ok ? (key >> sh) & 0xffu : 256u;  // 256 matches no real digit
            uint64_t peers = __ballot(ok);
#pragma unroll
            for (int b = 0; b < 9; ++b) {
                const uint64_t bb = __ballot((d >> b) & 1u);
                peers &= ((d >> b) & 1u) ? bb : ~bb;
            }
            for (int e = lane; e < 256; e += 64) s_cnt[w][e] = 0;
            __syncthreads();
            const uint32_t rank = (uint32_t)__popcll(peers & below);
            if (ok && rank == 0) s_cnt[w][d] = (uint32_t)__popcll(peers);
            __syncthreads();
            if (ok) {
                uint32_t pos = s_run[d] + rank;
                for (int q = 0; q < w; ++q) pos += s_cnt[q][d];
                s_key[dst][pos] = key;
                s_val[dst][pos] = val;
            }
            __syncthreads();
            uint32_t add = 0;
#pragma unroll
            for (int q = 0; q < NW; ++q) add += s_cnt[q][tid];
            s_run[tid] += add;
            __syncthreads();  // the next round clears s_cnt and reads s_run
        }
    }
    // after two passes the sorted window is in buffer 0
    for (int i = tid; i < n; i += kOrdThreads) order[base + i] = s_val[0][i];
    // tile unions: the window starts on a tile boundary (4096 = 256 tiles)
    for (int t = tid; t * 16 < n; t += kOrdThreads) {
        uint32_t m = 0;
        const int e = t * 16 + 16 < n ? t * 16 + 16 : n;
        for (int i = t * 16; i < e; ++i) m |= s_key[0][i];
        tile_mask[base / 16 + t] = m;
    }
}

}  // namespace pmg

using namespace pmg;

extern "C" {

size_t pmg_row_order_workspace_bytes(int64_t M) { return M < 0 ? 0 : 256; }

int pmg_row_order(const uint32_t* row_mask, int64_t M, int32_t* order, uint32_t* order_tile_mask, void* workspace,
                  size_t workspace_bytes, void* stream) {
    PMG_REQUIRE(row_mask && order && order_tile_mask, "null buffer");
    PMG_REQUIRE(M >= 0 && M < ((int64_t)1 << 31), "bad voxel count");
    (void)workspace;
    (void)workspace_bytes;
    if (M == 0) return PMG_OK;
    const int64_t nwin = (M + kOrdWindow - 1) / kOrdWindow;
    PMG_REQUIRE(nwin <= INT_MAX, "too many voxels");
    hipLaunchKernelGGL(order_window_k, dim3((unsigned)nwin), dim3(kOrdThreads), 0, (hipStream_t)stream, row_mask, M,
                       order, order_tile_mask);
    return check_launch("order_window_k");
}

}  // extern "C"
