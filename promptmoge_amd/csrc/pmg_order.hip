// Row order for the generic-map convolution: rows stably sorted by their 27-bit tap mask within windows of
// consecutive rows.
//
// The block-tiled convolution runs, for each chunk of 512 output rows, the taps that any row of the chunk has,
// and each wave multiplies its 16-row tiles by the weights of each tap one of its rows has. In the caller's row
// order (e.g. lexicographic coordinates of surfaces) 512 consecutive rows use ~27 of the 27 taps and 64 rows ~25,
// while a row uses ~10-13. Sorted by the whole mask, rows with one neighbourhood pattern are consecutive: a chunk
// then uses ~12 taps and a wave ~10 on the 1M-voxel surface set. The sort is stable, so the rows of one pattern
// stay in the caller's (spatial) order and a chunk's gathers stay local within its pattern. The order changes no
// result: each output row is computed from its own map row alone. Windows of the caller's order keep a window's
// gathers in a smaller part of the volume, at the price of less uniform chunks: on the 1M-voxel set the C = 64
// convolution, which walks taps per wave, runs 11 % faster with windows of 2^18 rows than with one window, while
// C = 128, which walks the chunk's tap union between block barriers, runs 6 % faster with one window (a 512-row
// chunk's union: 11.6 taps with one window, 16.0 with windows of 2^16 rows).
//
// Three steps: the masks become 64-bit keys; a stable LSD radix sort (the pool cache's, four 8-bit passes) gives
// the order; one kernel writes the tile unions of the sorted masks and the tap-major map in processing order
// (column p is the caller's row order[p]), so the convolution reads its map coalesced and only its output rows
// are scattered. The map comes from the row-major (M, 27) layout: each position reads one 108-byte row, where the
// tap-major layout would cost 27 scattered 4-byte reads.
#include <climits>

#include "pmg_common.h"
#include "pmg_internal.h"

namespace pmg {

// key = (window of row i, mask): the window index above the 27 mask bits
__global__ __launch_bounds__(256) void order_keys_k(const uint32_t* __restrict__ row_mask, int64_t M,
                                                    int64_t window, uint64_t* __restrict__ keys) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < M) keys[i] = ((uint64_t)(i / window) << 27) | (uint64_t)(row_mask[i] & 0x7ffffffu);
}

// One thread per processing position p: the permuted map column, and (every 16th thread) the tile union of
// the 16 sorted masks starting at p.
__global__ __launch_bounds__(256) void order_finish_k(const uint64_t* __restrict__ sorted_keys,
                                                      const int32_t* __restrict__ order,
                                                      const int32_t* __restrict__ nmap_rows, int64_t M,
                                                      uint32_t* __restrict__ tile_mask, int32_t* __restrict__ nmap_o) {
    const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (p >= M) return;
    if ((p & 15) == 0) {
        uint32_t m = 0;
        const int64_t e = p + 16 < M ? p + 16 : M;
        for (int64_t i = p; i < e; ++i) m |= (uint32_t)sorted_keys[i] & 0x7ffffffu;  // the mask bits of the key
        tile_mask[p >> 4] = m;
    }
    if (nmap_o) {
        const int64_t r = order[p];
#pragma unroll 9
        for (int v = 0; v < 27; ++v) nmap_o[v * M + p] = nmap_rows[r * 27 + v];
    }
}

}  // namespace pmg

using namespace pmg;

extern "C" {

size_t pmg_row_order_workspace_bytes(int64_t M) { return M < 0 ? 0 : radix_sort_workspace_bytes(M); }

int pmg_row_order(const uint32_t* row_mask, const int32_t* nmap_rows, int64_t M, int64_t window, int32_t* order,
                  uint32_t* order_tile_mask, int32_t* nmap_o, void* workspace, size_t workspace_bytes, void* stream) {
    PMG_REQUIRE(row_mask && order && order_tile_mask && workspace, "null buffer");
    PMG_REQUIRE(!nmap_o == !nmap_rows, "nmap_rows and nmap_o go together");
    PMG_REQUIRE(!nmap_o || nmap_o != nmap_rows, "the permuted map needs its own buffer");
    PMG_REQUIRE(M >= 0 && M < ((int64_t)1 << 31) && M * 27 < ((int64_t)1 << 62), "bad voxel count");
    PMG_REQUIRE((M + 2047) / 2048 * 256 <= INT_MAX, "too many voxels");
    PMG_REQUIRE(workspace_bytes >= pmg_row_order_workspace_bytes(M), "workspace too small");
    PMG_REQUIRE(window >= 0, "bad window");
    if (M == 0) return PMG_OK;
    if (window == 0 || window > M) window = M;
    const int64_t nwin = (M + window - 1) / window;
    const int bits = 27 + (nwin > 1 ? 64 - __builtin_clzll((uint64_t)(nwin - 1)) : 0);
    hipStream_t s = (hipStream_t)stream;
    RadixBufs rb = radix_bufs(workspace, M);
    const unsigned g = (unsigned)((M + 255) / 256);
    hipLaunchKernelGGL(order_keys_k, dim3(g), dim3(256), 0, s, row_mask, M, window, rb.keys[0]);
    if (int e = check_launch("order_keys_k")) return e;
    if (int e = radix_sort_pairs(rb, M, bits, order, s)) return e;
    hipLaunchKernelGGL(order_finish_k, dim3(g), dim3(256), 0, s, (const uint64_t*)rb.keys[rb.sorted],
                       (const int32_t*)order, nmap_rows, M, order_tile_mask, nmap_o);
    return check_launch("order_finish_k");
}

}  // extern "C"
