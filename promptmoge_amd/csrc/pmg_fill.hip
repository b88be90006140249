// Nearest-valid fill of a LiDAR prompt: promptmoge/model.py:61-72 (nearest_fill).
//
// The reference takes the index map of scipy.ndimage.distance_transform_edt(~valid, return_indices=True): every
// pixel receives the coordinates of the valid pixel nearest in Euclidean distance. Where several valid pixels
// are equally near, that feature transform (a separable pass along axis 0, then along axis 1) keeps the one with
// the smallest column and, within that column, the smallest row. The same result in three passes:
//
//   fill_mask_k   one 64-bit validity word per (row, 64-column strip), by wave ballot;
//   fill_col_k    per pixel, the nearest valid row of its own column (ties: the upper row), searched outward
//                 in the strip's words staged in LDS;
//   fill_row_k    per pixel, the nearest candidate over the columns of its row -- candidate c sits at
//                 (F[c], c) -- searched outward from its own column with the row's F staged in LDS, stopping
//                 once the column distance alone exceeds the best squared distance. On equal distances the
//                 left candidate (visited first at each radius) wins and the right one loses, which is the
//                 smallest-column rule.
//
// Distances are exact integers, so the result is bit-identical to the reference's for any input. The work per
// pixel is proportional to the size of the hole around it; valid pixels cost one LDS read in each search pass.
#include <climits>

#include "pmg_common.h"

namespace pmg {

constexpr int kFillMaxRows = 8192;  // one 64-bit word per row of a strip in LDS (64 KB)
constexpr int kFillMaxCols = 8192;  // one int32 per column of a row in LDS (32 KB)
constexpr int kFillColThreads = 512;
constexpr int kFillColRows = 64;  // rows per fill_col_k block (8 per wave)
constexpr int kFillRowThreads = 256;

__host__ __device__ inline int fill_strips(int w) { return (w + 63) >> 6; }
inline size_t fill_align(size_t x) { return (x + 255) & ~(size_t)255; }

// One wave per (image, row, strip): bit l of the word = pixel (i, 64*strip + l) is valid (depth > 0; NaN is not).
__global__ __launch_bounds__(256) void fill_mask_k(const float* __restrict__ depth, int h, int w,
                                                   int64_t n_words, uint64_t* __restrict__ words) {
    const int64_t wid = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wid >= n_words) return;  // whole waves leave together
    const int ns = fill_strips(w);
    const int64_t row = wid / ns;  // b*h + i
    const int j = (int)(wid - row * ns) * 64 + lane;
    const float d = j < w ? depth[row * w + j] : 0.0f;
    const uint64_t m = __ballot(d > 0.0f);
    if (lane == 0) words[wid] = m;
}

// grid (strips, ceil(h / 64), B). Lane = column of the strip; wave k of the block handles rows 8k .. 8k+7 of its
// 64-row chunk. F[b][i][j] = nearest valid row of column j (upper row on ties), -1 for an empty column.
__global__ __launch_bounds__(kFillColThreads) void fill_col_k(const uint64_t* __restrict__ words, int h, int w,
                                                              int32_t* __restrict__ F) {
    __shared__ uint64_t s_m[kFillMaxRows];
    const int s = blockIdx.x, b = blockIdx.z;
    const int ns = fill_strips(w);
    const uint64_t* src = words + (int64_t)b * h * ns + s;
    for (int i = threadIdx.x; i < h; i += kFillColThreads) s_m[i] = src[(int64_t)i * ns];
    __syncthreads();
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int j = s * 64 + lane;
    if (j >= w) return;  // no barrier follows
    const uint64_t bit = 1ull << lane;
    int32_t* out = F + (int64_t)b * h * w;
    const int i0 = blockIdx.y * kFillColRows + wv * (kFillColRows / 8);
    const int i1 = min(i0 + kFillColRows / 8, h);
    for (int i = i0; i < i1; ++i) {
        int found = -1;
        if (s_m[i] & bit) {
            found = i;
        } else {
            const int dmax = max(i, h - 1 - i);
            for (int d = 1; d <= dmax; ++d) {
                const int up = i - d, dn = i + d;
                if (up >= 0 && (s_m[up] & bit)) {
                    found = up;
                    break;
                }
                if (dn < h && (s_m[dn] & bit)) {
                    found = dn;
                    break;
                }
            }
        }
        out[(int64_t)i * w + j] = found;
    }
}

// grid (h, B): one block per image row.
__global__ __launch_bounds__(kFillRowThreads) void fill_row_k(const float* depth, const float* conf, int h, int w,
                                                              const int32_t* __restrict__ F, float* depth_out,
                                                              float* conf_out, int32_t* __restrict__ src_out) {
    // depth_out / conf_out may alias depth / conf: a pixel writes only its own entries, and every source read is
    // a valid pixel, whose value the write leaves unchanged.
    __shared__ int32_t s_f[kFillMaxCols];
    const int i = blockIdx.x, b = blockIdx.y;
    const int64_t img = (int64_t)b * h * w;
    const int64_t row = img + (int64_t)i * w;
    for (int j = threadIdx.x; j < w; j += kFillRowThreads) s_f[j] = F[row + j];
    __syncthreads();
    for (int j = threadIdx.x; j < w; j += kFillRowThreads) {
        const int f0 = s_f[j];
        int bc = -1, bd = INT_MAX;
        if (f0 >= 0) {
            bc = j;
            bd = (f0 - i) * (f0 - i);
        }
        // Squared distances are below 2 * 8192^2, so int arithmetic is exact.
        for (int r = 1; bd > 0 && r * r <= bd; ++r) {
            const int cl = j - r, cr = j + r;
            if (cl < 0 && cr >= w) break;
            if (cl >= 0) {
                const int f = s_f[cl];
                if (f >= 0) {
                    const int d2 = (f - i) * (f - i) + r * r;
                    if (d2 <= bd) {  // a tie goes to the smaller column
                        bd = d2;
                        bc = cl;
                    }
                }
            }
            if (cr < w) {
                const int f = s_f[cr];
                if (f >= 0) {
                    const int d2 = (f - i) * (f - i) + r * r;
                    if (d2 < bd) {
                        bd = d2;
                        bc = cr;
                    }
                }
            }
        }
        const bool valid = f0 == i;
        const int64_t p = row + j;
        const int src = bc >= 0 ? s_f[bc] * w + bc : -1;
        // A valid pixel is its own source (distance 0); a map with no valid pixel stays as it is.
        const float dv = bc >= 0 ? depth[img + src] : depth[p];
        if (conf_out) conf_out[p] = (valid || bc < 0) ? conf[p] : 1.0f;
        depth_out[p] = dv;
        if (src_out) src_out[p] = src;
    }
}

}  // namespace pmg

using namespace pmg;

extern "C" {

size_t pmg_nearest_fill_workspace_bytes(int B, int h, int w) {
    if (B < 1 || h < 1 || w < 1) return 0;
    const size_t words = (size_t)B * h * fill_strips(w) * sizeof(uint64_t);
    return fill_align(words) + (size_t)B * h * w * sizeof(int32_t);
}

int pmg_nearest_fill(const float* depth, const float* conf, int B, int h, int w, float* depth_out, float* conf_out,
                     int32_t* src_index, void* workspace, size_t workspace_bytes, void* stream) {
    PMG_REQUIRE(depth && depth_out && workspace, "null buffer");
    PMG_REQUIRE((conf == nullptr) == (conf_out == nullptr), "conf and conf_out go together");
    PMG_REQUIRE(B >= 1 && B <= 65535 && h >= 1 && w >= 1, "bad shape");
    PMG_REQUIRE(h <= kFillMaxRows && w <= kFillMaxCols, "nearest_fill supports maps up to 8192 x 8192");
    PMG_REQUIRE((int64_t)B * h * w <= INT_MAX, "map too large");
    PMG_REQUIRE(workspace_bytes >= pmg_nearest_fill_workspace_bytes(B, h, w), "workspace too small");
    hipStream_t s = (hipStream_t)stream;
    const int ns = fill_strips(w);
    uint64_t* words = (uint64_t*)workspace;
    int32_t* F = (int32_t*)((char*)workspace + fill_align((size_t)B * h * ns * sizeof(uint64_t)));
    const int64_t n_words = (int64_t)B * h * ns;
    fill_mask_k<<<(unsigned)((n_words + 3) / 4), 256, 0, s>>>(depth, h, w, n_words, words);
    if (int e = check_launch("fill_mask_k")) return e;
    fill_col_k<<<dim3(ns, (h + kFillColRows - 1) / kFillColRows, B), kFillColThreads, 0, s>>>(words, h, w, F);
    if (int e = check_launch("fill_col_k")) return e;
    fill_row_k<<<dim3(h, B), kFillRowThreads, 0, s>>>(depth, conf, h, w, F, depth_out, conf_out, src_index);
    return check_launch("fill_row_k");
}

}  // extern "C"
