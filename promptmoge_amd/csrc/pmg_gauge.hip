// The prompt gauge: a per-frame multiplicative correction exp(poly(u, v)) fitted robustly (IRLS) to
// log(prompt / prediction) on confident prompt pixels and applied at full resolution (prompt_gauge_poly,
// moge/model/v3.py:151-183; infer's default gauge_poly = 2, v3.py:841-853).
//
//   gauge_inputs_k  one thread per LiDAR pixel: the area-pooled valid depth z_lr (the window sums of
//                   where(ok, depth, 0) and of ok, each / height / width, as F.interpolate(mode='area')), the mask
//                   conf >= 2 & lidar > 0 & z_lr > 0 and y = log(max(lidar, 1e-3)) - log(max(z_lr, 1e-3))
//   per IRLS round  gauge_sums_k (a grid of blocks per frame: fp64 partial sums of the weighted normal equations
//                   (A w)^T (A w) c = (A w)^T (y w) over the confident pixels), gauge_solve_k (one wave per frame:
//                   the partials in a fixed order, Gaussian elimination with partial pivoting; the reference runs
//                   LAPACK least squares on the same fp32 products), and, for every round but the last, the exact
//                   lower median of |y - A c| (fp32 residuals) by three radix passes over its bits (gauge_hist_k:
//                   grid-wide 2048-bin histograms of the candidates; gauge_select_k: the bucket holding the rank)
//                   and the weights min(2 sc / max(|r|, 1e-6), 1), sc = 1.4826 median + 1e-4 (gauge_weights_k)
//   gauge_apply_k   one thread per output pixel: exp of the polynomial (a sequential fp32 sum over the basis)
//
// The basis is (1, u, v) or (1, u, v, u^2, uv, v^2) on torch.linspace(-1, 1, n) grids (the scalar rule: step
// 2 / (n - 1) in fp32, start + step i for the first half, end - step (n - 1 - i) for the second). A frame with
// fewer than 200 confident pixels, or a singular / non-finite system, gets the correction 1. The frame state (valid,
// count, median search) lives in device memory, so the whole sequence runs without a host round trip.
#include <climits>

#include "pmg_common.h"

namespace pmg {

constexpr int kGaugeMinPoints = 200;
constexpr int kGaugeMaxK = 6;

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

__device__ inline float linspace_at(int i, int n) {
    if (n == 1) return -1.0f;
    const float step = 2.0f / (float)(n - 1);
    return i < n / 2 ? -1.0f + step * (float)i : 1.0f - step * (float)(n - 1 - i);
}

__device__ inline void gauge_basis(float u, float v, float (&a)[kGaugeMaxK]) {
    a[0] = 1.0f;
    a[1] = u;
    a[2] = v;
    a[3] = u * u;
    a[4] = u * v;
    a[5] = v * v;
}

__global__ __launch_bounds__(256) void gauge_inputs_k(const float* __restrict__ depth, const float* __restrict__ lidar,
                                                      const float* __restrict__ conf, int H, int W, int h, int w,
                                                      int64_t n_out, float* __restrict__ y_out,
                                                      uint8_t* __restrict__ m_out) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= n_out) return;
    const int64_t plane = (int64_t)h * w;
    const int64_t b = q / plane;
    const int rem = (int)(q - b * plane);
    const int oh = rem / w, ow = rem - oh * w;
    const int r0 = (int)(((int64_t)oh * H) / h), r1 = (int)((((int64_t)oh + 1) * H + h - 1) / h);
    const int c0 = (int)(((int64_t)ow * W) / w), c1 = (int)((((int64_t)ow + 1) * W + w - 1) / w);
    const float* db = depth + b * H * W;
    float num = 0.0f, den = 0.0f;
    for (int r = r0; r < r1; ++r)
        for (int c = c0; c < c1; ++c) {
            const float d = db[(int64_t)r * W + c];
            const bool ok = __builtin_isfinite(d) && d > 0.0f;
            num = num + (ok ? d : 0.0f);
            den = den + (ok ? 1.0f : 0.0f);
        }
    const float kh = (float)(r1 - r0), kw = (float)(c1 - c0);
    const float nump = num / kh / kw, denp = den / kh / kw;
    const float z = denp > 0.5f ? nump / fmax_(denp, 1e-6f) : 0.0f;
    const float ld = lidar[q];
    const float cf = conf ? conf[q] : 2.0f;
    y_out[q] = log_f32(fmax_(ld, 1e-3f)) - log_f32(fmax_(z, 1e-3f));
    m_out[q] = (cf >= 2.0f && ld > 0.0f && z > 0.0f) ? 1 : 0;
}

// ---- the IRLS rounds, spread over the GPU: per round a grid of blocks sums the weighted normal equations
// (fp64 partials per block), one wave per frame reduces them in a fixed order and solves; then (all but the last
// round) three radix-select passes over the residual bits (11 + 11 + 10 bits: a grid-wide histogram of the
// candidates, then one block per frame picks the bucket holding the median's rank) and the new weights.
constexpr int kGaugeBlk = 256;       // threads of the grid kernels
constexpr int kGaugeMaxBlocks = 256; // blocks per frame
constexpr int kGaugeBins = 2048;
constexpr int kGaugeVals = 28;       // 21 normal-matrix entries + 6 right-hand sides + count (K = 6; fewer for 3)

struct GaugeState {
    uint32_t prefix;  // median bits found so far
    uint32_t rank;    // rank of the median among the candidates with that prefix
    int32_t count;    // confident pixels
    int32_t valid;    // 1 while the frame has a finite solution
};

__device__ inline void gauge_range(int64_t N, int nblk, int blk, int64_t& n0, int64_t& n1) {
    n0 = N * blk / nblk;
    n1 = N * (blk + 1) / nblk;
}

template <int K>
__global__ __launch_bounds__(kGaugeBlk) void gauge_sums_k(const float* __restrict__ y_all,
                                                          const uint8_t* __restrict__ m_all,
                                                          const float* __restrict__ w_all, int h, int w, int first,
                                                          const GaugeState* __restrict__ st, int nblk,
                                                          double* __restrict__ partials) {
    constexpr int NG = K * (K + 1) / 2;
    __shared__ double s_red[kGaugeBlk / 64][kGaugeVals];
    const int b = blockIdx.y, tid = threadIdx.x;
    if (!first && !st[b].valid) return;
    const int64_t N = (int64_t)h * w, base = (int64_t)b * N;
    int64_t n0, n1;
    gauge_range(N, nblk, blockIdx.x, n0, n1);
    double G[NG + K + 1];
#pragma unroll
    for (int k = 0; k < NG + K + 1; ++k) G[k] = 0.0;
    for (int64_t n = n0 + tid; n < n1; n += kGaugeBlk) {
        if (!m_all[base + n]) continue;
        float a[kGaugeMaxK];
        const int iy = (int)(n / w), ix = (int)(n - (int64_t)iy * w);
        gauge_basis(linspace_at(ix, w), linspace_at(iy, h), a);
        const float wn = first ? 1.0f : w_all[base + n];
        float wa[K];
#pragma unroll
        for (int k = 0; k < K; ++k) wa[k] = a[k] * wn;
        const float wy = y_all[base + n] * wn;
        int e = 0;
#pragma unroll
        for (int i = 0; i < K; ++i)
#pragma unroll
            for (int j = i; j < K; ++j) G[e++] += (double)wa[i] * (double)wa[j];
#pragma unroll
        for (int i = 0; i < K; ++i) G[NG + i] += (double)wa[i] * (double)wy;
        G[NG + K] += 1.0;
    }
    const int wv = tid >> 6, lane = tid & 63;
#pragma unroll
    for (int k = 0; k < NG + K + 1; ++k) {
        double v = G[k];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        if (lane == 0) s_red[wv][k] = v;
    }
    __syncthreads();
    if (tid < NG + K + 1) {
        double v = 0.0;
        for (int q = 0; q < kGaugeBlk / 64; ++q) v += s_red[q][tid];
        partials[((int64_t)b * nblk + blockIdx.x) * kGaugeVals + tid] = v;
    }
}

// One wave per frame: the fixed-order reduction of the block partials, the count test, the solve (lane 0), and
// the set-up of the median search; it also clears the frame's histogram for the first pass.
template <int K>
__global__ __launch_bounds__(64) void gauge_solve_k(const double* __restrict__ partials, int nblk, int first,
                                                    GaugeState* __restrict__ st, float* __restrict__ coef,
                                                    uint32_t* __restrict__ hist) {
    constexpr int NG = K * (K + 1) / 2;
    __shared__ double s_v[kGaugeVals];
    const int b = blockIdx.x, lane = threadIdx.x;
    for (int i = lane; i < kGaugeBins; i += 64) hist[(int64_t)b * kGaugeBins + i] = 0u;
    if (!first && !st[b].valid) return;
    if (lane < NG + K + 1) {
        double v = 0.0;
        for (int q = 0; q < nblk; ++q) v += partials[((int64_t)b * nblk + q) * kGaugeVals + lane];
        s_v[lane] = v;
    }
    __syncthreads();
    if (lane != 0) return;
    const int count = (int)s_v[NG + K];
    bool okk = count >= kGaugeMinPoints;  // v3.py:174-175: the frame keeps the correction 1
    double A[K][K + 1];
    {
        int e = 0;
        for (int i = 0; i < K; ++i) {
            for (int j = i; j < K; ++j) {
                A[i][j] = A[j][i] = s_v[e];
                ++e;
            }
            A[i][K] = s_v[NG + i];
        }
    }
    // Gaussian elimination with partial pivoting on [G | g]
    for (int c = 0; c < K && okk; ++c) {
        int p = c;
        for (int r = c + 1; r < K; ++r)
            if (fabs(A[r][c]) > fabs(A[p][c])) p = r;
        if (!(fabs(A[p][c]) > 0.0)) {
            okk = false;
            break;
        }
        if (p != c)
            for (int k = 0; k <= K; ++k) {
                const double t = A[c][k];
                A[c][k] = A[p][k];
                A[p][k] = t;
            }
        for (int r = c + 1; r < K; ++r) {
            const double f = A[r][c] / A[c][c];
            for (int k = c; k <= K; ++k) A[r][k] -= f * A[c][k];
        }
    }
    double x[K];
    for (int c = K - 1; c >= 0 && okk; --c) {
        double s = A[c][K];
        for (int k = c + 1; k < K; ++k) s -= A[c][k] * x[k];
        x[c] = s / A[c][c];
    }
    float cf[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int k = 0; k < K && okk; ++k) {
        cf[k] = (float)x[k];
        okk = __builtin_isfinite(cf[k]);
    }
    cf[7] = okk ? 1.0f : 0.0f;
    for (int k = 0; k < 8; ++k) coef[b * 8 + k] = okk || k == 7 ? cf[k] : 0.0f;
    GaugeState g;
    g.prefix = 0u;
    g.rank = okk ? (uint32_t)((count - 1) / 2) : 0u;  // torch.median: the lower middle element
    g.count = count;
    g.valid = okk ? 1 : 0;
    st[b] = g;
}

// Radix pass `pass` (bits 31..21, 20..10, 9..0) of the median of |y - A c| over the confident pixels; pass 0 also
// computes and keeps the residual bits (fp32, terms in basis order).
template <int K>
__global__ __launch_bounds__(kGaugeBlk) void gauge_hist_k(int pass, const float* __restrict__ y_all,
                                                          const uint8_t* __restrict__ m_all, int h, int w,
                                                          const float* __restrict__ coef,
                                                          const GaugeState* __restrict__ st, int nblk,
                                                          uint32_t* __restrict__ r_all, uint32_t* __restrict__ hist) {
    __shared__ uint32_t s_h[kGaugeBins];
    const int b = blockIdx.y, tid = threadIdx.x;
    if (!st[b].valid) return;
    for (int i = tid; i < kGaugeBins; i += kGaugeBlk) s_h[i] = 0u;
    __syncthreads();
    const int64_t N = (int64_t)h * w, base = (int64_t)b * N;
    int64_t n0, n1;
    gauge_range(N, nblk, blockIdx.x, n0, n1);
    const int sh = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const uint32_t bmask = pass == 2 ? 0x3ffu : 0x7ffu;
    const uint32_t hmask = pass == 0 ? 0u : (pass == 1 ? 0xffe00000u : 0xfffffc00u);
    const uint32_t prefix = st[b].prefix;
    float c[kGaugeMaxK];
#pragma unroll
    for (int k = 0; k < kGaugeMaxK; ++k) c[k] = k < K ? coef[b * 8 + k] : 0.0f;
    for (int64_t n = n0 + tid; n < n1; n += kGaugeBlk) {
        if (!m_all[base + n]) continue;
        uint32_t v;
        if (pass == 0) {
            float a[kGaugeMaxK];
            const int iy = (int)(n / w), ix = (int)(n - (int64_t)iy * w);
            gauge_basis(linspace_at(ix, w), linspace_at(iy, h), a);
            float p = 0.0f;
#pragma unroll
            for (int k = 0; k < K; ++k) p = p + a[k] * c[k];
            v = __float_as_uint(fabsf(y_all[base + n] - p));
            r_all[base + n] = v;
        } else {
            v = r_all[base + n];
        }
        if ((v & hmask) == prefix) atomicAdd(&s_h[(v >> sh) & bmask], 1u);
    }
    __syncthreads();
    uint32_t* hg = hist + (int64_t)b * kGaugeBins;
    for (int i = tid; i < kGaugeBins; i += kGaugeBlk)
        if (s_h[i]) atomicAdd(&hg[i], s_h[i]);
}

// One block per frame: the bucket of the pass that holds the rank; clears the histogram for the next pass.
__global__ __launch_bounds__(kGaugeBlk) void gauge_select_k(int pass, GaugeState* __restrict__ st,
                                                            uint32_t* __restrict__ hist) {
    __shared__ uint32_t s_h[kGaugeBins];
    __shared__ uint32_t s_part[kGaugeBlk];
    const int b = blockIdx.x, tid = threadIdx.x;
    uint32_t* hg = hist + (int64_t)b * kGaugeBins;
    const bool valid = st[b].valid != 0;
    constexpr int PER = kGaugeBins / kGaugeBlk;  // 8 bins per thread
    uint32_t sum = 0u;
    for (int k = 0; k < PER; ++k) {
        const uint32_t v = valid ? hg[tid * PER + k] : 0u;
        s_h[tid * PER + k] = v;
        sum += v;
    }
    s_part[tid] = sum;
    __syncthreads();
    for (int i = tid; i < kGaugeBins; i += kGaugeBlk) hg[i] = 0u;
    if (!valid || tid != 0) return;
    const int sh = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const int nb = pass == 2 ? 1024 : 2048;
    uint32_t k = st[b].rank, cum = 0u;
    int t = 0;
    while (t < kGaugeBlk - 1 && cum + s_part[t] <= k) cum += s_part[t++];
    int bkt = t * PER;
    for (; bkt < nb - 1; ++bkt) {
        if (cum + s_h[bkt] > k) break;
        cum += s_h[bkt];
    }
    st[b].prefix |= (uint32_t)bkt << sh;
    st[b].rank = k - cum;
}

__global__ __launch_bounds__(kGaugeBlk) void gauge_weights_k(const uint8_t* __restrict__ m_all, int h, int w,
                                                             const GaugeState* __restrict__ st, int nblk,
                                                             const uint32_t* __restrict__ r_all,
                                                             float* __restrict__ w_all) {
    const int b = blockIdx.y, tid = threadIdx.x;
    if (!st[b].valid) return;
    const int64_t N = (int64_t)h * w, base = (int64_t)b * N;
    int64_t n0, n1;
    gauge_range(N, nblk, blockIdx.x, n0, n1);
    const float med = __uint_as_float(st[b].prefix);
    const float sc = 1.4826f * med + 1e-4f;
    for (int64_t n = n0 + tid; n < n1; n += kGaugeBlk) {
        if (!m_all[base + n]) continue;
        w_all[base + n] = fmin_((2.0f * sc) / fmax_(__uint_as_float(r_all[base + n]), 1e-6f), 1.0f);
    }
}

template <int K>
__global__ __launch_bounds__(256) void gauge_apply_k(const float* __restrict__ coef, int H, int W, int64_t n_out,
                                                     float* __restrict__ out) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= n_out) return;
    const int64_t plane = (int64_t)H * W;
    const int64_t b = q / plane;
    const int rem = (int)(q - b * plane);
    const int i = rem / W, j = rem - i * W;
    const float* c = coef + b * 8;
    if (c[7] == 0.0f) {
        out[q] = 1.0f;
        return;
    }
    float a[kGaugeMaxK];
    gauge_basis(linspace_at(j, W), linspace_at(i, H), a);
    float p = 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k) p = p + a[k] * c[k];
    out[q] = exp_f32(p);
}

}  // namespace pmg

using namespace pmg;

static int gauge_blocks(int64_t N) {
    const int64_t nb = (N + 1023) / 1024;
    return (int)(nb < 1 ? 1 : (nb > kGaugeMaxBlocks ? kGaugeMaxBlocks : nb));
}

template <int K>
static int gauge_rounds(const float* y, const uint8_t* m, int B, int h, int w, int iters, float* wt, uint32_t* rb,
                        double* partials, uint32_t* hist, GaugeState* st, float* coef, hipStream_t s) {
    const int nblk = gauge_blocks((int64_t)h * w);
    const dim3 grid((unsigned)nblk, (unsigned)B);
    for (int it = 0; it < iters; ++it) {
        const int first = it == 0;
        hipLaunchKernelGGL(gauge_sums_k<K>, grid, dim3(kGaugeBlk), 0, s, y, m, wt, h, w, first, st, nblk, partials);
        if (int e = check_launch("gauge_sums_k")) return e;
        hipLaunchKernelGGL(gauge_solve_k<K>, dim3(B), dim3(64), 0, s, partials, nblk, first, st, coef, hist);
        if (int e = check_launch("gauge_solve_k")) return e;
        if (it + 1 == iters) break;  // the last weights are never used
        for (int pass = 0; pass < 3; ++pass) {
            hipLaunchKernelGGL(gauge_hist_k<K>, grid, dim3(kGaugeBlk), 0, s, pass, y, m, h, w, coef, st, nblk, rb,
                               hist);
            if (int e = check_launch("gauge_hist_k")) return e;
            hipLaunchKernelGGL(gauge_select_k, dim3(B), dim3(kGaugeBlk), 0, s, pass, st, hist);
            if (int e = check_launch("gauge_select_k")) return e;
        }
        hipLaunchKernelGGL(gauge_weights_k, grid, dim3(kGaugeBlk), 0, s, m, h, w, st, nblk, rb, wt);
        if (int e = check_launch("gauge_weights_k")) return e;
    }
    return PMG_OK;
}

extern "C" {

size_t pmg_gauge_poly_workspace_bytes(int B, int h, int w) {
    if (B < 1 || h < 1 || w < 1) return 0;
    const size_t n = (size_t)B * h * w;
    const int nblk = gauge_blocks((int64_t)h * w);
    return align256(n * 4) + align256(n) + align256(n * 4) + align256(n * 4) +
           align256((size_t)B * nblk * kGaugeVals * sizeof(double)) + align256((size_t)B * kGaugeBins * 4) +
           align256((size_t)B * sizeof(GaugeState));
}

int pmg_gauge_poly(const float* depth, int B, int H, int W, const float* lidar, const float* conf, int h, int w,
                   int degree, int iters, float* corr, float* coef, void* workspace, size_t workspace_bytes,
                   void* stream) {
    PMG_REQUIRE(depth && lidar && corr && coef, "null buffer");
    PMG_REQUIRE(B >= 1 && H >= 1 && W >= 1 && h >= 1 && w >= 1, "bad shape");
    PMG_REQUIRE((int64_t)B * H * W < INT_MAX && (int64_t)B * h * w < INT_MAX && B <= 65535, "map too large");
    PMG_REQUIRE(degree >= 1, "degree must be >= 1");
    PMG_REQUIRE(iters >= 1 && iters <= 64, "iters must be in [1, 64]");
    PMG_REQUIRE(workspace && workspace_bytes >= pmg_gauge_poly_workspace_bytes(B, h, w), "workspace too small");
    hipStream_t s = (hipStream_t)stream;
    const int64_t n_lr = (int64_t)B * h * w, n_out = (int64_t)B * H * W;
    const int nblk = gauge_blocks((int64_t)h * w);
    uint8_t* p = (uint8_t*)workspace;
    float* y = (float*)p;
    p += align256((size_t)n_lr * 4);
    uint8_t* m = p;
    p += align256((size_t)n_lr);
    float* wt = (float*)p;
    p += align256((size_t)n_lr * 4);
    uint32_t* rb = (uint32_t*)p;
    p += align256((size_t)n_lr * 4);
    double* partials = (double*)p;
    p += align256((size_t)B * nblk * kGaugeVals * sizeof(double));
    uint32_t* hist = (uint32_t*)p;
    p += align256((size_t)B * kGaugeBins * 4);
    GaugeState* st = (GaugeState*)p;
    hipLaunchKernelGGL(gauge_inputs_k, dim3((unsigned)((n_lr + 255) / 256)), dim3(256), 0, s, depth, lidar, conf, H, W,
                       h, w, n_lr, y, m);
    if (int e = check_launch("gauge_inputs_k")) return e;
    if (degree >= 2) {
        if (int e = gauge_rounds<6>(y, m, B, h, w, iters, wt, rb, partials, hist, st, coef, s)) return e;
        hipLaunchKernelGGL(gauge_apply_k<6>, dim3((unsigned)((n_out + 255) / 256)), dim3(256), 0, s, coef, H, W, n_out,
                           corr);
    } else {
        if (int e = gauge_rounds<3>(y, m, B, h, w, iters, wt, rb, partials, hist, st, coef, s)) return e;
        hipLaunchKernelGGL(gauge_apply_k<3>, dim3((unsigned)((n_out + 255) / 256)), dim3(256), 0, s, coef, H, W, n_out,
                           corr);
    }
    return check_launch("gauge_apply_k");
}

}  // extern "C"
