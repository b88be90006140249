// The prompt gauge: a per-frame multiplicative correction exp(poly(u, v)) fitted robustly (IRLS) to
// log(prompt / prediction) on confident prompt pixels and applied at full resolution (prompt_gauge_poly,
// moge/model/v3.py:151-183; infer's default gauge_poly = 2, v3.py:841-853).
//
//   gauge_inputs_k  one thread per LiDAR pixel: the area-pooled valid depth z_lr (the window sums of
//                   where(ok, depth, 0) and of ok, each / height / width, as F.interpolate(mode='area')), the mask
//                   conf >= 2 & lidar > 0 & z_lr > 0 and y = log(max(lidar, 1e-3)) - log(max(z_lr, 1e-3))
//   gauge_fit_k     one 1024-thread block per frame runs the iterations: the weighted normal equations
//                   (A w)^T (A w) c = (A w)^T (y w) summed in fp64 and solved by Gaussian elimination with partial
//                   pivoting (the reference: LAPACK least squares on the same fp32 products), the residuals
//                   r = y - A c in fp32, their exact lower median by a 4-pass radix select on the float bits (LDS
//                   histograms), and the weights min(2 sc / max(|r|, 1e-6), 1), sc = 1.4826 median + 1e-4
//   gauge_apply_k   one thread per output pixel: exp of the polynomial (a sequential fp32 sum over the basis)
//
// The basis is (1, u, v) or (1, u, v, u^2, uv, v^2) on torch.linspace(-1, 1, n) grids (the scalar rule: step
// 2 / (n - 1) in fp32, start + step i for the first half, end - step (n - 1 - i) for the second). A frame with
// fewer than 200 confident pixels, or a non-finite solution, gets the correction 1. The fit is latency-bound work
// on one CU per frame: the LiDAR map is at most a few hundred thousand pixels and the loop runs 3 times.
#include <climits>

#include "pmg_common.h"

namespace pmg {

constexpr int kGaugeThreads = 1024;
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

// Sum of a double over the block (all threads get it); `red` holds one slot per wave.
__device__ inline double block_sum_f64(double v, double* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();  // `red` is free
    if (lane == 0) red[wv] = v;
    __syncthreads();
    double s = 0.0;
    for (int k = 0; k < kGaugeThreads / 64; ++k) s += red[k];  // fixed order: identical in every thread
    return s;
}

template <int K>
__global__ __launch_bounds__(kGaugeThreads) void gauge_fit_k(const float* __restrict__ y_all,
                                                             const uint8_t* __restrict__ m_all, int h, int w,
                                                             int iters, float* __restrict__ w_all,
                                                             uint32_t* __restrict__ r_all, float* __restrict__ coef_out) {
    constexpr int NG = K * (K + 1) / 2;  // normal-matrix entries (upper triangle)
    __shared__ double s_red[kGaugeThreads / 64];
    __shared__ double s_sys[K][K + 1];
    __shared__ float s_coef[K];
    __shared__ int s_state;  // 1: valid solution
    __shared__ uint32_t s_hist[256];
    __shared__ uint32_t s_sel[2];  // radix select: prefix, rank

    const int tid = threadIdx.x;
    const int64_t N = (int64_t)h * w;
    const int64_t base = (int64_t)blockIdx.x * N;
    const float* y = y_all + base;
    const uint8_t* m = m_all + base;
    float* wt = w_all + base;
    uint32_t* rb = r_all + base;

    auto basis_at = [&](int64_t n, float (&a)[kGaugeMaxK]) {
        const int iy = (int)(n / w), ix = (int)(n - (int64_t)iy * w);
        gauge_basis(linspace_at(ix, w), linspace_at(iy, h), a);
    };

    int count = 0;
    for (int it = 0; it < iters; ++it) {
        // normal equations of lstsq(A * wgt[:, None], y * wgt) (v3.py:178), fp64 sums of the fp32 products
        double G[NG], g[K];
#pragma unroll
        for (int k = 0; k < NG; ++k) G[k] = 0.0;
#pragma unroll
        for (int k = 0; k < K; ++k) g[k] = 0.0;
        int cnt = 0;
        for (int64_t n = tid; n < N; n += kGaugeThreads) {
            if (!m[n]) continue;
            float a[kGaugeMaxK];
            basis_at(n, a);
            const float wn = it == 0 ? 1.0f : wt[n];
            float wa[K];
#pragma unroll
            for (int k = 0; k < K; ++k) wa[k] = a[k] * wn;
            const float wy = y[n] * wn;
            int e = 0;
#pragma unroll
            for (int i = 0; i < K; ++i) {
#pragma unroll
                for (int j = i; j < K; ++j) G[e++] += (double)wa[i] * (double)wa[j];
                g[i] += (double)wa[i] * (double)wy;
            }
            ++cnt;
        }
        if (it == 0) count = (int)block_sum_f64((double)cnt, s_red);
        if (count < kGaugeMinPoints) {  // v3.py:174-175: the frame keeps the correction 1
            if (tid == 0) s_state = 0;
            break;
        }
        {
            int e = 0;
#pragma unroll
            for (int i = 0; i < K; ++i) {
#pragma unroll
                for (int j = i; j < K; ++j) {
                    const double v = block_sum_f64(G[e++], s_red);
                    if (tid == 0) s_sys[i][j] = s_sys[j][i] = v;
                }
                const double v = block_sum_f64(g[i], s_red);
                if (tid == 0) s_sys[i][K] = v;
            }
        }
        if (tid == 0) {
            // Gaussian elimination with partial pivoting on [G | g]
            bool okk = true;
            for (int c = 0; c < K && okk; ++c) {
                int p = c;
                for (int r = c + 1; r < K; ++r)
                    if (fabs(s_sys[r][c]) > fabs(s_sys[p][c])) p = r;
                if (!(fabs(s_sys[p][c]) > 0.0)) {
                    okk = false;
                    break;
                }
                if (p != c)
                    for (int k = 0; k <= K; ++k) {
                        const double t = s_sys[c][k];
                        s_sys[c][k] = s_sys[p][k];
                        s_sys[p][k] = t;
                    }
                for (int r = c + 1; r < K; ++r) {
                    const double f = s_sys[r][c] / s_sys[c][c];
                    for (int k = c; k <= K; ++k) s_sys[r][k] -= f * s_sys[c][k];
                }
            }
            double x[K];
            for (int c = K - 1; c >= 0 && okk; --c) {
                double s = s_sys[c][K];
                for (int k = c + 1; k < K; ++k) s -= s_sys[c][k] * x[k];
                x[c] = s / s_sys[c][c];
            }
            for (int k = 0; k < K && okk; ++k) {
                s_coef[k] = (float)x[k];
                okk = __builtin_isfinite(s_coef[k]);
            }
            s_state = okk ? 1 : 0;
        }
        __syncthreads();
        if (!s_state || it + 1 == iters) break;  // the last weights are never used

        // residuals |y - A c| (fp32, terms in basis order), then their lower median over the masked pixels
        for (int64_t n = tid; n < N; n += kGaugeThreads) {
            if (!m[n]) continue;
            float a[kGaugeMaxK];
            basis_at(n, a);
            float p = 0.0f;
#pragma unroll
            for (int k = 0; k < K; ++k) p = p + a[k] * s_coef[k];
            rb[n] = __float_as_uint(fabsf(y[n] - p));
        }
        if (tid == 0) {
            s_sel[0] = 0u;
            s_sel[1] = (uint32_t)((count - 1) / 2);  // torch.median: the lower middle element
        }
        for (int pass = 0; pass < 4; ++pass) {
            const int sh = 24 - 8 * pass;
            const uint32_t hmask = pass == 0 ? 0u : (0xffffffffu << (sh + 8));
            if (tid < 256) s_hist[tid] = 0u;
            __syncthreads();
            const uint32_t prefix = s_sel[0];
            for (int64_t n = tid; n < N; n += kGaugeThreads) {
                if (!m[n]) continue;
                const uint32_t v = rb[n];
                if ((v & hmask) == prefix) atomicAdd(&s_hist[(v >> sh) & 0xffu], 1u);
            }
            __syncthreads();
            if (tid == 0) {
                uint32_t k = s_sel[1], cum = 0u;
                int bkt = 0;
                for (; bkt < 255; ++bkt) {
                    if (cum + s_hist[bkt] > k) break;
                    cum += s_hist[bkt];
                }
                s_sel[0] = prefix | ((uint32_t)bkt << sh);
                s_sel[1] = k - cum;
            }
            __syncthreads();
        }
        const float med = __uint_as_float(s_sel[0]);
        const float sc = 1.4826f * med + 1e-4f;
        for (int64_t n = tid; n < N; n += kGaugeThreads) {
            if (!m[n]) continue;
            wt[n] = fmin_((2.0f * sc) / fmax_(__uint_as_float(rb[n]), 1e-6f), 1.0f);
        }
        __syncthreads();
    }
    __syncthreads();
    if (tid < 8) {
        float v = 0.0f;
        if (tid < K) v = s_state ? s_coef[tid] : 0.0f;
        if (tid == 7) v = s_state ? 1.0f : 0.0f;
        coef_out[blockIdx.x * 8 + tid] = v;
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

extern "C" {

size_t pmg_gauge_poly_workspace_bytes(int B, int h, int w) {
    if (B < 1 || h < 1 || w < 1) return 0;
    const size_t n = (size_t)B * h * w;
    return align256(n * 4) + align256(n) + align256(n * 4) + align256(n * 4);
}

int pmg_gauge_poly(const float* depth, int B, int H, int W, const float* lidar, const float* conf, int h, int w,
                   int degree, int iters, float* corr, float* coef, void* workspace, size_t workspace_bytes,
                   void* stream) {
    PMG_REQUIRE(depth && lidar && corr && coef, "null buffer");
    PMG_REQUIRE(B >= 1 && H >= 1 && W >= 1 && h >= 1 && w >= 1, "bad shape");
    PMG_REQUIRE((int64_t)B * H * W < INT_MAX && (int64_t)B * h * w < INT_MAX, "map too large");
    PMG_REQUIRE(degree >= 1, "degree must be >= 1");
    PMG_REQUIRE(iters >= 1 && iters <= 64, "iters must be in [1, 64]");
    PMG_REQUIRE(workspace && workspace_bytes >= pmg_gauge_poly_workspace_bytes(B, h, w), "workspace too small");
    hipStream_t s = (hipStream_t)stream;
    const int64_t n_lr = (int64_t)B * h * w, n_out = (int64_t)B * H * W;
    uint8_t* p = (uint8_t*)workspace;
    float* y = (float*)p;
    p += align256((size_t)n_lr * 4);
    uint8_t* m = p;
    p += align256((size_t)n_lr);
    float* wt = (float*)p;
    p += align256((size_t)n_lr * 4);
    uint32_t* rb = (uint32_t*)p;
    hipLaunchKernelGGL(gauge_inputs_k, dim3((unsigned)((n_lr + 255) / 256)), dim3(256), 0, s, depth, lidar, conf, H, W,
                       h, w, n_lr, y, m);
    if (int e = check_launch("gauge_inputs_k")) return e;
    if (degree >= 2) {
        hipLaunchKernelGGL(gauge_fit_k<6>, dim3(B), dim3(kGaugeThreads), 0, s, y, m, h, w, iters, wt, rb, coef);
    } else {
        hipLaunchKernelGGL(gauge_fit_k<3>, dim3(B), dim3(kGaugeThreads), 0, s, y, m, h, w, iters, wt, rb, coef);
    }
    if (int e = check_launch("gauge_fit_k")) return e;
    if (degree >= 2) {
        hipLaunchKernelGGL(gauge_apply_k<6>, dim3((unsigned)((n_out + 255) / 256)), dim3(256), 0, s, coef, H, W, n_out,
                           corr);
    } else {
        hipLaunchKernelGGL(gauge_apply_k<3>, dim3((unsigned)((n_out + 255) / 256)), dim3(256), 0, s, coef, H, W, n_out,
                           corr);
    }
    return check_launch("gauge_apply_k");
}

}  // extern "C"
