// Robust scale/shift metric fit: fit_scale_shift (moge/model/modules/prompt_stem.py:211-240) on the GPU.
//
//   w = mask; ok = sum(w) >= min_points; k = max(long(fp32(1-trim) * fp32(count)), min_points)
//   repeat iters+1 times:  closed-form weighted LS (s, t) on w (kept only if ok); unless last:
//       r = |s*z + t - target| / max(target, 1e-3) on mask, +inf elsewhere
//       thr = kthvalue(r, min(k, N));  w = mask & (r <= thr)
//
// Design. One persistent kernel per batch item; its whole grid is resident, so phases are separated by a
// device-wide barrier instead of kernel launches, and every element's (z, target, mask) lives in registers for
// the whole fit: HBM is read once. Sums are accumulated in fp64 (n*sxx - sx^2 cancels badly in fp32) in a fixed
// order (thread, wave butterfly, wave order, then block order), and every block reduces the per-block partials
// itself, so all blocks hold bit-identical (s, t) without another barrier. The threshold is the exact k-th
// smallest residual: non-negative fp32 values order like their bit patterns, so a radix select over the 32 bits
// in digits of 11, 11 and 10 bits finds it (LDS histogram per block, merged with one global atomic per non-empty
// bin, then every block scans the merged histogram). 4 barriers per trim round, 1 for the final solve.
// This replaces the reference device engine's approximate two-level histogram (MetricFit.metal:141-189).
#include <climits>

#include "pmg_common.h"
#include "pmg_internal.h"

namespace pmg {

constexpr int kFitThreads = 256;
constexpr int kFitEPT = 16;  // elements per thread held in registers
constexpr int kFitBins = 2048;

struct FitArgs {
    int mode;  // 0: (z, target, mask) arrays; 1: prompt map (logz, LiDAR, conf)
    const float* z;
    const float* tg;
    const uint8_t* mask;
    const float* logz;
    int64_t stride;
    const float* lidar;
    const float* conf;
    int H, W, dh, dw;
    int64_t N;
    int iters;
    float keep;  // fp32(1 - trim)
    int min_points;
    int b;  // batch item
    float* st;
    int32_t* info;
    uint64_t* partials;  // [nblocks][5] fp64 bit patterns
    unsigned* hist;      // [iters][3][kFitBins]
    unsigned* counter;
    int* err;
};

__device__ inline double wave_sum_f64(double v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Fixed-order block reduction of 5 doubles; result valid in thread 0.
__device__ inline void block_sum5(double (&v)[5], double (*red)[4]) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        v[k] = wave_sum_f64(v[k]);
        if (lane == 0) red[k][w] = v[k];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int k = 0; k < 5; ++k) v[k] = ((red[k][0] + red[k][1]) + red[k][2]) + red[k][3];
    }
    __syncthreads();
}

// Exclusive scan of one unsigned per thread over the block; also returns the block total.
__device__ inline unsigned block_excl_scan(unsigned v, unsigned* tmp, unsigned& total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    unsigned inc = v;
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
    }
    if (lane == 63) tmp[w] = inc;
    __syncthreads();
    unsigned before = 0;
    for (int k = 0; k < w; ++k) before += tmp[k];
    total = tmp[0] + tmp[1] + tmp[2] + tmp[3];
    __syncthreads();
    return before + inc - v;
}

__device__ inline void load_element(const FitArgs& a, int64_t i, float& z, float& tg, bool& m) {
    if (a.mode == 0) {
        const int64_t o = (int64_t)a.b * a.N + i;
        z = a.z[o];
        tg = a.tg[o];
        m = a.mask[o] != 0;
    } else {
        // v3.py:373-378 with the nearest index rule of F.interpolate.
        const int row = (int)(i / a.W), col = (int)(i - (int64_t)(i / a.W) * a.W);
        const float scy = (float)a.dh / (float)a.H, scx = (float)a.dw / (float)a.W;
        int sy = (int)__builtin_floorf((float)row * scy);
        int sx = (int)__builtin_floorf((float)col * scx);
        sy = sy < a.dh - 1 ? sy : a.dh - 1;
        sx = sx < a.dw - 1 ? sx : a.dw - 1;
        const int64_t p = ((int64_t)a.b * a.dh + sy) * a.dw + sx;
        const float d = a.lidar[p];
        const float c = fmin_(fmax_(a.conf[p] / 2.0f, 0.0f), 1.0f);
        z = exp_f32(a.logz[((int64_t)a.b * a.N + i) * a.stride]);
        tg = d;
        m = __builtin_isfinite(d) && d > 0.0f && c >= 0.999f;
    }
}

__global__ __launch_bounds__(kFitThreads) void fit_k(FitArgs a) {
    __shared__ double red[5][4];
    __shared__ unsigned lh[kFitBins];
    __shared__ unsigned tmp[4];
    __shared__ float s_sh, t_sh;
    __shared__ int64_t kk_sh;
    __shared__ int ok_sh;
    __shared__ unsigned bin_sh, below_sh;

    const unsigned nb = gridDim.x;
    const int64_t T = (int64_t)nb * kFitThreads;
    const int64_t gt = (int64_t)blockIdx.x * kFitThreads + threadIdx.x;

    float zr[kFitEPT], tr[kFitEPT];
    uint32_t mbits = 0, vbits = 0;
#pragma unroll
    for (int j = 0; j < kFitEPT; ++j) {
        const int64_t i = gt + j * T;
        zr[j] = 0.0f;
        tr[j] = 0.0f;
        if (i < a.N) {
            bool m;
            load_element(a, i, zr[j], tr[j], m);
            vbits |= 1u << j;
            mbits |= (m ? 1u : 0u) << j;
        }
    }
    uint32_t wbits = mbits;
    unsigned bar = 0;
    float s = 1.0f, t = 0.0f;
    uint32_t thr = 0;

    for (int it = 0; it <= a.iters; ++it) {
        // ---- weighted sums, fp64, fixed order
        double v[5] = {0.0, 0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int j = 0; j < kFitEPT; ++j) {
            if ((wbits >> j) & 1u) {
                const double zd = zr[j], td = tr[j];
                v[0] += 1.0;
                v[1] += zd;
                v[2] += td;
                v[3] += zd * zd;
                v[4] += zd * td;
            }
        }
        block_sum5(v, red);
        if (threadIdx.x == 0) {
#pragma unroll
            for (int k = 0; k < 5; ++k)
                __hip_atomic_store(&a.partials[blockIdx.x * 5 + k], __builtin_bit_cast(uint64_t, v[k]),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        grid_barrier(a.counter, bar++, nb, a.err);
        double g[5] = {0.0, 0.0, 0.0, 0.0, 0.0};
        for (unsigned q = threadIdx.x; q < nb; q += kFitThreads) {
#pragma unroll
            for (int k = 0; k < 5; ++k)
                g[k] += __builtin_bit_cast(double, __hip_atomic_load(&a.partials[q * 5 + k], __ATOMIC_RELAXED,
                                                                     __HIP_MEMORY_SCOPE_AGENT));
        }
        block_sum5(g, red);
        if (threadIdx.x == 0) {
            const double n = g[0], sx = g[1], sy = g[2], sxx = g[3], sxy = g[4];
            if (it == 0) {
                const int64_t count = (int64_t)n;
                ok_sh = count >= a.min_points;
                int64_t k = (int64_t)(a.keep * (float)count);
                if (k < a.min_points) k = a.min_points;
                kk_sh = k < a.N ? k : a.N;
                if (a.info && blockIdx.x == 0) {
                    a.info[5 * a.b + 0] = (int32_t)count;
                    a.info[5 * a.b + 1] = (int32_t)k;
                    a.info[5 * a.b + 2] = ok_sh;
                }
            }
            const double nn = n > 1.0 ? n : 1.0;
            const double den = nn * sxx - sx * sx;
            const double sn = den > 1e-12 ? (nn * sxy - sx * sy) / (den > 1e-12 ? den : 1e-12) : 1.0;
            const double tn = (sy - sn * sx) / nn;
            if (ok_sh) {
                s = (float)sn;
                t = (float)tn;
            }
            s_sh = s;
            t_sh = t;
        }
        __syncthreads();
        s = s_sh;
        t = t_sh;
        if (it == a.iters) break;

        // ---- relative residuals as ordered bit patterns (+inf off the mask)
        uint32_t rb[kFitEPT];
#pragma unroll
        for (int j = 0; j < kFitEPT; ++j) {
            float r = u2f(0x7f800000u);
            if ((mbits >> j) & 1u) {
                float e = s * zr[j];
                e = e + t;
                e = e - tr[j];
                r = __builtin_fabsf(e) / fmax_(tr[j], 1e-3f);
            }
            rb[j] = f2u(r);
        }

        // ---- exact k-th smallest: radix select, digits 11/11/10 bits from the top
        uint32_t prefix = 0, pmask = 0;
        unsigned rank = (unsigned)kk_sh;
#pragma unroll
        for (int pass = 0; pass < 3; ++pass) {
            const int sh = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
            const int nbins = pass == 2 ? 1024 : 2048;
            for (int q = threadIdx.x; q < nbins; q += kFitThreads) lh[q] = 0;
            __syncthreads();
#pragma unroll
            for (int j = 0; j < kFitEPT; ++j)
                if (((vbits >> j) & 1u) && (rb[j] & pmask) == prefix)
                    atomicAdd(&lh[(rb[j] >> sh) & (unsigned)(nbins - 1)], 1u);
            __syncthreads();
            unsigned* gh = a.hist + ((int64_t)it * 3 + pass) * kFitBins;
            for (int q = threadIdx.x; q < nbins; q += kFitThreads)
                if (lh[q]) atomicAdd(&gh[q], lh[q]);
            grid_barrier(a.counter, bar++, nb, a.err);
            const int per = nbins / kFitThreads;  // 8 or 4 consecutive bins per thread
            unsigned cnt[8];
            unsigned local = 0;
            for (int e = 0; e < per; ++e) {
                cnt[e] = __hip_atomic_load(&gh[threadIdx.x * per + e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                local += cnt[e];
            }
            if (threadIdx.x == 0) {
                bin_sh = 0;
                below_sh = 0;
            }
            unsigned total;
            const unsigned excl = block_excl_scan(local, tmp, total);
            if (excl < rank && rank <= excl + local) {
                unsigned cum = excl;
                for (int e = 0; e < per; ++e) {
                    if (cum + cnt[e] >= rank) {
                        bin_sh = (unsigned)(threadIdx.x * per + e);
                        below_sh = cum;
                        break;
                    }
                    cum += cnt[e];
                }
            }
            __syncthreads();
            prefix |= bin_sh << sh;
            pmask |= (unsigned)(nbins - 1) << sh;
            rank -= below_sh;
            __syncthreads();
        }
        thr = prefix;
        wbits = 0;
#pragma unroll
        for (int j = 0; j < kFitEPT; ++j)
            if (((mbits >> j) & 1u) && rb[j] <= thr) wbits |= 1u << j;
    }

    if (blockIdx.x == 0 && threadIdx.x == 0) {
        a.st[2 * a.b] = s;
        a.st[2 * a.b + 1] = t;
        if (a.info) {
            a.info[5 * a.b + 3] = (int32_t)thr;
            a.info[5 * a.b + 4] = __hip_atomic_load(a.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

static int fit_blocks(int64_t N) {
    const int64_t per_block = (int64_t)kFitThreads * kFitEPT;
    int64_t nb = (N + per_block - 1) / per_block;
    if (nb < 256) nb = 256;
    return (int)nb;
}

size_t fit_workspace_bytes(int64_t N, int iters) {
    const int nb = fit_blocks(N);
    return 256 + (size_t)nb * 5 * sizeof(uint64_t) + (size_t)(iters > 0 ? iters : 1) * 3 * kFitBins * sizeof(unsigned);
}

int launch_fit(const FitLaunch& f, hipStream_t s) {
    PMG_REQUIRE(f.N > 0 && f.N <= (int64_t)1 << 22, "N must be in [1, 2^22]");
    PMG_REQUIRE(f.iters >= 0 && f.iters <= 64, "iters must be in [0, 64]");
    PMG_REQUIRE(f.min_points >= 1, "min_points must be >= 1");
    PMG_REQUIRE(f.trim >= 0.0f && f.trim < 1.0f, "trim must be in [0, 1)");
    PMG_REQUIRE(f.workspace && f.workspace_bytes >= fit_workspace_bytes(f.N, f.iters), "workspace too small");
    const int nb = fit_blocks(f.N);
    static int max_resident = -1;
    if (max_resident < 0) {
        int per_cu = 0;
        PMG_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fit_k, kFitThreads, 0));
        max_resident = per_cu * num_cus();
    }
    PMG_REQUIRE(nb <= max_resident, "fit grid of " + std::to_string(nb) + " blocks cannot be resident (max " +
                                        std::to_string(max_resident) + ")");
    uint8_t* ws = (uint8_t*)f.workspace;
    unsigned* counter = (unsigned*)ws;
    int* err = (int*)(ws + 4);
    uint64_t* partials = (uint64_t*)(ws + 256);
    unsigned* hist = (unsigned*)(partials + (size_t)nb * 5);
    const int64_t hist_words = (int64_t)(f.iters > 0 ? f.iters : 1) * 3 * kFitBins;
    fill_u32(err, 0u, 1, s);
    for (int b = 0; b < f.B; ++b) {
        fill_u32(counter, 0u, 1, s);
        fill_u32(hist, 0u, hist_words, s);
        FitArgs a{f.mode, f.z, f.tg, f.mask, f.logz, f.stride, f.lidar, f.conf, f.H, f.W, f.dh, f.dw,
                  f.N, f.iters, (float)(1.0 - (double)f.trim), f.min_points, b, f.st, f.info,
                  partials, hist, counter, err};
        hipLaunchKernelGGL(fit_k, dim3(nb), dim3(kFitThreads), 0, s, a);
        if (int e = check_launch("fit_k")) return e;
    }
    return PMG_OK;
}

}  // namespace pmg

using namespace pmg;

extern "C" {

size_t pmg_fit_workspace_bytes(int64_t N, int iters) { return fit_workspace_bytes(N, iters); }

int pmg_fit_scale_shift(const float* z, const float* target, const uint8_t* mask, int B, int64_t N, int iters,
                        float trim, int min_points, float* st, int32_t* info, void* workspace,
                        size_t workspace_bytes, void* stream) {
    PMG_REQUIRE(z && target && mask && st, "null buffer");
    PMG_REQUIRE(B >= 1, "bad batch");
    FitLaunch f{};
    f.mode = 0;
    f.z = z;
    f.tg = target;
    f.mask = mask;
    f.B = B;
    f.N = N;
    f.iters = iters;
    f.trim = trim;
    f.min_points = min_points;
    f.st = st;
    f.info = info;
    f.workspace = workspace;
    f.workspace_bytes = workspace_bytes;
    return launch_fit(f, (hipStream_t)stream);
}

int pmg_fit_prompt(const float* logz, int64_t stride, const float* lidar, const float* conf, int B, int H, int W,
                   int dh, int dw, int iters, float trim, int min_points, float* st, int32_t* info,
                   void* workspace, size_t workspace_bytes, void* stream) {
    PMG_REQUIRE(logz && lidar && conf && st, "null buffer");
    PMG_REQUIRE(B >= 1 && H >= 1 && W >= 1 && dh >= 1 && dw >= 1 && stride >= 1, "bad shape");
    FitLaunch f{};
    f.mode = 1;
    f.logz = logz;
    f.stride = stride;
    f.lidar = lidar;
    f.conf = conf;
    f.B = B;
    f.H = H;
    f.W = W;
    f.dh = dh;
    f.dw = dw;
    f.N = (int64_t)H * W;
    f.iters = iters;
    f.trim = trim;
    f.min_points = min_points;
    f.st = st;
    f.info = info;
    f.workspace = workspace;
    f.workspace_bytes = workspace_bytes;
    return launch_fit(f, (hipStream_t)stream);
}

}  // extern "C"
