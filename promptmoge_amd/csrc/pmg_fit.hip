// Robust scale/shift metric fit: fit_scale_shift (moge/model/modules/prompt_stem.py:211-240) on the GPU.
//
//   w = mask; ok = sum(w) >= min_points; k = max(long(fp32(1-trim) * fp32(count)), min_points)
//   repeat iters+1 times:  closed-form weighted LS (s, t) on w (kept only if ok); unless last:
//       r = |s*z + t - target| / max(target, 1e-3) on mask, +inf elsewhere
//       thr = kthvalue(r, min(k, N));  w = mask & (r <= thr)
//
// Design. One persistent kernel per batch item with few, fat blocks (256 threads x 16, 24 or 32 elements by the
// size, held in registers for the whole fit, so HBM is read once): a device-wide barrier costs more the more blocks
// arrive, and a trim round is latency-bound, not bandwidth-bound. Phases are separated by a device-wide barrier of
// per-block flags (fit_barrier). Sums are accumulated in fp64
// (n*sxx - sx^2 cancels badly in fp32) in a fixed order, and every block reduces the published per-block partials
// itself, so all blocks hold bit-identical (s, t) and take identical branches.
//
// The threshold is the exact k-th smallest residual; non-negative fp32 values order like their bit patterns ("keys").
// A trim round costs ONE barrier when the threshold stays inside a bracket [lo, hi] predicted from the previous
// rounds (along the last move's direction half of it, against it a quarter, plus a margin of ~32 expected
// candidates): each block publishes how many of its residuals fall below lo, its fp64 sums over those (they are in
// the new weight set whatever the exact threshold), and its residuals inside the bracket ("candidates", with z and
// target). After the barrier every block loads all candidates into LDS, selects the exact k-th among them (each
// thread ranks one candidate when there are at most 96, else an LDS radix select), and adds the candidates at or
// below it to the sums -- the next (s, t) without a second barrier. When the predicted bracket would hold more than
// ~1500 candidates (large moves), a histogram pass over a window of twice its range goes first (2048 bins of a
// power-of-two width, LDS histogram per block, merged by atomics), and the stage runs on the bin that holds the
// k-th; a bracket that misses is followed by such a window on the side that holds the k-th, and round 1 takes a
// window over 16 octaves around round 0's threshold. Round 0 (no threshold yet), and a window that misses, run
// radix passes over the whole key range (bins of 2^21 keys, then 2^10 within the first bin, then single keys, each
// only while the bin holds more than 2048 keys); when one key value holds the k-th and more than kCandCap
// elements, it is the threshold and the sums take one more barrier.
// The stage checks that its bracket holds the k-th, so a prediction can cost time but never change a result.
//
// Fixed point: once a round reproduces the previous round's (s, t) bit for bit, every later round would repeat
// it exactly, so the loop stops there with the bit-identical result (on the synthetic scenes after 3 rounds).
// This replaces the reference device engine's approximate two-level histogram (MetricFit.metal:141-189).
//
// Workspace: zero-filled once before its first use; the kernel leaves it reusable (the barrier flags and their
// epoch only grow, histograms are cleared at the start of every launch, everything else is overwritten before it is
// read). A bounded wait that expires (the grid was not co-resident, e.g. another stream held CUs) sets the launch's
// error flag; the launch then completes without waiting, the last block to finish reports the flag in info, writes
// (s, t) = NaN, counts the failure in a sticky word (read by pmg_refiner_check) and returns the barrier state to its
// initial zeros, so the next launch on the workspace starts clean.
#include <climits>
#include <mutex>

#include "pmg_common.h"
#include "pmg_internal.h"

namespace pmg {

constexpr int kFitThreads = 256;
constexpr int kFitWaves = kFitThreads / 64;
constexpr int kFitEPTMax = 32;                         // elements per thread, in registers (16 or 32)
constexpr int kFitPerBlockMax = kFitThreads * kFitEPTMax;  // 8192
constexpr int kFitMaxBlocks = kFitThreads;             // N <= 2^21
constexpr int kFitBins = 2048;
constexpr int kFitHistWords = kFitBins + 64;           // one global histogram: the bins, then 16 below-window counts
constexpr int kFitHistSlots = 6;                       // histogram passes a round can take (window 3 + radix 3)
constexpr int kCandCap = 32768;                        // candidates every block holds in LDS (128 KiB)
constexpr unsigned kStageMax = 2048;                   // a pass bin with more elements is split by another pass
constexpr double kBracketMax = 1536.0;                 // expected candidates above which a window pass goes first
constexpr uint32_t kInvalid = 0xffffffffu;             // residual key of a padding slot: above every residual
constexpr int kFitTraceRounds = 64;
constexpr size_t kFitHeader = 4096;                    // barrier, error flag, trace, completion count
constexpr size_t kFitErrOffset = 64;                   // the launch's error flag
constexpr size_t kFitDoneOffset = 3904;                // finished blocks (after the trace, which ends below 3800)
static_assert(kFitErrSeenOffset == 3968, "pmg_internal.h names the sticky failure count's offset");

struct FitWs {
    unsigned* bar;        // [2]: the synchronisation epoch (the last flag value of the previous launch)
    unsigned* flags;      // [kFitMaxBlocks][16]: each block's arrival count, one 64-byte line per block
    int* err;
    uint32_t* trace;      // block 0's record: per round the selection path | candidates << 4 and the wall clock
                          // (100 MHz) at its end, per round the threshold bits; launch and first-solve times
    unsigned* done;       // blocks of the current launch that have finished (the last one resets it to 0)
    unsigned* err_seen;   // launches whose bounded wait expired since the owner last cleared it (sticky)
    uint64_t* partials;   // [2][kFitMaxBlocks][5] fp64 bit patterns
    unsigned* hist;       // [iters][kFitHistSlots][kFitHistWords]
    uint32_t* c_key;      // [2][nb][elements per block]: residual bits | mask << 31
    float* c_z;           // [2][nb][elements per block]
    float* c_t;           // [2][nb][elements per block]
};

struct FitArgs {
    int mode;  // 0: (z, target, mask) arrays; 1: prompt map (logz, LiDAR, conf); 2: final fit, LiDAR at the map's size
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
    unsigned spin_limit;  // polls of one barrier wait before it gives up
    int plan_debug;       // test hook: 0, or a deliberately wrong round plan (see pmg_debug_fit_plan)
    FitWs ws;
};

// Device-wide barrier for a fully resident grid, by per-block flags: block b's thread 0 publishes (release, agent
// scope) the barrier's sequence number, with a 32-bit payload, in its own flag line; thread t < nb waits (bounded)
// until block t's flag has reached it, then acquires, and returns block t's payload (0 in other threads). Global
// writes before it are visible after it. Flag values only grow within a launch and across launches (the epoch in
// bar[2]), so a block that is already one barrier ahead still satisfies a late waiter; the flag of an even barrier
// and that of an odd one are separate 64-bit words of the line (sequence number low, payload high, one atomic
// store), and every data buffer exchanged across a barrier is double-buffered, so that block cannot overwrite what
// the late waiter is about to read (a block cannot get two barriers ahead). Half the cost of a central arrival
// counter (no serialised read-modify-write, and every waiter polls one line in parallel with the others); the
// payload carries a stage's candidate counts, which saves the read of them after the barrier.
__device__ inline unsigned fit_barrier(const FitWs& ws, unsigned nb, unsigned want, unsigned spin_limit,
                                       unsigned payload = 0u) {
    __syncthreads();
    uint64_t* const f64 = (uint64_t*)ws.flags;  // 8 words per block's 64-byte line: [0] even barriers, [1] odd
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __hip_atomic_store(&f64[blockIdx.x * 8 + (want & 1u)], ((uint64_t)payload << 32) | want, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    unsigned got = 0;
    if (threadIdx.x < nb && __hip_atomic_load(ws.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0) {
        unsigned spins = 0;
        for (;;) {
            const uint64_t v =
                __hip_atomic_load(&f64[threadIdx.x * 8 + (want & 1u)], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((int)((unsigned)v - want) >= 0) {
                got = (unsigned)(v >> 32);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            if (++spins > spin_limit) {
                __hip_atomic_store(ws.err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    return got;
}

// Fixed-order block reduction of 5 doubles (DPP wave scans, then waves in order); result in every thread.
__device__ inline void block_sum5(double (&v)[5], double (*red)[kFitWaves]) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        v[k] = wave_incl_scan_f64(v[k]);
        if (lane == 63) red[k][w] = v[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        double s = red[k][0];
        for (int q = 1; q < kFitWaves; ++q) s += red[k][q];
        v[k] = s;
    }
    __syncthreads();
}

// Exclusive scan of one unsigned per thread over the block; also returns the block total.
__device__ inline unsigned block_excl_scan(unsigned v, unsigned* tmp, unsigned& total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const unsigned inc = wave_incl_scan_u32(v);
    if (lane == 63) tmp[w] = inc;
    __syncthreads();
    unsigned before = 0;
    total = 0;
    for (int k = 0; k < kFitWaves; ++k) {
        before += k < w ? tmp[k] : 0u;
        total += tmp[k];
    }
    __syncthreads();
    return before + inc - v;
}

// Two exclusive scans in one pass (returns a's exclusive prefix; totals of a and b).
__device__ inline unsigned block_excl_scan2(unsigned a, unsigned b, uint2* tmp, unsigned& ta, unsigned& tb) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const unsigned ia = wave_incl_scan_u32(a), ib = wave_incl_scan_u32(b);
    if (lane == 63) tmp[w] = make_uint2(ia, ib);
    __syncthreads();
    unsigned before = 0;
    ta = 0;
    tb = 0;
    for (int k = 0; k < kFitWaves; ++k) {
        const uint2 q = tmp[k];
        before += k < w ? q.x : 0u;
        ta += q.x;
        tb += q.y;
    }
    __syncthreads();
    return before + ia - a;
}

// Phase timestamps of block 0 (100 MHz wall clock) into the workspace header, for profiling the selection phases;
// compiled in with -DPMG_FIT_PHASE_TRACE.
#ifdef PMG_FIT_PHASE_TRACE
#define FIT_MARK(k)                                                                                      \
    do {                                                                                                 \
        if (b == 0 && tid == 0 && it < 32) ws.trace[256 + it * 8 + (k)] = (uint32_t)wall_clock64();     \
    } while (0)
#define FIT_MARK0(k)                                                                                     \
    do {                                                                                                 \
        if (b == 0 && tid == 0) ws.trace[900 + (k)] = (uint32_t)wall_clock64();                          \
    } while (0)
#else
#define FIT_MARK(k) \
    do {            \
    } while (0)
#define FIT_MARK0(k) \
    do {             \
    } while (0)
#endif
struct FitShared {
    unsigned hist[kFitBins];
    alignas(16) uint32_t cand[kCandCap];
    unsigned off[kFitMaxBlocks + 1];
    double red[5][kFitWaves];
    unsigned tmp[kFitWaves];
    uint2 tmp2[kFitWaves];
    float s, t;
    long long kk;
    int ok;
    unsigned bin, below;
    unsigned bincnt, hbelow;  // elements in the found bin; this block's keys below a pass window
    int found;                // find_bin found the rank in the histogram
    unsigned total_below, total_cand;
    uint32_t blo_last, bhi_last;  // bracket of the last stage
    int last;                     // this block is the launch's last one to finish
};

// Finds, in a 2048-bin histogram whose bins follow `base` smaller elements, the bin holding the rank-th element
// (1-based); sets sh.bin, sh.below (the count before it, base included), sh.bincnt (the bin's count) and sh.found
// (0 when the rank-th element lies below the bins or above them). The bins are read through `load` and base
// through `load_base`, all in one round trip.
template <class Load, class LoadBase>
__device__ inline void find_bin(FitShared& sh, unsigned rank, Load load, LoadBase load_base) {
    constexpr int per = kFitBins / kFitThreads;  // 8 consecutive bins per thread
    unsigned cnt[per];
    unsigned local = 0;
    const unsigned base = load_base();
#pragma unroll
    for (int e = 0; e < per; ++e) {
        cnt[e] = load(threadIdx.x * per + e);
        local += cnt[e];
    }
    if (threadIdx.x == 0) {
        sh.bin = 0;
        sh.below = 0;
        sh.bincnt = 0;
        sh.found = 0;
    }
    unsigned total;
    const unsigned excl = block_excl_scan(local, sh.tmp, total) + base;
    if (excl < rank && rank <= excl + local) {
        unsigned cum = excl;
#pragma unroll
        for (int e = 0; e < per; ++e) {
            if (cum + cnt[e] >= rank) {
                sh.bin = (unsigned)(threadIdx.x * per + e);
                sh.below = cum;
                sh.bincnt = cnt[e];
                sh.found = 1;
                break;
            }
            cum += cnt[e];
        }
    }
    __syncthreads();
}

template <int kFitEPT>
__global__ __launch_bounds__(kFitThreads) void fit_k(FitArgs a) {
    constexpr int kFitPerBlock = kFitThreads * kFitEPT;
    static_assert(kFitEPT <= 32, "element masks are 32-bit");
    __shared__ FitShared sh;
    const int nb = (int)gridDim.x, b = (int)blockIdx.x, tid = (int)threadIdx.x;
    const FitWs& ws = a.ws;
    const int64_t cap_words = (int64_t)nb * kFitPerBlock;
    // barrier sequence numbers continue from the previous launch's last one (every block performs the same
    // barriers; block 0 advances the epoch when it is done, after every block has read it here)
    unsigned sync_seq = __hip_atomic_load(&ws.bar[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    if (b == 0 && tid == 0) ws.trace[2 * kFitTraceRounds + 1] = (uint32_t)wall_clock64();  // launch start
    // clear this launch's global histograms; the first barrier orders this before any use
    {
        const int64_t words = (int64_t)(a.iters > 0 ? a.iters : 1) * kFitHistSlots * kFitHistWords;
        for (int64_t q = (int64_t)b * kFitThreads + tid; q < words; q += (int64_t)nb * kFitThreads) ws.hist[q] = 0u;
    }

    // ---- elements into registers: every load of the thread is issued before any is used
    float zr[kFitEPT], tr[kFitEPT];
    uint32_t mbits = 0, vbits = 0;
    {
        const uint32_t i0 = (uint32_t)b * kFitPerBlock + tid;  // N <= 2^21
#pragma unroll
        for (int j = 0; j < kFitEPT; ++j)
            if ((int64_t)i0 + j * kFitThreads < a.N) vbits |= 1u << j;
        // Loads are unconditional (padding slots read the last element) so that none sits under a branch: a
        // branch would make the compiler wait for each element's load before the next one is issued.
        const int64_t last = a.N - 1;
        if (a.mode == 0) {
            uint8_t mk[kFitEPT];
            const int64_t o0 = (int64_t)a.b * a.N;
#pragma unroll
            for (int j = 0; j < kFitEPT; ++j) {
                int64_t i = (int64_t)i0 + j * kFitThreads;
                i = i < last ? i : last;
                zr[j] = a.z[o0 + i];
                tr[j] = a.tg[o0 + i];
                mk[j] = a.mask[o0 + i];
            }
#pragma unroll
            for (int j = 0; j < kFitEPT; ++j) mbits |= ((vbits >> j) & (mk[j] != 0 ? 1u : 0u)) << j;
        } else if (a.mode == 2) {
            // the final fit on a LiDAR map of the depth map's own size (v3.py:768-775): every area window is one
            // pixel, so the pooled depth is exp(logz) itself (0 + z and z / 1 / 1 are exact) and the mask is
            // conf >= 2 & lidar > 0 & z > 0 (& mask_binary), as final_inputs_k forms them for larger windows
            const int64_t o0 = (int64_t)a.b * a.N;
            float lc[kFitEPT];
            uint8_t mb[kFitEPT];
#pragma unroll
            for (int j = 0; j < kFitEPT; ++j) {
                int64_t i = (int64_t)i0 + j * kFitThreads;
                i = i < last ? i : last;
                zr[j] = a.logz[(o0 + i) * a.stride];
                tr[j] = a.lidar[o0 + i];
                lc[j] = a.conf[o0 + i];
                mb[j] = a.mask ? a.mask[o0 + i] : (uint8_t)1;
            }
#pragma unroll
            for (int j = 0; j < kFitEPT; ++j) {
                zr[j] = exp_f32(zr[j]);
                const bool m = ((vbits >> j) & 1u) && lc[j] >= 2.0f && tr[j] > 0.0f && zr[j] > 0.0f && mb[j] != 0;
                mbits |= (m ? 1u : 0u) << j;
            }
        } else {
            // v3.py:373-378: z = exp(logz); nearest LiDAR sample (F.interpolate's index rule); mask = valid & c >= 0.999
            const uint32_t W = (uint32_t)a.W;
            const float scy = (float)a.dh / (float)a.H, scx = (float)a.dw / (float)a.W;
            float lc[kFitEPT];
#pragma unroll
            for (int j = 0; j < kFitEPT; ++j) {
                int64_t i = (int64_t)i0 + j * kFitThreads;
                i = i < last ? i : last;
                const uint32_t ij = (uint32_t)i;
                const uint32_t row = ij / W, col = ij - row * W;  // branch-free 32-bit division
                int sy = (int)__builtin_floorf((float)row * scy);
                int sx = (int)__builtin_floorf((float)col * scx);
                sy = sy < a.dh - 1 ? sy : a.dh - 1;
                sx = sx < a.dw - 1 ? sx : a.dw - 1;
                const int64_t p = ((int64_t)a.b * a.dh + sy) * a.dw + sx;
                zr[j] = a.logz[((int64_t)a.b * a.N + i) * a.stride];
                tr[j] = a.lidar[p];
                lc[j] = a.conf[p];
            }
#pragma unroll
            for (int j = 0; j < kFitEPT; ++j) {
                const float d = tr[j];
                const float c = fmin_(fmax_(lc[j] / 2.0f, 0.0f), 1.0f);
                zr[j] = exp_f32(zr[j]);
                const bool m = ((vbits >> j) & 1u) && __builtin_isfinite(d) && d > 0.0f && c >= 0.999f;
                mbits |= (m ? 1u : 0u) << j;
            }
        }
#pragma unroll
        for (int j = 0; j < kFitEPT; ++j) {  // padding slots hold zeros
            zr[j] = ((vbits >> j) & 1u) ? zr[j] : 0.0f;
            tr[j] = ((vbits >> j) & 1u) ? tr[j] : 0.0f;
        }
    }

    int stage = 0;  // publish buffers alternate between consecutive publishes
    // Publishes this block's fp64 sums into buffer `stage & 1` (a bracket stage's counts ride on its barrier).
    auto publish = [&](double (&v)[5]) {
        block_sum5(v, sh.red);
        if (tid == 0) {
            uint64_t* p = ws.partials + ((size_t)(stage & 1) * kFitMaxBlocks + b) * 5;
#pragma unroll
            for (int k = 0; k < 5; ++k) p[k] = __builtin_bit_cast(uint64_t, v[k]);
        }
    };
    // Sum of all blocks' published partials of buffer `stage & 1`, in block order, in every thread.
    auto gather_partials = [&](double (&g)[5]) {
#pragma unroll
        for (int k = 0; k < 5; ++k) g[k] = 0.0;
        if (tid < nb) {
            const uint64_t* p = ws.partials + ((size_t)(stage & 1) * kFitMaxBlocks + tid) * 5;
#pragma unroll
            for (int k = 0; k < 5; ++k)
                g[k] = __builtin_bit_cast(double, __hip_atomic_load(&p[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        }
        block_sum5(g, sh.red);
    };
    double pp[5];  // this thread's share of the published partials (threads < nb), loaded right after a barrier
    auto load_partials = [&]() {
#pragma unroll
        for (int k = 0; k < 5; ++k) pp[k] = 0.0;
        if (tid < nb) {
            const uint64_t* p = ws.partials + ((size_t)(stage & 1) * kFitMaxBlocks + tid) * 5;
#pragma unroll
            for (int k = 0; k < 5; ++k)
                pp[k] = __builtin_bit_cast(double, __hip_atomic_load(&p[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        }
    };
    float s = 1.0f, t = 0.0f;
    bool same = false;  // the last solve reproduced the previous (s, t) bit for bit
    // Closed-form weighted LS on the global sums (prompt_stem.py:222-232). The first solve: thread 0 also decides
    // the fallback and k, all threads read. Later solves: every thread holds the same sums (fixed-order block
    // reductions), so each computes the same (s, t) with the same fp64 operations and no broadcast is needed.
    auto ls = [&](const double (&g)[5], bool ok, float& ns, float& nt) {
        const double n = g[0], sx = g[1], sy = g[2], sxx = g[3], sxy = g[4];
        const double nn = n > 1.0 ? n : 1.0;
        const double den = nn * sxx - sx * sx;
        const double sn = den > 1e-12 ? (nn * sxy - sx * sy) / (den > 1e-12 ? den : 1e-12) : 1.0;
        const double tn = (sy - sn * sx) / nn;
        ns = s;
        nt = t;
        if (ok) {
            ns = (float)sn;
            nt = (float)tn;
        }
    };
    auto solve = [&](const double (&g)[5], bool first) {
        if (!first) {
            float ns, nt;
            ls(g, sh.ok != 0, ns, nt);
            same = f2u(ns) == f2u(s) && f2u(nt) == f2u(t);
            s = ns;
            t = nt;
            return;
        }
        if (tid == 0) {
            const int64_t count = (int64_t)g[0];
            sh.ok = count >= a.min_points;
            int64_t k = (int64_t)(a.keep * (float)count);
            if (k < a.min_points) k = a.min_points;
            sh.kk = k < a.N ? k : a.N;
            if (a.info && b == 0) {
                a.info[5 * a.b + 0] = (int32_t)count;
                a.info[5 * a.b + 1] = (int32_t)k;
                a.info[5 * a.b + 2] = sh.ok;
            }
            float ns, nt;
            ls(g, sh.ok != 0, ns, nt);
            sh.s = ns;
            sh.t = nt;
        }
        __syncthreads();
        same = false;
        s = sh.s;
        t = sh.t;
        __syncthreads();
    };

    // ---- round 0 weights: the mask
    {
        double v[5] = {0.0, 0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int j = 0; j < kFitEPT; ++j) {
            if ((mbits >> j) & 1u) {
                const double zd = zr[j], td = tr[j];
                v[0] += 1.0;
                v[1] += zd;
                v[2] += td;
                v[3] += zd * zd;
                v[4] += zd * td;
            }
        }
        FIT_MARK0(0);
        publish(v);
        FIT_MARK0(1);
        fit_barrier(ws, nb, ++sync_seq, a.spin_limit);
        FIT_MARK0(2);
        double g[5];
        gather_partials(g);
        ++stage;
        solve(g, true);
    }

    if (b == 0 && tid == 0) ws.trace[2 * kFitTraceRounds] = (uint32_t)wall_clock64();  // initial solve done
    if (tid == 0) {  // the last stage's record, read by the next round's plan before any stage has run
        sh.total_cand = 0;
        sh.blo_last = 0;
        sh.bhi_last = 0;
    }
    __syncthreads();
    uint32_t thr = 0, thr_prev = 0;
    bool have_prev = false;
    // the next round's plan (see its computation at the end of a round): mode, bracket, window
    int plan_mode = 2, plan_wsh = 0;
    uint32_t lo = 0, hi = 0, plan_wlo = 0;
    float dens = 0.0f;  // candidates per key near the threshold, from the last stage with enough of them

    // A fit that falls back to (1, 0) never changes (s, t): its trim rounds cannot affect the result.
    int rounds = 0;  // trim rounds run (the loop stops early at a fixed point)
    for (int it = 0; it < (sh.ok ? a.iters : 0); ++it) {
        rounds = it + 1;
        // The element values and mask bits are loop-invariant; hiding that from the compiler keeps it from hoisting
        // their fp64 products and per-element lane masks out of the loop into hundreds of extra registers.
#pragma unroll
        for (int j = 0; j < kFitEPT; ++j) asm volatile("" : "+v"(zr[j]), "+v"(tr[j]));
        asm volatile("" : "+v"(mbits), "+v"(vbits));
        // ---- relative residuals as ordered bit patterns (+inf off the mask, kInvalid on padding)
        uint32_t rb[kFitEPT];
#pragma unroll
        for (int j = 0; j < kFitEPT; ++j) {
            float e = s * zr[j];
            e = e + t;
            e = e - tr[j];
            const float r = __builtin_fabsf(e) / fmax_(tr[j], 1e-3f);
            const uint32_t rm = ((mbits >> j) & 1u) ? f2u(r) : 0x7f800000u;
            rb[j] = ((vbits >> j) & 1u) ? rm : kInvalid;
        }
        const unsigned kk = (unsigned)sh.kk;

        // Publishes below-count, below-sums and the candidates in [blo, bhi]; then a barrier; then the totals.
        auto stage_bracket = [&](uint32_t blo, uint32_t bhi) {
            FIT_MARK(0);
            asm volatile("" : "+v"(mbits), "+v"(vbits));  // no per-element lane masks kept across phases
            // branch-free: below-count, masked below-sums (fp64; z*z and z*t are exact in fp64), candidate count
            double v[5] = {0.0, 0.0, 0.0, 0.0, 0.0};
            unsigned below = 0, nc = 0, nm = 0;
#pragma unroll
            for (int j = 0; j < kFitEPT; ++j) {
                const uint32_t k = rb[j];
                const bool isb = k < blo;
                const bool inc = isb && ((mbits >> j) & 1u);
                below += isb ? 1u : 0u;
                nm += inc ? 1u : 0u;
                nc += (!isb && k <= bhi) ? 1u : 0u;
                const double zd = inc ? (double)zr[j] : 0.0;
                const double td = inc ? (double)tr[j] : 0.0;
                v[1] += zd;
                v[2] += td;
                v[3] += zd * zd;
                v[4] += zd * td;
            }
            v[0] = (double)nm;
            // one scan for both counts: below in the high half, candidates in the low half (each <= 8192 per block)
            unsigned packed_total;
            const unsigned packed = block_excl_scan((below << 16) | nc, sh.tmp, packed_total);
            unsigned slot = packed & 0xffffu;
            const unsigned ncb = packed_total & 0xffffu;
            const size_t base = (size_t)(stage & 1) * cap_words + (size_t)b * kFitPerBlock;
#pragma unroll
            for (int j = 0; j < kFitEPT; ++j) {
                const uint32_t k = rb[j];
                if (k >= blo && k <= bhi) {
                    ws.c_key[base + slot] = k | (((mbits >> j) & 1u) << 31);
                    ws.c_z[base + slot] = zr[j];
                    ws.c_t[base + slot] = tr[j];
                    ++slot;
                }
            }
            publish(v);
            FIT_MARK(1);
            // the block's counts (below in the high half, candidates in the low half) ride on the barrier's flag
            const unsigned counts = fit_barrier(ws, nb, ++sync_seq, a.spin_limit, packed_total);
            FIT_MARK(2);
            load_partials();  // needed only by the sums after the selection: in flight with the candidate loads
            // totals and region offsets, in block order
            unsigned cb = 0, cc = 0;
            if (tid < nb) {
                cb = counts >> 16;
                cc = counts & 0xffffu;
                // a block publishes at most its own element count; the clamp only matters after an expired wait,
                // when the counts may be another launch's, and keeps every candidate read inside this launch's
                // regions
                cb = cb < (unsigned)kFitPerBlock ? cb : (unsigned)kFitPerBlock;
                cc = cc < (unsigned)kFitPerBlock ? cc : (unsigned)kFitPerBlock;
            }
            unsigned tb, tc;
            const unsigned offc = block_excl_scan2(cc, cb, sh.tmp2, tc, tb);
            if (tid < nb) sh.off[tid] = offc;
            if (tid == 0) {
                sh.off[nb] = tc;
                sh.total_below = tb;
                sh.total_cand = tc;
                sh.blo_last = blo;
                sh.bhi_last = bhi;
            }
            __syncthreads();
            FIT_MARK(3);
        };

        // Exact k-th among the published candidates (all in [blo, bhi]) and the new (s, t); buffer `stage & 1`.
        auto select_and_solve = [&](uint32_t blo, uint32_t bhi) {
            const unsigned total = sh.total_cand;
            unsigned rank = kk - sh.total_below;
            const size_t bufo = (size_t)(stage & 1) * cap_words;
            // Thread (r, j) = (tid % nb, tid / nb) owns slots j, j + per, j + 2 per, ... of block r's region: no
            // search from a flat index to a region, and its loads are independent. Keys go to LDS in flat order
            // (region r at off[r]); the first kHold of the thread's candidates also keep z and target in registers
            // for the sums (loaded with the keys: usually no second round trip).
            constexpr int kHold = 12;
            const int per = kFitThreads / nb;  // threads per region (nb <= kFitThreads)
            const int rr = tid % nb, jj = tid / nb;
            const bool act = jj < per;
            const unsigned cr = act ? sh.off[rr + 1] - sh.off[rr] : 0u;
            const unsigned obase = act ? sh.off[rr] : 0u;
            const size_t rbase = bufo + (size_t)rr * kFitPerBlock;
            uint32_t hw[kHold];
            float hz[kHold], ht[kHold];
#pragma unroll
            for (int u = 0; u < kHold; ++u) {
                const unsigned slot = (unsigned)(jj + u * per);
                hw[u] = 0;
                hz[u] = 0.0f;
                ht[u] = 0.0f;
                if (slot < cr) {
                    hw[u] = ws.c_key[rbase + slot];
                    hz[u] = ws.c_z[rbase + slot];
                    ht[u] = ws.c_t[rbase + slot];
                }
            }
#pragma unroll
            for (int u = 0; u < kHold; ++u) {
                const unsigned slot = (unsigned)(jj + u * per);
                if (slot < cr) sh.cand[obase + slot] = hw[u];
            }
            for (unsigned s0 = (unsigned)(jj + kHold * per); s0 < cr; s0 += (unsigned)(kHold * per)) {
                uint32_t w[kHold];
#pragma unroll
                for (int u = 0; u < kHold; ++u) {
                    const unsigned slot = s0 + (unsigned)(u * per);
                    w[u] = slot < cr ? ws.c_key[rbase + slot] : 0u;
                }
#pragma unroll
                for (int u = 0; u < kHold; ++u) {
                    const unsigned slot = s0 + (unsigned)(u * per);
                    if (slot < cr) sh.cand[obase + slot] = w[u];
                }
            }
            __syncthreads();
            FIT_MARK(4);
            uint32_t prefix = 0, pmask = 0;
            int top = 0;
            if (total <= 96u) {
                // few candidates: each thread ranks its own against all of them (LDS broadcast reads; beyond ~100
                // candidates the radix select below is faster)
                if (tid == 0) sh.bin = 0;
                __syncthreads();
                if ((unsigned)tid < total) {
                    const uint32_t key = sh.cand[tid] & 0x7fffffffu;
                    unsigned less = 0, eq = 0;
                    // four keys per 16-byte LDS read and four reads in flight per trip: one 4-byte read per trip
                    // waited out its latency every time (107 candidates took 5.6 us)
                    const unsigned t4 = total & ~3u;
#pragma unroll 4
                    for (unsigned g = 0; g < t4; g += 4) {
                        const uint4 q = *(const uint4*)&sh.cand[g];
                        const uint32_t kq[4] = {q.x & 0x7fffffffu, q.y & 0x7fffffffu, q.z & 0x7fffffffu,
                                                q.w & 0x7fffffffu};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            less += kq[e] < key ? 1u : 0u;
                            eq += kq[e] == key ? 1u : 0u;
                        }
                    }
                    for (unsigned g = t4; g < total; ++g) {
                        const uint32_t kg = sh.cand[g] & 0x7fffffffu;
                        less += kg < key ? 1u : 0u;
                        eq += kg == key ? 1u : 0u;
                    }
                    if (less < rank && rank <= less + eq) sh.bin = key - blo;  // equal keys write equal values
                }
                __syncthreads();
                prefix = sh.bin;
            } else {
                // MSD radix select over key - blo in [0, bhi - blo], 11 bits per pass
                const uint32_t range = bhi - blo;
                top = range ? 32 - __builtin_clz(range) : 0;
            }
            while (top > 0) {
                const int width = top < 11 ? top : 11;
                const int shb = top - width;
                const uint32_t dmask = (1u << width) - 1u;
                for (int q = tid; q < kFitBins; q += kFitThreads) sh.hist[q] = 0;
                __syncthreads();
                for (unsigned f = tid; f < total; f += kFitThreads) {
                    const uint32_t key = (sh.cand[f] & 0x7fffffffu) - blo;
                    if ((key & pmask) == prefix) atomicAdd(&sh.hist[(key >> shb) & dmask], 1u);
                }
                __syncthreads();
                find_bin(sh, rank, [&](int q) { return sh.hist[q]; }, [] { return 0u; });
                prefix |= sh.bin << shb;
                pmask |= dmask << shb;
                rank -= sh.below;
                top = shb;
            }
            thr = blo + prefix;
            FIT_MARK(5);
            // sums: this thread's share of the published below-partials, then its candidates at or under thr in
            // flat order; then one fixed-order block reduction
            double v[5] = {pp[0], pp[1], pp[2], pp[3], pp[4]};
#pragma unroll
            for (int u = 0; u < kHold; ++u) {
                const uint32_t w = hw[u];
                if ((w >> 31) && (w & 0x7fffffffu) <= thr) {
                    const double zd = hz[u], td = ht[u];
                    v[0] += 1.0;
                    v[1] += zd;
                    v[2] += td;
                    v[3] += zd * zd;
                    v[4] += zd * td;
                }
            }
            for (unsigned s0 = (unsigned)(jj + kHold * per); s0 < cr; s0 += (unsigned)(kHold * per)) {
                // kHold candidates per trip: all loads issued before any is used
                float cz[kHold], ct[kHold];
                bool use[kHold];
#pragma unroll
                for (int u = 0; u < kHold; ++u) {
                    const unsigned slot = s0 + (unsigned)(u * per);
                    const uint32_t w = slot < cr ? sh.cand[obase + slot] : 0u;
                    use[u] = (w >> 31) && (w & 0x7fffffffu) <= thr;
                    cz[u] = use[u] ? ws.c_z[rbase + slot] : 0.0f;
                    ct[u] = use[u] ? ws.c_t[rbase + slot] : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < kHold; ++u) {
                    if (use[u]) {
                        const double zd = cz[u], td = ct[u];
                        v[0] += 1.0;
                        v[1] += zd;
                        v[2] += td;
                        v[3] += zd * zd;
                        v[4] += zd * td;
                    }
                }
            }
            block_sum5(v, sh.red);
            ++stage;
            solve(v, false);
            FIT_MARK(6);
        };

        // Histogram pass over a window of keys: bin q counts the keys in [wlo + q 2^wsh, wlo + (q+1) 2^wsh), q < 2048,
        // and one more counter the keys below wlo; blocks merge their LDS histograms into this round's global slot
        // `hslot` by atomics, and after one barrier every block finds the bin holding the kk-th key. Returns false
        // when that key lies outside the window; else pbin_lo / pbin_cnt give the bin's first key and its count.
        // One call site serves the radix passes and the predicted windows (the unrolled element loop exists once).
        int hslot = 0;
        uint32_t pbin_lo = 0;
        unsigned pbin_cnt = 0, pbin_below = 0;
        // `below` is the count of keys below wlo when the caller knows it (the radix range starts at 0, and a pass
        // that splits a bin follows the keys before that bin), else kNoBelow: the pass counts them, into 16 words
        // (block b adds to word b % 16) so that the 75-94 blocks' atomics do not all queue on one address.
        constexpr unsigned kNoBelow = 0xffffffffu;
        auto hist_pass = [&](uint32_t wlo, int wsh, unsigned below) -> bool {
            asm volatile("" : "+v"(mbits), "+v"(vbits));
            for (int q = tid; q < kFitBins; q += kFitThreads) sh.hist[q] = 0;
            if (tid == 0) sh.hbelow = 0;
            __syncthreads();
            unsigned nbelow = 0;
#pragma unroll
            for (int j = 0; j < kFitEPT; ++j) {  // one branch per element (around its LDS atomic)
                const uint32_t k = rb[j];
                const bool v = (vbits >> j) & 1u;
                const uint32_t q = (k - wlo) >> wsh;
                nbelow += (v && k < wlo) ? 1u : 0u;
                if (v && k >= wlo && q < (uint32_t)kFitBins) atomicAdd(&sh.hist[q], 1u);
            }
            const bool count_below = below == kNoBelow;
            if (count_below) {
                nbelow = wave_incl_scan_u32(nbelow);
                if ((tid & 63) == 63 && nbelow) atomicAdd(&sh.hbelow, nbelow);
            }
            __syncthreads();
            unsigned* gh = ws.hist + ((int64_t)it * kFitHistSlots + hslot) * kFitHistWords;
            hslot = hslot + 1 < kFitHistSlots ? hslot + 1 : hslot;  // at most 6 passes a round (never reached)
            for (int q = tid; q < kFitBins; q += kFitThreads)
                if (sh.hist[q]) atomicAdd(&gh[q], sh.hist[q]);
            if (count_below && tid == 0 && sh.hbelow) atomicAdd(&gh[kFitBins + (b & 15)], sh.hbelow);
            fit_barrier(ws, nb, ++sync_seq, a.spin_limit);
            find_bin(
                sh, kk, [&](int q) { return __hip_atomic_load(&gh[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); },
                [&] {
                    if (!count_below) return below;
                    unsigned v = 0;
#pragma unroll
                    for (int q = 0; q < 16; ++q)
                        v += __hip_atomic_load(&gh[kFitBins + q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    return v;
                });
            if (!sh.found) return false;  // below or above the window (read from LDS: the block branches as one)
            pbin_lo = wlo + (sh.bin << wsh);
            pbin_cnt = sh.bincnt;
            pbin_below = sh.below;
            return true;
        };

        // The round's selection. mode 0: one bracket stage on the predicted bracket [lo, hi]; 1: a histogram pass on
        // the predicted window, then a stage on its bin; 2: radix passes over the whole key range (bits 31..21, then
        // 20..10 of the first bin, then single values, each only while the bin holds more than kStageMax keys),
        // then a stage on the bin. A bracket stage that misses the k-th is followed by a window on the side that
        // holds it; a window that misses it, by the radix passes. Trace codes: 0 bracket, 1 bracket missed -> radix
        // (no key above it), 2 radix, 4 window, 5 bracket missed -> window, 6 window missed -> radix, 7 bracket and
        // window missed -> radix; +8 when one
        // value holds the k-th and more than kCandCap keys (its sums take a barrier of their own).
        int mode = plan_mode;
        int path = mode == 0 ? 0 : (mode == 1 ? 4 : 2);
        int passes = 0;
        uint32_t blo = lo, bhi = hi, wlo = plan_wlo;
        int wsh = plan_wsh;
#pragma nounroll
        for (;;) {
            if (mode != 0) {
                if (mode == 2) {
                    wlo = 0;
                    wsh = 21;
                }
                bool hit;
                unsigned below = mode == 2 ? 0u : kNoBelow;
#pragma nounroll
                for (;;) {
                    hit = hist_pass(wlo, wsh, below);
                    ++passes;
                    if (!hit || pbin_cnt <= kStageMax || wsh == 0) break;
                    wlo = pbin_lo;  // split the bin: 2048 sub-bins of 2^(wsh - 11) keys
                    wsh = wsh > 11 ? wsh - 11 : 0;
                    below = pbin_below;
                }
                if (!hit) {
                    if (mode == 2) break;  // the whole range holds every key: only after an expired wait
                    mode = 2;
                    path = path == 5 ? 7 : 6;
                    continue;
                }
                blo = pbin_lo;
                const uint64_t e = (uint64_t)pbin_lo + ((1ull << wsh) - 1u);
                bhi = e > 0xffffffffull ? 0xffffffffu : (uint32_t)e;
                if (pbin_cnt > (unsigned)kCandCap) {
                    // one value (wsh == 0) holds the k-th and more keys than LDS holds: it is the threshold; the
                    // sums over the keys at or below it take one more barrier
                    path |= 8;
                    thr = blo;
                    double v[5] = {0.0, 0.0, 0.0, 0.0, 0.0};
#pragma unroll
                    for (int j = 0; j < kFitEPT; ++j) {
                        if (((mbits >> j) & 1u) && rb[j] <= thr) {
                            const double zd = zr[j], td = tr[j];
                            v[0] += 1.0;
                            v[1] += zd;
                            v[2] += td;
                            v[3] += zd * zd;
                            v[4] += zd * td;
                        }
                    }
                    publish(v);
                    fit_barrier(ws, nb, ++sync_seq, a.spin_limit);
                    double g[5];
                    gather_partials(g);
                    ++stage;
                    solve(g, false);
                    break;
                }
            }
            stage_bracket(blo, bhi);
            const unsigned tbl = sh.total_below, tcd = sh.total_cand;
            if (tbl < kk && kk <= tbl + tcd && tcd <= (unsigned)kCandCap) {
                select_and_solve(blo, bhi);
                break;
            }
            ++stage;
            if (mode != 0) break;  // a pass bin the stage does not confirm: only after an expired wait
            // the bracket missed: a window of 2^plan_wsh-key bins on the side that holds the k-th (or, when the
            // bracket held it among more candidates than LDS holds, a window over the bracket itself)
            mode = 1;
            path = 5;
            wsh = plan_wsh;
            const uint64_t span = (uint64_t)kFitBins << wsh;
            if (kk <= tbl) {
                wlo = (uint64_t)blo > span ? blo - (uint32_t)span : 0u;
            } else if (kk <= tbl + tcd) {
                wlo = blo;
                wsh = 0;
                while (((uint64_t)kFitBins << wsh) < (uint64_t)bhi - blo + 1u && wsh < 21) ++wsh;
            } else if (bhi == 0xffffffffu) {
                mode = 2;
                path = 1;
            } else {
                wlo = bhi + 1u;
            }
        }

        if (b == 0 && tid == 0 && it < kFitTraceRounds) {
            ws.trace[2 * it] = (uint32_t)path | ((uint32_t)(passes < 15 ? passes : 15) << 4) | (sh.total_cand << 8);
            ws.trace[768 + it] = thr;
            ws.trace[2 * it + 1] = (uint32_t)wall_clock64();
        }
        // Fixed point: when a round reproduces the previous (s, t) bit for bit, the next round sees the same
        // residuals, hence the same k-th value, weights and sums, so every remaining round -- and the final
        // solve -- returns exactly these (s, t). Stopping here gives the bit-identical result.
        // ---- the next round's plan. The threshold's move from round to round (in keys, which order like the
        // values) shrinks by 2-5x per round on the refined maps, keeps its sign while it is large, and jitters by
        // ~10^3 keys near the fixed point. The bracket reaches a quarter of the last move against it and half a move
        // along it, plus a margin of at least 2048 keys and ~32 expected candidates; when that bracket would hold
        // more than kBracketMax candidates at the density the stages saw (candidates per key, kept from the last
        // stage with at least 64), a window pass over twice that range goes first, its bins sized for 2048 over the
        // range. A move of more than an octave is the first trim dropping the outliers of an exact point map: the
        // next round usually repeats the threshold, so the bracket is ~256 expected candidates around it.
        if (same) break;  // the fixed point below: no next round to plan
        // (heuristics only, in fp32 with the hardware reciprocal: the plan never changes a result)
        if (sh.total_cand >= 64u || dens <= 0.0f)
            dens = (float)sh.total_cand * __builtin_amdgcn_rcpf((float)(sh.bhi_last - sh.blo_last) + 1.0f);
        plan_mode = 2;
        if (!have_prev) {
            // after round 0: the first trim drops the outliers' pull, and the threshold falls by up to ~11 octaves
            // (exact point maps) or moves by under one (noisy ones); a window from 14 octaves below to 2 above it
            // in 2048 bins of 2^16 keys (1/128 octave) holds it
            plan_mode = 1;
            plan_wsh = 16;
            plan_wlo = thr > (14u << 23) ? thr - (14u << 23) : 0u;
        } else {
            // keys are below 2^31 (non-negative floats, NaN included), so every range here fits 32 bits
            const bool up = thr >= thr_prev;
            const uint32_t am = up ? thr - thr_prev : thr_prev - thr;
            const float rdens = dens > 0.0f ? __builtin_amdgcn_rcpf(dens) : 0.0f;
            auto keys_for = [&](float cands) {  // keys that hold about `cands` candidates, in [2048, 2^18]
                const float k = dens > 0.0f ? cands * rdens : 2048.0f;
                return (uint32_t)(k < 2048.0f ? 2048.0f : (k > 262144.0f ? 262144.0f : k));
            };
            const bool jump = am > (1u << 23);  // a jump of over an octave predicts no move
            uint32_t along = am / 2 + keys_for(32.0f), against = am / 4 + keys_for(32.0f);
            if (jump) along = against = keys_for(128.0f);
            const float expect = dens * ((float)(along + against) + 1.0f);
            const uint32_t dn = up ? against : along, dp = up ? along : against;
            if (expect <= kBracketMax || jump) {
                plan_mode = 0;
                lo = thr > dn ? thr - dn : 0u;
                hi = thr + dp < thr ? 0xffffffffu : thr + dp;
            } else {
                plan_mode = 1;
            }
            // window bins: the smallest power of two that spans twice the bracket's range in 2048 bins
            const uint32_t span = 2 * (along + against);
            const int lg = 32 - __builtin_clz(span - 1u);  // ceil(log2(span)), span >= 2^13
            plan_wsh = lg > 11 ? (lg - 11 < 21 ? lg - 11 : 21) : 0;
            plan_wlo = thr > 2 * dn ? thr - 2 * dn : 0u;
        }
        // Test hook: plans that are wrong on purpose, to exercise the fallbacks (the results must not change).
        // 1: a bracket just above its predicted range (the k-th usually lies below: a window on that side follows);
        // 2: every plan a window above +inf (it misses: the radix passes follow); 3: windows of 2^21-key bins from
        // 2^24 keys below the threshold (split passes with a counted below-window part).
        if (a.plan_debug == 1 && plan_mode == 0) {
            const uint32_t w = hi - lo;
            lo = hi < 0xffffffffu ? hi + 1u : hi;
            hi = lo + w < lo ? 0xffffffffu : lo + w;
        } else if (a.plan_debug == 2) {
            plan_mode = 1;
            plan_wlo = 0x7f800001u;
            plan_wsh = 0;
        } else if (a.plan_debug == 3 && plan_mode == 1) {
            plan_wlo = thr > (1u << 24) ? thr - (1u << 24) : 0u;
            plan_wsh = 21;
        }
        thr_prev = thr;
        have_prev = true;
    }

    if (b == 0 && tid == 0) {
        __hip_atomic_store(&ws.bar[2], sync_seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        a.st[2 * a.b] = s;
        a.st[2 * a.b + 1] = t;
        if (a.info) a.info[5 * a.b + 3] = (int32_t)thr;
        ws.trace[2 * kFitTraceRounds + 2] = (uint32_t)rounds;
    }

    // Completion. The last block to finish sees every block's writes; it reports the launch's error flag. After
    // an expired wait the blocks may have passed different numbers of barriers, so their flags and the epoch no
    // longer agree: it zeroes all of them (every flag line, not only this grid's, since the epoch restarts at 0),
    // clears the flag, counts the failure and replaces (s, t), which raced, by NaN.
    __syncthreads();
    if (tid == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const unsigned prev = __hip_atomic_fetch_add(ws.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sh.last = prev == (unsigned)nb - 1u;
        if (sh.last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    if (!sh.last) return;
    const int err = __hip_atomic_load(ws.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (err) {
        for (int q = tid; q < kFitMaxBlocks * 16; q += kFitThreads)
            __hip_atomic_store(&ws.flags[q], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (tid == 0) {
        if (err) {
            const float nan = __builtin_nanf("");
            a.st[2 * a.b] = nan;
            a.st[2 * a.b + 1] = nan;
            __hip_atomic_store(&ws.bar[2], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(ws.err, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(ws.err_seen, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (a.info) a.info[5 * a.b + 4] = err;
        __hip_atomic_store(ws.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Elements per thread: 16 up to 2^19 elements (twice the blocks: faster loads and per-block passes, while the
// device-wide barrier still costs little), 24 up to 1.5 M (config H's 762,048: 124 blocks; measured against 20 and
// 28 per thread, 149 / 109 blocks, and the 32 used before: the fits on H's input / refined map took 85 / 210 us
// against 96 / 239, 86 / 212 and 91 / 220), else 32.
static int fit_ept(int64_t N) {
    return N <= (int64_t(1) << 19) ? 16 : N <= (int64_t)kFitThreads * 24 * kFitMaxBlocks ? 24 : 32;
}
static int fit_blocks(int64_t N) {
    const int64_t per = (int64_t)kFitThreads * fit_ept(N);
    return (int)((N + per - 1) / per);
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t fit_workspace_bytes(int64_t N, int iters) {
    const int64_t n = N > 0 ? N : 1;
    const size_t nb = (size_t)fit_blocks(n);
    const size_t hist = (size_t)(iters > 0 ? iters : 1) * kFitHistSlots * kFitHistWords * sizeof(unsigned);
    const size_t cand = 2 * nb * (size_t)kFitThreads * fit_ept(n) * sizeof(uint32_t);
    return kFitHeader + align256(kFitMaxBlocks * 64) + align256(2 * kFitMaxBlocks * 5 * sizeof(uint64_t)) +
           align256(hist) + 3 * align256(cand);
}

// Polls of one barrier wait before it expires (~0.1 s at the default); lowered only by the test hook
// pmg_debug_fit_spin_limit, so that tests can make waits expire with every kernel still exiting normally.
static unsigned g_fit_spin_limit = 1u << 23;
// Wrong-on-purpose round plans for tests (pmg_debug_fit_plan); 0 in normal use.
static int g_fit_plan_debug = 0;

int launch_fit(const FitLaunch& f, hipStream_t s) {
    PMG_REQUIRE(f.N > 0 && f.N <= (int64_t)kFitMaxBlocks * kFitPerBlockMax, "N must be in [1, 2^21]");
    PMG_REQUIRE(f.iters >= 0 && f.iters <= 64, "iters must be in [0, 64]");
    PMG_REQUIRE(f.min_points >= 1, "min_points must be >= 1");
    PMG_REQUIRE(f.trim >= 0.0f && f.trim < 1.0f, "trim must be in [0, 1)");
    PMG_REQUIRE(f.workspace && f.workspace_bytes >= fit_workspace_bytes(f.N, f.iters), "workspace too small");
    PMG_REQUIRE(aligned16(f.workspace), "workspace must be 16-byte aligned");
    const int nb = fit_blocks(f.N);
    const int ept = fit_ept(f.N);
    static int max_resident[3] = {-1, -1, -1};
    int& mr = max_resident[ept == 16 ? 0 : ept == 24 ? 1 : 2];
    if (mr < 0) {
        int per_cu = 0;
        if (ept == 16)
            PMG_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fit_k<16>, kFitThreads, 0));
        else if (ept == 24)
            PMG_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fit_k<24>, kFitThreads, 0));
        else
            PMG_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fit_k<32>, kFitThreads, 0));
        mr = per_cu * num_cus();
    }
    const int max_resident_n = mr;
    PMG_REQUIRE(nb <= max_resident_n && nb <= kFitMaxBlocks,
                "fit grid of " + std::to_string(nb) + " blocks cannot be resident (max " +
                    std::to_string(max_resident_n) + ")");
    uint8_t* p = (uint8_t*)f.workspace;
    FitWs ws;
    ws.bar = (unsigned*)p;
    ws.err = (int*)(p + kFitErrOffset);
    ws.trace = (uint32_t*)(p + 128);
    ws.done = (unsigned*)(p + kFitDoneOffset);
    ws.err_seen = (unsigned*)(p + kFitErrSeenOffset);
    p += kFitHeader;
    ws.flags = (unsigned*)p;
    p += align256(kFitMaxBlocks * 64);
    ws.partials = (uint64_t*)p;
    p += align256(2 * kFitMaxBlocks * 5 * sizeof(uint64_t));
    ws.hist = (unsigned*)p;
    p += align256((size_t)(f.iters > 0 ? f.iters : 1) * kFitHistSlots * kFitHistWords * sizeof(unsigned));
    const size_t cand = align256(2 * (size_t)nb * kFitThreads * ept * sizeof(uint32_t));
    ws.c_key = (uint32_t*)p;
    ws.c_z = (float*)(p + cand);
    ws.c_t = (float*)(p + 2 * cand);
    for (int b = 0; b < f.B; ++b) {
        FitArgs a{f.mode, f.z, f.tg, f.mask, f.logz, f.stride, f.lidar, f.conf, f.H, f.W, f.dh, f.dw,
                  f.N, f.iters, (float)(1.0 - (double)f.trim), f.min_points, b, f.st, f.info,
                  g_fit_spin_limit, g_fit_plan_debug, ws};
        if (ept == 16)
            hipLaunchKernelGGL(fit_k<16>, dim3(nb), dim3(kFitThreads), 0, s, a);
        else if (ept == 24)
            hipLaunchKernelGGL(fit_k<24>, dim3(nb), dim3(kFitThreads), 0, s, a);
        else
            hipLaunchKernelGGL(fit_k<32>, dim3(nb), dim3(kFitThreads), 0, s, a);
        if (int e = check_launch("fit_k")) return e;
    }
    return PMG_OK;
}

// ------------------------------------------------------------------------------------------------------------
// Final metric fit inputs (v3.py:768-775), one thread per LiDAR pixel: d_lr = F.interpolate(depth, (dh, dw),
// mode='area') of z = exp(logz) -- adaptive average pooling, the window [floor(o*H/dh), ceil((o+1)*H/dh)) summed
// in fp32 in row-major order and divided by its height, then by its width, as adaptive_avg_pool2d does -- and
// mask = conf >= 2 & lidar > 0 & d_lr > 0 (& the pooled mask_binary > 0.99).
__global__ __launch_bounds__(256) void final_inputs_k(const float* __restrict__ logz, int64_t stride,
                                                      const float* __restrict__ lidar, const float* __restrict__ conf,
                                                      const uint8_t* __restrict__ mask_binary, int H, int W, int dh,
                                                      int dw, int64_t n_out, float* __restrict__ z_out,
                                                      uint8_t* __restrict__ m_out) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= n_out) return;
    const int64_t plane = (int64_t)dh * dw;
    const int64_t b = q / plane;
    const int rem = (int)(q - b * plane);
    const int oh = rem / dw, ow = rem - oh * dw;
    const int r0 = (int)(((int64_t)oh * H) / dh), r1 = (int)((((int64_t)oh + 1) * H + dh - 1) / dh);
    const int c0 = (int)(((int64_t)ow * W) / dw), c1 = (int)((((int64_t)ow + 1) * W + dw - 1) / dw);
    const int64_t base = b * H * W;
    float sz = 0.0f, sm = 0.0f;
    for (int r = r0; r < r1; ++r)
        for (int c = c0; c < c1; ++c) {
            const int64_t p = base + (int64_t)r * W + c;
            sz = sz + exp_f32(logz[p * stride]);
            if (mask_binary) sm = sm + (mask_binary[p] ? 1.0f : 0.0f);
        }
    const float kh = (float)(r1 - r0), kw = (float)(c1 - c0);
    const float z = sz / kh / kw;
    const float d = lidar[q];
    bool m = conf[q] >= 2.0f && d > 0.0f && z > 0.0f;
    if (mask_binary) m = m && (sm / kh / kw > 0.99f);
    z_out[q] = z;
    m_out[q] = m ? 1 : 0;
}

// post_depth (MetricFit.metal:200-211; v3.py:776 depth = s * z + t): the metric depth of every pixel from the refined
// log depth and the final fit of its frame, d = s * exp(logz) + t in fp32; +inf where the mask is 0 or d <= 0.
__global__ __launch_bounds__(256) void post_depth_k(const float* __restrict__ logz, int64_t stride,
                                                    const uint8_t* __restrict__ mask, int64_t HW, int64_t n,
                                                    const float* __restrict__ st, float* __restrict__ depth) {
    const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (p >= n) return;
    const int64_t b = p / HW;
    const float d = st[2 * b] * exp_f32(logz[p * stride]) + st[2 * b + 1];
    const bool ok = (mask == nullptr || mask[p] != 0) && d > 0.0f;
    depth[p] = ok ? d : __builtin_inff();
}

size_t final_fit_workspace_bytes(int B, int dh, int dw, int iters) {
    const size_t n = (size_t)B * dh * dw;
    return align256(fit_workspace_bytes((int64_t)dh * dw, iters)) + align256(n * sizeof(float)) + align256(n);
}

int launch_final_fit(const FinalFit& f, hipStream_t s) {
    PMG_REQUIRE(f.logz && f.lidar && f.conf && f.st, "null buffer");
    PMG_REQUIRE(f.B >= 1 && f.H >= 1 && f.W >= 1 && f.dh >= 1 && f.dw >= 1 && f.stride >= 1, "bad shape");
    PMG_REQUIRE((int64_t)f.dh * f.dw <= (int64_t)kFitMaxBlocks * kFitPerBlockMax, "LiDAR map larger than 2^21 pixels");
    PMG_REQUIRE(f.workspace && f.workspace_bytes >= final_fit_workspace_bytes(f.B, f.dh, f.dw, f.iters),
                "workspace too small");
    const int64_t N = (int64_t)f.dh * f.dw;
    const int64_t n_out = (int64_t)f.B * N;
    const size_t fit_bytes = align256(fit_workspace_bytes(N, f.iters));
    if (f.dh == f.H && f.dw == f.W) {
        // one-pixel area windows: the fit reads exp(logz), the LiDAR, conf and mask_binary itself (no
        // final_inputs_k launch; the same values)
        FitLaunch g{};
        g.mode = 2;
        g.logz = f.logz;
        g.stride = f.stride;
        g.lidar = f.lidar;
        g.conf = f.conf;
        g.mask = f.mask_binary;
        g.H = f.H;
        g.W = f.W;
        g.dh = f.dh;
        g.dw = f.dw;
        g.B = f.B;
        g.N = N;
        g.iters = f.iters;
        g.trim = f.trim;
        g.min_points = f.min_points;
        g.st = f.st;
        g.info = f.info;
        g.workspace = f.workspace;
        g.workspace_bytes = fit_bytes;
        return launch_fit(g, s);
    }
    float* z_lr = (float*)((uint8_t*)f.workspace + fit_bytes);
    uint8_t* m_lr = (uint8_t*)f.workspace + fit_bytes + align256((size_t)n_out * sizeof(float));
    hipLaunchKernelGGL(final_inputs_k, dim3((unsigned)((n_out + 255) / 256)), dim3(256), 0, s, f.logz, f.stride,
                       f.lidar, f.conf, f.mask_binary, f.H, f.W, f.dh, f.dw, n_out, z_lr, m_lr);
    if (int e = check_launch("final_inputs_k")) return e;
    FitLaunch g{};
    g.mode = 0;
    g.z = z_lr;
    g.tg = f.lidar;
    g.mask = m_lr;
    g.B = f.B;
    g.N = N;
    g.iters = f.iters;
    g.trim = f.trim;
    g.min_points = f.min_points;
    g.st = f.st;
    g.info = f.info;
    g.workspace = f.workspace;
    g.workspace_bytes = fit_bytes;
    return launch_fit(g, s);
}

// ------------------------------------------------------------------------------------------------------------
// Allocation-free fit: the workspace is a file-scope device array, one copy per GPU, instead of caller memory.
// 14 MiB holds the workspace of N <= 2^19 elements per batch item at iters <= 16 (13.4 MB). Host code never uses
// the array's name as an address: at a device's first call its address is looked up with hipGetSymbolAddress
// (the device current), kept per device, and only that pointer reaches kernels.
constexpr size_t kStaticFitBytes = (size_t)14 << 20;
constexpr int kStaticFitMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kStaticFitBytes];

__global__ void zero_words_k(uint32_t* p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

static std::mutex g_static_fit_mu;
static void* g_static_fit_ptr[kStaticFitMaxDevices];

// The current device's scratch address. At the device's first call it also enqueues, on `s`, the clearing of the
// part of the workspace the fit requires at zero before its first launch (the barrier epoch, error flag, completion
// count and per-block flags; the rest is cleared or overwritten by every launch).
static int static_fit_scratch(hipStream_t s, void** out) {
    int dev = -1;
    PMG_CHECK_HIP(hipGetDevice(&dev));
    PMG_REQUIRE(dev >= 0 && dev < kStaticFitMaxDevices, "device index out of range for the static fit scratch");
    std::lock_guard<std::mutex> lock(g_static_fit_mu);
    if (!g_static_fit_ptr[dev]) {
        void* p = nullptr;
        PMG_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        const int64_t words = (int64_t)(kFitHeader + align256((size_t)kFitMaxBlocks * 64)) / 4;
        hipLaunchKernelGGL(zero_words_k, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, s, (uint32_t*)p, words);
        if (int e = check_launch("zero_words_k")) return e;
        g_static_fit_ptr[dev] = p;
    }
    *out = g_static_fit_ptr[dev];
    return PMG_OK;
}

}  // namespace pmg

using namespace pmg;

extern "C" {

size_t pmg_fit_workspace_bytes(int64_t N, int iters) { return fit_workspace_bytes(N, iters); }

int pmg_fit_scale_shift_static(const float* z, const float* target, const uint8_t* mask, int B, int64_t N, int iters,
                               float trim, int min_points, float* st, int32_t* info, void* stream) {
    PMG_REQUIRE(z && target && mask && st, "null buffer");
    PMG_REQUIRE(B >= 1, "bad batch");
    PMG_REQUIRE(N > 0 && N <= ((int64_t)1 << 19) && iters >= 0 && iters <= 16,
                "pmg_fit_scale_shift_static: N = " + std::to_string(N) + ", iters = " + std::to_string(iters) +
                    " exceed the static scratch (N <= 2^19 per batch item, iters <= 16); use pmg_fit_scale_shift "
                    "with a caller workspace");
    PMG_REQUIRE(fit_workspace_bytes(N, iters) <= kStaticFitBytes, "static fit scratch too small");
    hipStream_t s = (hipStream_t)stream;
    void* ws = nullptr;
    if (int e = static_fit_scratch(s, &ws)) return e;
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
    f.workspace = ws;
    f.workspace_bytes = kStaticFitBytes;
    return launch_fit(f, s);
}

unsigned pmg_debug_fit_spin_limit(unsigned polls) {
    const unsigned prev = g_fit_spin_limit;
    g_fit_spin_limit = polls ? polls : (1u << 23);
    return prev;
}

unsigned pmg_debug_fit_plan(unsigned mode) {
    const unsigned prev = (unsigned)g_fit_plan_debug;
    g_fit_plan_debug = mode <= 3 ? (int)mode : 0;
    return prev;
}

size_t pmg_fit_final_workspace_bytes(int B, int dh, int dw, int iters) {
    if (B < 1 || dh < 1 || dw < 1) return 0;
    return final_fit_workspace_bytes(B, dh, dw, iters);
}

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

int pmg_post_depth(const float* logz, int64_t stride, const uint8_t* mask, int B, int H, int W, const float* st,
                   float* depth, void* stream) {
    PMG_REQUIRE(logz && st && depth, "null buffer");
    PMG_REQUIRE(B >= 1 && H >= 1 && W >= 1 && stride >= 1, "bad shape");
    const int64_t HW = (int64_t)H * W, n = (int64_t)B * HW;
    hipLaunchKernelGGL(post_depth_k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, logz,
                       stride, mask, HW, n, st, depth);
    return check_launch("post_depth_k");
}

int pmg_fit_final(const float* logz, int64_t stride, const float* lidar, const float* conf, const uint8_t* mask_binary,
                  int B, int H, int W, int dh, int dw, int iters, float trim, int min_points, float* st, int32_t* info,
                  void* workspace, size_t workspace_bytes, void* stream) {
    FinalFit f{logz, stride, lidar, conf, mask_binary, B, H, W, dh, dw, iters, trim, min_points, st, info,
               workspace, workspace_bytes};
    return launch_final_fit(f, (hipStream_t)stream);
}

}  // extern "C"
