/*
 * pmg.h -- C ABI of libpmg.so, the MI355X (gfx950) implementation of PromptMoGe's sparse 3-D refiner step.
 *
 * Conventions
 *   - Every pointer argument named as a buffer is a DEVICE pointer owned by the caller, except where a comment says
 *     "host". Nothing here allocates device memory except pmg_refiner_create (its persistent workspace).
 *   - Every call is asynchronous on `stream` (a hipStream_t, NULL = the legacy default stream) and returns an int
 *     status: PMG_OK, or an error code with a message available from pmg_last_error() (thread-local).
 *   - Shapes are validated on the host before any launch; a launch whose shape the kernel does not support is
 *     refused with PMG_E_INVALID, never attempted.
 *   - Voxel index conventions follow the reference: M voxels in raster (b, i, j) order at level 0; a neighbour map
 *     entry is the row index of the neighbour or -1; tap v = (di+1)*9 + (dj+1)*3 + (dz+1) for the 27 offsets of
 *     make_conv_kernel_delta (promptmoge/_fallback/flex_gemm/_core.py:65-82), so the centre tap is v = 13.
 *
 * Which reference interface each entry point replaces is given with file:line into the reference tree.
 */
#ifndef PMG_H
#define PMG_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    PMG_OK = 0,
    PMG_E_INVALID = 1,  /* bad argument or unsupported shape (reference: assert / ValueError, _core.py:324, 351) */
    PMG_E_HIP = 2,      /* a HIP runtime call failed */
    PMG_E_OVERFLOW = 3, /* a capacity was exceeded; the caller grows and retries (VoxelStructure.swift:200-216) */
    PMG_E_DEVICE = 4    /* a kernel reported an error through its device flag (e.g. a bounded wait expired) */
};

/* Message of the last failed call on this thread ("" if none). */
const char* pmg_last_error(void);
/* ABI version, bumped on any signature change. */
int pmg_version(void);

/* ------------------------------------------------------------------------------------------------------------ *
 * Numerics test hooks: evaluate the shared bit-reproducible fp32 functions (exp, log, silu) on the host CPU or on
 * the GPU, so tests can show that both and the NumPy oracle produce identical bits. op: 0 exp, 1 log, 2 silu;
 * device only, op 3: in = n pairs (y, mult), out[i] = the int8 code clamp(rint(silu(y) * mult), +-127) as the
 * epilogues compute it (hardware exp2/rcp with an exact re-evaluation near rounding ties).
 * ------------------------------------------------------------------------------------------------------------ */
int pmg_math_host(int op, const float* in_host, float* out_host, int64_t n);
int pmg_math_device(int op, const float* in, float* out, int64_t n, void* stream);

/* Peak probes (no counterpart in the reference): the device's practical rates with the kernels' instruction forms,
 * for reporting kernels against measured as well as published peaks. pmg_probe_copy streams `bytes` from src to
 * dst (16-byte vectors); pmg_probe_mfma_i8 runs iters x 16 independent v_mfma_i32_16x16x64_i8 per wave on
 * waves_per_cu waves per CU (32768 * 16 * iters int8 ops per wave); sink receives nothing but must be valid. The
 * caller times them with events on `stream`. */
int pmg_probe_copy(const void* src, void* dst, int64_t bytes, void* stream);
int pmg_probe_mfma_i8(int iters, int waves_per_cu, int32_t* sink, void* stream);

/* ------------------------------------------------------------------------------------------------------------ *
 * (1) Voxelisation -- replaces MoGeModel._voxelize (moge/model/v3.py:305-344).
 *   zq[b,i,j] = rint(logz[b,i,j] * resolution)       (round half to even, as torch.round; v3.py:332)
 *   zmin[b] = min over (i,j) of zq, zmax[b] = max     (v3.py:333-335; the z coordinate is zq - zmin[b] and the
 *                                                      z extent is max_b(zmax - zmin) + 1)
 * logz: [B*H*W] fp32 (the third channel of the point map, passed with its element stride `stride`, 1 for a plain
 * map, 3 for the (x/z, y/z, logz) point map). zq: [B*H*W] int32; zmin, zmax: [B] int32.
 * ------------------------------------------------------------------------------------------------------------ */
int pmg_voxelize(const float* logz, int64_t stride, int B, int H, int W, float resolution, int32_t* zq,
                 int32_t* zmin, int32_t* zmax, void* stream);

/* ------------------------------------------------------------------------------------------------------------ *
 * (2) Submanifold neighbour maps.
 *
 * pmg_nmap_column -- the level-0 column stencil, replaces _build_submanifold_nmap_column (_core.py:269-295):
 *   nmap[(b,i,j), v] = flat(b, i+di, j+dj) iff that pixel is in frame and zq there == zq[b,i,j] + dz, else -1.
 * Outputs (each may be NULL):
 *   nmap_t    [27][M] int32, tap-major (the layout the convolutions read)
 *   nmap_rows [M][27] int32, the reference's row-major (M, 27) layout
 *   tile_mask [ceil(M/16)] uint32: bit v set iff any of the tile's 16 rows has tap v
 *   coords    [M][4] int32 (b, i, j, zq - zmin[b]), the reference's coords (v3.py:337-340); needs zmin
 * ------------------------------------------------------------------------------------------------------------ */
int pmg_nmap_column(const int32_t* zq, const int32_t* zmin, int B, int H, int W, int32_t* nmap_t,
                    int32_t* nmap_rows, uint32_t* tile_mask, int32_t* coords, void* stream);

/* pmg_nmap_hash -- generic coordinates, replaces _SortedIndex + _build_submanifold_nmap_sorted
 * (_core.py:105-124, 298-304) with an open-addressing GPU hash of 4x4x4 bricks keyed by _linearise
 * (_core.py:89-94) on the brick grid. coords: [M][4] int32 (b, x, y, z), unique, inside sparse_shape (host array
 * of 4 int64); M < 2^30. Same outputs as pmg_nmap_column (coords excluded), plus row_mask [M] uint32 (bit v set
 * iff row m has tap v; may be NULL). The workspace (any contents) holds the table: 8 + 256 bytes per bucket,
 * buckets = a power of two >= 1.5 M. */
size_t pmg_hash_workspace_bytes(int64_t M);
int pmg_nmap_hash(const int32_t* coords, int64_t M, const int64_t* sparse_shape_host, int32_t* nmap_t,
                  int32_t* nmap_rows, uint32_t* tile_mask, uint32_t* row_mask, void* workspace,
                  size_t workspace_bytes, void* stream);

/* pmg_nmap_sorted -- pmg_nmap_hash for coordinates in strictly increasing _linearise order (_core.py:89-94): the
 * order of _SortedIndex's sorted keys (_core.py:105-124, which sorts them itself) and of the voxel sets that
 * voxelisation and pool caches produce. Same outputs as pmg_nmap_hash, found through a dense table of the (b, x, y)
 * columns' row runs instead of a hash. The precondition is checked on the device: a row outside sparse_shape or
 * not after its predecessor sets bit 0 of the status word (the first 4 bytes of the workspace), and the outputs
 * are then not valid. Workspace: pmg_sorted_workspace_bytes(sparse_shape) bytes (0: more than 2^31 columns),
 * 16-byte aligned; its status word must be zero before the first call and is never cleared by a call (sticky);
 * the rest may hold anything. Calls that share a workspace must not overlap. M < 2^31 - 1. */
size_t pmg_sorted_workspace_bytes(const int64_t* sparse_shape_host);
int pmg_nmap_sorted(const int32_t* coords, int64_t M, const int64_t* sparse_shape_host, int32_t* nmap_t,
                    int32_t* nmap_rows, uint32_t* tile_mask, uint32_t* row_mask, void* workspace,
                    size_t workspace_bytes, void* stream);

/* pmg_row_order -- a processing order for pmg_spconv_i8_ordered (no counterpart in the reference; it changes no
 * result): within each window of `window` consecutive rows (0: one window), the rows sorted, stably, by their
 * 27-bit tap mask (row_mask [M], bit v = tap v present, as pmg_nmap_hash writes it), so that the tiles and chunks
 * of the convolution run few taps while a window's rows stay in one part of the volume and rows of one
 * neighbourhood pattern keep the caller's order. order [M] int32 = row indices in processing order;
 * order_tile_mask [ceil(M/16)] = the union of the tap masks of order[16t .. 16t+15]; nmap_o [27][M] (optional,
 * with nmap_rows, the row-major (M, 27) map pmg_nmap_hash writes) = the tap-major map in processing order,
 * nmap_o[v][p] = nmap_rows[order[p]][v] -- the map pmg_spconv_i8_ordered reads. Workspace:
 * pmg_row_order_workspace_bytes(M) (any contents). M < 2^31. */
size_t pmg_row_order_workspace_bytes(int64_t M);
int pmg_row_order(const uint32_t* row_mask, const int32_t* nmap_rows, int64_t M, int64_t window, int32_t* order,
                  uint32_t* order_tile_mask, int32_t* nmap_o, void* workspace, size_t workspace_bytes, void* stream);

/* pmg_pool_cache -- build_pool_cache (promptmoge/_fallback/flex_gemm/_core.py:339-395) for the perfect-partition
 * pool MoGe uses (kernel == stride, padding 0), output coordinates not given: the output voxels are the distinct
 * floor(coords / stride) in increasing _linearise order on the output grid (_core.py:89-94). coords [M][4] int32
 * (b, x, y, z) inside sparse_shape (host int64[4]); stride host int32[3]; out_sparse_shape host int64[4] (the
 * batch extent unchanged). Outputs (device, capacity M): out_coords [num_out][4], parent [M] (input row -> output
 * row), seg_indices [M] (stable argsort of parent), seg_offsets [num_out + 1] (int64); counts [2] int64 on the
 * device: num_out, and the number of input voxels outside sparse_shape (then the cache is not valid). */
size_t pmg_pool_cache_workspace_bytes(int64_t M);
int pmg_pool_cache(const int32_t* coords, int64_t M, const int64_t* sparse_shape, const int32_t* stride,
                   const int64_t* out_sparse_shape, int32_t* out_coords, int32_t* parent, int32_t* seg_indices,
                   int64_t* seg_offsets, int64_t* counts, void* workspace, size_t workspace_bytes, void* stream);

/* pmg_sparse_pool -- sparse_pool (_core.py:444-481) on a pool cache: out[r] = sum of feats[seg_indices[k]],
 * k in [seg_offsets[r], seg_offsets[r+1]), accumulated in that (input) order in fp32 like the reference's
 * index_add_, divided by the group size for reduce = 1 ('mean'); reduce = 0 is 'sum'. feats [M][C] fp32, C a
 * multiple of 4; out [num_out][C]. */
int pmg_sparse_pool(const float* feats, int64_t M, int C, const int32_t* seg_indices, const int64_t* seg_offsets,
                    int64_t num_out, int reduce, float* out, void* stream);

/* pmg_sparse_upsample -- sparse_upsample 'nearest' (_core.py:484-505) with the transposed pool cache:
 * out[i] = feats[parent[i]] for rows of row_bytes bytes (a multiple of 16; any element type). */
int pmg_sparse_upsample(const void* feats, int64_t row_bytes, const int32_t* parent, int64_t rows_out, void* out,
                        void* stream);

/* pmg_nmap_from_rows -- a caller-supplied (M, 27) map (a NeighborCache.nmap, _core.py:131-176) into the tap-major
 * layout and tile masks the convolutions read. */
int pmg_nmap_from_rows(const int32_t* nmap_rows, int64_t M, int32_t* nmap_t, uint32_t* tile_mask, void* stream);

/* pmg_kmap_compact -- the 27 offset-major kernel maps, compacted: for each tap v, the output rows that have a
 * neighbour at v in ascending order and the neighbour rows, exactly the reference's per-tap
 * `rows = valid.nonzero()` and `src = idx[rows]` (_core.py:430-437).
 *   offsets [28] int64 (device): tap v occupies [offsets[v], offsets[v+1]) of out_rows / in_rows
 *   out_rows, in_rows: int32, capacity entries each (27*M always suffices)
 * Returns PMG_E_OVERFLOW (after writing offsets) if the total exceeds capacity. */
size_t pmg_kmap_workspace_bytes(int64_t M);
int pmg_kmap_compact(const int32_t* nmap_t, int64_t M, int64_t* offsets, int32_t* out_rows, int32_t* in_rows,
                     int64_t capacity, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------------------------ *
 * (3) Submanifold 3x3x3 convolutions, output-stationary implicit GEMM on MFMA, replacing submanifold_conv
 * (_core.py:399-441):  out[m, n] = bias[n] + sum_v sum_c W[n, v, c] * x[nmap[v][m], c].
 * Weights are in the reference module's own layout, (Co, 3, 3, 3, Ci) = [Co][27][Ci] (nn/__init__.py:30).
 * Ci and Co must be multiples of 16 (int8, fp16) or of 4 and 16 (fp32). tile_mask must come from the same map.
 *
 * int8 (the deployed contract, moge/model/modules/qat.py:1-16 and SparseConvInt8.metal:36-142):
 *   acc = sum int8*int8 in int32, then by epilogue
 *     PMG_EPI_ACC   out int32 [M][Co] = acc                                          (parity dump)
 *     PMG_EPI_Q     out int8  [M][Co] = quant(silu((acc*a_scale)*w_scale[n] + bias[n]), out_mult)
 *     PMG_EPI_R     out fp32  [M][Co] = ((acc*a_scale)*w_scale[n] + bias[n]) + skip[m][n]   (skip may alias out)
 *     PMG_EPI_BIAS  out fp32  [M][Co] = (acc*a_scale)*w_scale[n] + bias[n]
 *     PMG_EPI_QLIN  out int8  [M][Co] = quant((acc*a_scale)*w_scale[n] + bias[n], out_mult), no activation: with
 *                   a_scale = out_mult = 1 and no bias, the plain per-channel requantisation clamp(rint(acc*m[n]))
 *   a_scale = clip/127 of the input activation, w_scale per output channel; quant(y, mult) =
 *   clamp(rint(y * mult), -127, 127) with mult = 127/clip of the output activation, the requantisation of the
 *   reference's deployed kernels (SparseConvInt8.metal:109; mult computed as in Refiner.swift:148).
 * fp16 (teacher; fp32 accumulation): PMG_EPI_ACC / PMG_EPI_BIAS -> fp32 [M][Co] = acc (+ bias[n]);
 *   PMG_EPI_SILU -> fp16 [M][Co] = half(silu(acc + bias[n])); PMG_EPI_R -> fp32 = (acc + bias[n]) + skip.
 * fp32 (the flex_gemm shim on fp32 features): PMG_EPI_ACC / PMG_EPI_BIAS -> fp32.
 * bias may be NULL (zero).
 * ------------------------------------------------------------------------------------------------------------ */
enum { PMG_EPI_ACC = 0, PMG_EPI_Q = 1, PMG_EPI_R = 2, PMG_EPI_BIAS = 3, PMG_EPI_SILU = 4, PMG_EPI_RLN = 5,
       PMG_EPI_ROUT = 6, PMG_EPI_QLIN = 7 };

int pmg_spconv_i8(const int8_t* x, const int32_t* nmap_t, const uint32_t* tile_mask, int64_t M, int Ci, int Co,
                  const int8_t* w, int epilogue, float a_scale, const float* w_scale, const float* bias,
                  float out_mult, const float* skip, void* out, void* stream);
/* pmg_spconv_i8 with the rows processed in `order` (pmg_row_order): nmap_o is the map in processing order
 * (pmg_row_order's nmap_o) and order_tile_mask its tile masks; output row order[p] is computed from map column p.
 * The same results as pmg_spconv_i8 on the caller's map, with each chunk of rows running only its rows' taps.
 * Ci = Co = 64 or 128. */
int pmg_spconv_i8_ordered(const int8_t* x, const int32_t* nmap_o, const int32_t* order,
                          const uint32_t* order_tile_mask, int64_t M, int Ci, int Co, const int8_t* w, int epilogue,
                          float a_scale, const float* w_scale, const float* bias, float out_mult, const float* skip,
                          void* out, void* stream);
int pmg_spconv_f16(const uint16_t* x, const int32_t* nmap_t, const uint32_t* tile_mask, int64_t M, int Ci, int Co,
                   const uint16_t* w, int epilogue, const float* bias, const float* skip, void* out, void* stream);
int pmg_spconv_f32(const float* x, const int32_t* nmap_t, const uint32_t* tile_mask, int64_t M, int Ci, int Co,
                   const float* w, int epilogue, const float* bias, float* out, void* stream);
/* bf16 features and weights (the refiner under bf16 autocast, sparse_unet.py:155-158, through
 * submanifold_conv, _core.py:399-441): bf16 MFMA with fp32 accumulation, fp32 output; epilogues ACC, BIAS and R.
 * ABI version 4. */
int pmg_spconv_bf16(const uint16_t* x, const int32_t* nmap_t, const uint32_t* tile_mask, int64_t M, int Ci, int Co,
                    const uint16_t* w, int epilogue, const float* bias, const float* skip, float* out, void* stream);

/* pmg_spconv_col -- the level-0 convolution computed straight from the voxel keys zq [B][H][W] (pmg_voxelize),
 * with the column-stencil neighbourhood of _build_submanifold_nmap_column (_core.py:269-295) derived on the fly
 * (no neighbour map is read), as one fused layer of the residual block (flex_sparse_blocks.py:229-234):
 *   precision PMG_PREC_INT8: x int8 [M][C], w int8 [C][27][C]; PMG_PREC_FP16: x, w fp16.
 *   PMG_EPI_ACC   out int32 (int8) / fp32 (fp16) [M][C] = acc
 *   PMG_EPI_Q     int8: out int8 = quant(silu((acc*a_scale)*w_scale[n] + bias[n]), out_mult);
 *                 fp16: out fp16 = half(silu(acc + bias[n]))
 *   PMG_EPI_R     out fp32 = y + skip, y = (acc*a_scale)*w_scale[n] + bias[n] (int8) or acc + bias[n] (fp16)
 *   PMG_EPI_RLN   as R, and next_q [M][C] = quant(silu(LayerNorm(out) * ln_gamma + ln_beta), next_mult) (int8) or
 *                 half(silu(...)) (fp16): the next block's input (out may alias skip)
 *   PMG_EPI_ROUT  as R without storing it; delta = out_b + out_w . x_new; then points_out[m] = (points[m].xy,
 *                 points[m].z + delta), or, with points NULL, out fp32 [M] = delta (the refiner module's output)
 * LayerNorm and the out_proj dot product sum in a fixed order: channels n = 16j + 4g + i are summed per group g
 * (j outer, i inner) and the four group sums combined as ((s0 + s1) + (s2 + s3)). C in {16, 32, 48, 64, 128}. */
typedef struct {
    float a_scale;         /* int8: input activation scale clip/127 */
    const float* w_scale;  /* int8: [C] per-output-channel weight scale */
    const float* bias;     /* [C] or NULL */
    float out_mult;        /* PMG_EPI_Q (int8): requantisation multiplier 127/clip of the output */
    const float* skip;     /* residual epilogues: [M][C] fp32 */
    void* out;             /* main output (PMG_EPI_ROUT: the [M] delta when points is NULL) */
    const float* ln_gamma; /* PMG_EPI_RLN: next block's LayerNorm affine [C] */
    const float* ln_beta;
    float ln_eps;
    float next_mult;  /* int8: 127/clip of the next block's conv1 input */
    void* next_q;     /* [M][C] int8 or fp16 */
    const float* out_w; /* PMG_EPI_ROUT: out_proj weight [C] and bias [1] */
    const float* out_b;
    const float* points; /* [M][3] input point map, or NULL (PMG_EPI_ROUT writes delta to out) */
    float* points_out;   /* [M][3] refined point map (may alias points) */
} pmg_conv_epilogue;

int pmg_spconv_col(int precision, const void* x, const int32_t* zq, int B, int H, int W, int C, const void* w,
                   int epilogue, const pmg_conv_epilogue* e, void* stream);

/* ------------------------------------------------------------------------------------------------------------ *
 * Row operations of the residual block (SparseResBlock3d, moge/model/modules/flex_sparse_blocks.py:70-75;
 * device design Refiner.metal:75-131).
 *   pmg_ln_silu_quant: q[m] = quant(silu(LayerNorm(x[m]) * gamma + beta), out_mult)   -> int8 [M][C]
 *   pmg_ln_silu_f16:   h[m] = half(silu(LayerNorm(x[m]) * gamma + beta))                -> fp16 [M][C]
 * LayerNorm is two-pass (mean, then mean of squared deviations), eps inside the sqrt, with the sums in the order of
 * pmg_spconv_col's PMG_EPI_RLN (per group g of channels 16j+4g+i, then ((s0 + s1) + (s2 + s3))).
 * C in {16, 32, 48, 64, 96, 128}.
 * ------------------------------------------------------------------------------------------------------------ */
int pmg_ln_silu_quant(const float* x, int64_t M, int C, const float* gamma, const float* beta, float eps,
                      float out_mult, int8_t* q, void* stream);
int pmg_ln_silu_f16(const float* x, int64_t M, int C, const float* gamma, const float* beta, float eps,
                    uint16_t* h, void* stream);

/* ------------------------------------------------------------------------------------------------------------ *
 * (4) Robust metric fit -- replaces fit_scale_shift (moge/model/modules/prompt_stem.py:211-240): trimmed least
 * squares target ~= s*z + t on mask, `iters` trim rounds then a final solve; k = max(long(fp32(1-trim)*count),
 * min_points) and the trim threshold is the exact k-th smallest relative residual (torch.kthvalue), selected
 * inside a bracket around the previous round's threshold, or by radix passes when it leaves the bracket; (1, 0)
 * when fewer than min_points mask pixels. Sums in fp64, one persistent kernel per batch item with device-wide
 * barriers, no host round trip.
 *   z, target: [B][N] fp32; mask: [B][N] uint8 (0/1); st: [B][2] fp32 (s, t) written on device.
 *   info (may be NULL): [B][5] int32 = (count, k, ok, threshold bits of the last trim round, device error flag:
 *   nonzero if a bounded device-wide wait expired -- the grid was not co-resident -- in which case (s, t) = NaN).
 *   workspace: pmg_fit_workspace_bytes(N, iters) bytes, zero-filled before its first use; every call leaves it
 *   ready for the next one, also after an expired wait (calls that share a workspace must be ordered, e.g. on one
 *   stream).
 * N <= 2^21 per batch item.
 * ------------------------------------------------------------------------------------------------------------ */
size_t pmg_fit_workspace_bytes(int64_t N, int iters);
/* pmg_fit_scale_shift_static -- pmg_fit_scale_shift without a workspace argument and without allocating. It has
 * no counterpart in the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc). The workspace is a static 14 MiB device array that each
 * GPU the library runs on holds until the process ends; it limits N to 2^19 per batch item and iters to 16 (larger
 * sizes are refused with PMG_E_INVALID). Results are those of pmg_fit_scale_shift bit for bit. Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams, other threads) race; order them. */
int pmg_fit_scale_shift_static(const float* z, const float* target, const uint8_t* mask, int B, int64_t N, int iters,
                               float trim, int min_points, float* st, int32_t* info, void* stream);
/* Test hook (no counterpart in the reference): polls of one device-wide wait before it expires, for the fits
 * enqueued after the call (0 restores the default, about 0.1 s). Returns the previous value. A tiny limit makes
 * waits expire with every kernel still running to its end, so tests can exercise the error path. */
unsigned pmg_debug_fit_spin_limit(unsigned polls);
/* Test hook (no counterpart in the reference): makes the metric fit's round plans wrong on purpose, for the fits
 * enqueued after the call, so that tests reach the selection's fallbacks -- 1: each predicted bracket moved just
 * above its range (a window on the side that holds the k-th follows its miss); 2: each plan a window above every
 * finite residual (the radix passes follow its miss); 3: windows of 2^21-key bins (split passes); 0 (or any other
 * value) restores the normal plan. Results do not depend on the plan. Returns the previous mode. ABI version 5. */
unsigned pmg_debug_fit_plan(unsigned mode);
int pmg_fit_scale_shift(const float* z, const float* target, const uint8_t* mask, int B, int64_t N, int iters,
                        float trim, int min_points, float* st, int32_t* info, void* workspace,
                        size_t workspace_bytes, void* stream);

/* The prompt fit of MoGeModel._lidar_in_affine_frame (v3.py:362-383), prepared on the fly: z = exp(logz) on the
 * H x W map (logz with element stride `stride`), target = nearest-resized LiDAR (F.interpolate 'nearest' index
 * rule), mask = finite(d) & d > 0 & clamp(conf/2, 0, 1) >= 0.999. lidar, conf: [B][dh][dw] fp32. */
int pmg_fit_prompt(const float* logz, int64_t stride, const float* lidar, const float* conf, int B, int H, int W,
                   int dh, int dw, int iters, float trim, int min_points, float* st, int32_t* info,
                   void* workspace, size_t workspace_bytes, void* stream);

/* The final metric fit of MoGeModel.forward (v3.py:768-778, metric_from='lidar_ls'), at LiDAR resolution:
 * d_lr = F.interpolate(depth, (dh, dw), mode='area') of depth z = exp(logz) on the H x W map (adaptive average
 * pooling: fp32 window sum in row-major order / height / width), mask = conf >= 2 & lidar > 0 & d_lr > 0, and
 * with mask_binary ([B][H][W] uint8, or NULL) also area-pooled mask_binary > 0.99; then fit (s, t) of
 * lidar ~= s*d_lr + t as pmg_fit_scale_shift. The workspace (pmg_fit_final_workspace_bytes) must be zero-filled
 * before its first use and is reusable afterwards. */
size_t pmg_fit_final_workspace_bytes(int B, int dh, int dw, int iters);
int pmg_fit_final(const float* logz, int64_t stride, const float* lidar, const float* conf, const uint8_t* mask_binary,
                  int B, int H, int W, int dh, int dw, int iters, float trim, int min_points, float* st, int32_t* info,
                  void* workspace, size_t workspace_bytes, void* stream);

/* pmg_post_depth -- the metric depth after the final fit (post_depth, MetricFit.metal:200-211; v3.py:776):
 * depth[b,i,j] = s[b] * exp(logz[b,i,j]) + t[b] in fp32, +inf where mask[b,i,j] == 0 (mask [B][H][W] uint8, the
 * model's mask, or NULL: all pixels) or where that depth is not > 0. logz with element stride `stride` (3 for the
 * point map); st [B][2] (the final fit's output, read on the device); depth [B][H][W] fp32. */
int pmg_post_depth(const float* logz, int64_t stride, const uint8_t* mask, int B, int H, int W, const float* st,
                   float* depth, void* stream);

/* ------------------------------------------------------------------------------------------------------------ *
 * (5) LiDAR prompt fill.
 *
 * pmg_nearest_fill -- replaces nearest_fill (promptmoge/model.py:61-72): every pixel with depth <= 0 (or NaN)
 * takes the depth of the nearest valid pixel and conf 1; valid pixels keep depth and conf; an image with no
 * valid pixel is left as it is. "Nearest" is scipy.ndimage.distance_transform_edt's feature transform: least
 * Euclidean distance, ties to the smallest column, then the smallest row -- the result is exact.
 * depth, conf: [B][h][w] fp32 (conf may be NULL together with conf_out); depth_out / conf_out may alias them.
 * src_index: [B][h][w] int32 flat index i*w + j of each pixel's source within its image (-1: no valid pixel),
 * or NULL. h, w <= 8192. The workspace (pmg_nearest_fill_workspace_bytes) needs no initialisation.
 * ------------------------------------------------------------------------------------------------------------ */
size_t pmg_nearest_fill_workspace_bytes(int B, int h, int w);
int pmg_nearest_fill(const float* depth, const float* conf, int B, int h, int w, float* depth_out, float* conf_out,
                     int32_t* src_index, void* workspace, size_t workspace_bytes, void* stream);

/* pmg_gauge_poly -- replaces MoGeModel.prompt_gauge_poly (moge/model/v3.py:151-183), the per-frame prompt gauge
 * that infer applies by default (gauge_poly=2, v3.py:841-853): corr[b] = exp(poly(u, v)) with (u, v) on
 * linspace(-1, 1) grids, the polynomial (1, u, v) for degree 1 or (1, u, v, u^2, uv, v^2) for degree >= 2 fitted
 * by `iters` IRLS rounds to log(max(lidar, 1e-3)) - log(max(z_lr, 1e-3)) on the pixels with conf >= 2, lidar > 0
 * and z_lr > 0, z_lr the area-pooled valid (finite, > 0) depth; fewer than 200 such pixels or a singular /
 * non-finite system give corr 1. depth: [B][H][W] fp32; lidar, conf: [B][h][w] fp32 (conf NULL: all 2);
 * corr: [B][H][W] fp32 out; coef: [B][8] fp32 out (the coefficients in basis order, [7] = 1 if the frame was
 * fitted, else 0). iters in [1, 64]. The workspace (pmg_gauge_poly_workspace_bytes) needs no initialisation.
 */
size_t pmg_gauge_poly_workspace_bytes(int B, int h, int w);
int pmg_gauge_poly(const float* depth, int B, int H, int W, const float* lidar, const float* conf, int h, int w,
                   int degree, int iters, float* corr, float* coef, void* workspace, size_t workspace_bytes,
                   void* stream);

/* ------------------------------------------------------------------------------------------------------------ *
 * The fused refiner step -- replaces one iteration of the refine loop (v3.py:547-576) for a single-level
 * refiner: prompt fit -> prompt residual/gate -> voxelise -> column neighbour map -> input_proj (+ prompt_proj)
 * -> n_blocks residual blocks (LN, SiLU, conv1, SiLU, conv2, + skip) -> out_proj -> logz += delta
 * (_refine_logz, v3.py:346-360; scaled by the output gate if configured) -> optionally the elastic anchor (a
 * second prompt-style fit on the refined depth, then the per-pixel pull toward the LiDAR, v3.py:570-573), then
 * optionally the metric fit on the refined depth. All on `stream`, no host
 * synchronisation; the sequence is captured once into a HIP graph and replayed while the buffers and the stream
 * are unchanged (on the legacy default stream, which cannot be captured, it is enqueued eagerly).
 * ------------------------------------------------------------------------------------------------------------ */
enum { PMG_PREC_INT8 = 0, PMG_PREC_FP16 = 1 };

typedef struct {
    int B, H, W;            /* point-map batch and size; M = B*H*W voxels at level 0 */
    int C;                  /* refiner width (16 .. 128, multiple of 16) */
    int n_blocks;           /* residual blocks; conv layers = 2 * n_blocks */
    int precision;          /* PMG_PREC_INT8 or PMG_PREC_FP16 */
    float depth_resolution; /* refiner_depth_resolution (v3.py:29), 256 */
    int dh, dw;             /* LiDAR map size */
    int fit_iters;          /* trim rounds of each fit */
    float fit_trim;         /* 0.2 */
    int fit_min_points;     /* 32 */
    int use_prompt;         /* feed (residual, gate) through prompt_proj (v3.py:549-555) */
    int soft_gate;          /* soft_residual_gate (v3.py:379-382) */
    int final_fit;          /* also run the final metric fit (pmg_fit_final) on the refined depth */
    int use_graph;          /* capture the step into a HIP graph and replay it */
    int output_gate;        /* refiner_output_gate (v3.py:565-569): logz + g * delta, g = floor + (1 - floor) * u,
                               u the LiDAR uncertainty of the pixel (v3.py:386-393) */
    float output_gate_floor;/* output_gate_floor, 0.1 */
    float anchor;           /* anchor_strength beta (v3.py:570-573): after the update, logz moves by
                               beta * gate * (log_d_aff - logz) with the LiDAR re-fitted to the refined depth; 0 = off */
} pmg_refiner_config;

typedef struct {
    const float* ln_gamma; /* [C] */
    const float* ln_beta;  /* [C] */
    const void* w1;        /* conv1 [C][27][C], int8 or fp16 by precision */
    const float* w1_scale; /* [C] per-output-channel weight scale (int8 only) */
    const float* b1;       /* [C] */
    float a1_scale;        /* conv1 input activation scale clip1/127 (int8 only) */
    float q1_mult;         /* 127/clip1: quantises conv1's input (int8 only) */
    const void* w2;
    const float* w2_scale;
    const float* b2;
    float a2_scale; /* clip2/127 */
    float q2_mult;  /* 127/clip2: conv1's requantisation into conv2's input */
} pmg_block_weights;

typedef struct {
    const float* in_w;  /* input_proj weight [C][3] */
    const float* in_b;  /* [C] */
    const float* pr_w;  /* prompt_proj weight [C][2] (NULL if !use_prompt) */
    const float* pr_b;  /* [C] */
    const float* out_w; /* out_proj weight [1][C] */
    const float* out_b; /* [1] */
    int n_blocks;
    const pmg_block_weights* blocks; /* host array of n_blocks; the pointers inside are device pointers */
} pmg_refiner_weights;

typedef struct pmg_refiner pmg_refiner;

pmg_refiner* pmg_refiner_create(const pmg_refiner_config* cfg);
void pmg_refiner_destroy(pmg_refiner* r);
int pmg_refiner_set_weights(pmg_refiner* r, const pmg_refiner_weights* w);
/* points: [B][H][W][3] (x/z, y/z, logz) input; points_out: the same map with the refined logz (may alias points,
 * the reference loop's `current_coord = cat(xy, refined_logz)`, v3.py:574). lidar, conf: [B][dh][dw] fp32.
 * st_prompt: [B][2] prompt-fit (s, t) or NULL; st_final: [B][2] or NULL. */
int pmg_refiner_step(pmg_refiner* r, const float* points, float* points_out, const float* lidar, const float* conf,
                     float* st_prompt, float* st_final, void* stream);
/* The refiner module alone -- Sparse3DUNet.forward (moge/model/modules/sparse_unet.py:176-258) for a single-level
 * refiner, the call _refine_logz makes at v3.py:356-357: out = out_proj(blocks(input_proj(feats) +
 * prompt_proj(prompt_feats))), (M, 1). feats: [M][3] fp32 (the point map reshaped, v3.py:342), M = B*H*W in
 * raster order; coords: [M][4] int32 (b, i, j, z) as _voxelize builds them (v3.py:337-340) -- only the z column
 * is read, as the key of the level-0 stencil -- or NULL to key by rint(feats[:, 2] * depth_resolution), the same
 * key up to a per-batch offset; prompt_feats: [M][2] fp32 or NULL (then no prompt_proj, sparse_unet.py:191);
 * out: [M] fp32. No fit runs. Captured into a HIP graph per (buffers, stream) like pmg_refiner_step. */
int pmg_refiner_forward(pmg_refiner* r, const float* feats, const int32_t* coords, const float* prompt_feats,
                        float* out, void* stream);
/* Synchronises `stream` and reports a device-side error flag of the last steps (PMG_E_DEVICE). */
int pmg_refiner_check(pmg_refiner* r, void* stream);
/* Device buffers of the last step, for parity tests: 0 zq (voxel keys [M]), 3 x (fp32 residual [M][C] entering the
 * last block), 4 q1 (the last block's conv1 input codes), 5 q2 (its conv2 input codes). NULL for any other id. */
const void* pmg_refiner_buffer(pmg_refiner* r, int id);

/* ------------------------------------------------------------------------------------------------------------ *
 * The multi-level refiner -- Sparse3DUNet (moge/model/modules/sparse_unet.py:17-258) in the deployed int8
 * arithmetic (qat.py:1-16; the device engine's sequence Refiner.swift:224-292, Refiner.metal:133-322): input_proj
 * (+ prompt_proj) -> per level: SparseResBlock3d stage, PoolDown (mean pool, int8 linear) -> encoder conditioning
 * (encoder_fuse on the token grid + encoder_bias_map, gathered by column) -> fuse_proj (int8 linear, SiLU, int8
 * linear) -> bottleneck stage -> per level: NearestUp (int8 linear at the coarse level, upsample, + skip), stage ->
 * out_proj. Level structure: level 0 = one voxel per pixel (raster order); level k+1 = the stride-2 perfect-partition
 * pool of level k (flex_sparse_blocks.py:78-90, _core.py:339-395), voxels in (b, i, j, z) order; submanifold maps per
 * level (_core.py:269-304). Every level is built and sized on the device: no host synchronisation, the forward is
 * captured into a HIP graph per (buffers, stream). Buffers are allocated for B*H*W voxels on every level.
 * ------------------------------------------------------------------------------------------------------------ */
typedef struct {
    int B, H, W;            /* point map; level 0 = B*H*W voxels; H, W multiples of 2^(levels-1) */
    int levels;             /* len(model_channels), 2 .. 8; downsample factors 2 (encoder_downsample 2^(levels-1)) */
    int channels[8];        /* model_channels: level 0 in {16, 32, 48, 64, 128}; others in {16, 32, 48, 64, 96,
                               128, 192, 256} */
    int enc_blocks[8];      /* encoder_blocks_per_level (down_stages[k]) */
    int dec_blocks[8];      /* decoder_blocks_per_level: dec_blocks[i] is up_stages[i], at level levels-2-i; the last
                               (level 0) needs >= 1 block (out_proj runs in its last convolution's epilogue) */
    int bottleneck_blocks;
    int enc_channels;       /* encoder_fuse in_features (multiple of 16) */
    float depth_resolution; /* refiner_depth_resolution (v3.py:29): keys when no coords are given */
    int use_graph;
    int precision;          /* PMG_PREC_INT8 (the deployed refiners) or PMG_PREC_FP16 (the teacher, PromptMoGe-L:
                               fp16 activations and weights in every conv and linear, fp32 accumulation, fp32
                               residual streams; level widths up to 512, level 0 16 .. 64) */
} pmg_unet_config;

typedef struct {
    const void* w;        /* [N][K], nn.Linear's (out, in) layout: int8, or fp16 with PMG_PREC_FP16 */
    const float* w_scale; /* [N] per-output-channel weight scale (int8 only) */
    const float* bias;    /* [N] */
    float a_scale;        /* clip/127 of the input activation (int8 only) */
    float q_mult;         /* 127/clip: quantises the input (int8 only) */
} pmg_linear_weights;

typedef struct {
    const float* in_w;  /* input_proj [C0][3], [C0] */
    const float* in_b;
    const float* pr_w;  /* prompt_proj [C0][2], [C0], or both NULL */
    const float* pr_b;
    const float* out_w; /* out_proj [C0], [1] */
    const float* out_b;
    int n_blocks;       /* sum(enc_blocks) + bottleneck_blocks + sum(dec_blocks) */
    const pmg_block_weights* blocks;   /* host array in module order: down_stages[0..L-1], bottleneck_stage,
                                          up_stages[0..L-2]; conv weights [C][27][C] int8 (fp16: fp16, and the
                                          scales and clips are not read) */
    int n_linears;      /* 2 (levels - 1) + 3 */
    const pmg_linear_weights* linears; /* host array: downsample_blocks[0..L-2].linear, encoder_fuse, fuse_proj.0,
                                          fuse_proj.2, upsample_blocks[0..L-2].linear */
} pmg_unet_weights;

typedef struct pmg_unet pmg_unet;

pmg_unet* pmg_unet_create(const pmg_unet_config* cfg);
void pmg_unet_destroy(pmg_unet* u);
/* Bytes of the context's device workspace (allocated by pmg_unet_create). */
size_t pmg_unet_workspace_bytes(const pmg_unet* u);
/* Voxel capacity of every level (B*H*W). */
int64_t pmg_unet_capacity(const pmg_unet* u);
int pmg_unet_set_weights(pmg_unet* u, const pmg_unet_weights* w);
/* Sparse3DUNet.forward (sparse_unet.py:176-258), the call _refine_logz makes (v3.py:356-357): feats [M][3] fp32 (the
 * point map reshaped, v3.py:342), M = B*H*W in raster order; coords [M][4] int32 (b, i, j, z) as _voxelize builds
 * them (v3.py:337-340) or NULL to voxelise feats[:, 2] with depth_resolution; prompt_feats [M][2] or NULL (no
 * prompt_proj, sparse_unet.py:191); encoder_feature [B][enc_channels][H/ds][W/ds] fp32 (ds = 2^(levels-1));
 * encoder_bias_map [B][C_{L-1}][H/ds][W/ds] fp32 or NULL (sparse_unet.py:235-239); out [M] fp32. */
int pmg_unet_forward(pmg_unet* u, const float* feats, const int32_t* coords, const float* prompt_feats,
                     const float* encoder_feature, const float* encoder_bias_map, float* out, void* stream);
/* Device buffers of the last forward, for parity tests: PMG_UNET_COUNTS int64 [levels] voxels per level;
 * PMG_UNET_COORDS [cap][4] int32 of `level`; PMG_UNET_PARENT [cap] int32, level -> level + 1; PMG_UNET_NMAP
 * [27][cap] int32 and PMG_UNET_TILE_MASK [cap/16] (levels >= 1); PMG_UNET_COL_OFFSETS the column CSR
 * [B*H_k*W_k + 1] int32 (levels >= 1); PMG_UNET_DOWN [cap][C] fp32, the down stage's output at `level`;
 * PMG_UNET_UP [cap][C] fp32, the up stage's (the bottleneck's at the deepest level); PMG_UNET_ENC_TOKENS
 * [B*(H/ds)*(W/ds)][C_{L-1}] fp32, encoder_fuse + bias map per token. NULL for an id the level does not have. */
enum { PMG_UNET_COUNTS = 0, PMG_UNET_COORDS = 1, PMG_UNET_PARENT = 2, PMG_UNET_NMAP = 3, PMG_UNET_TILE_MASK = 4,
       PMG_UNET_DOWN = 5, PMG_UNET_UP = 6, PMG_UNET_ENC_TOKENS = 7, PMG_UNET_COL_OFFSETS = 8, PMG_UNET_STEP_ST = 9 };
/* PMG_UNET_STEP_ST (any level): [3][B][2] fp32, the last pmg_unet_step's prompt, final and anchor fits (s, t) (the
 * prompt and final rows are written there only when the caller passes no st_prompt / st_final). */
const void* pmg_unet_buffer(pmg_unet* u, int id, int level);

/* ------------------------------------------------------------------------------------------------------------ *
 * One refine-loop step with the multi-level refiner: the body of the loop at moge/model/v3.py:547-576 around
 * _refine_logz (v3.py:346-360) with Sparse3DUNet (sparse_unet.py:176-258), in the device engine's order
 * (Refiner.swift:224-292) -- prompt fit (fit_scale_shift of _lidar_in_affine_frame, v3.py:362-378) -> per-voxel
 * (residual, gate) prompt features (v3.py:548-555) -> _voxelize (v3.py:305-344) -> level structure -> the U-Net ->
 * logz + out_proj (v3.py:359), optionally through the output gate (v3.py:565-569) -> optionally the elastic anchor
 * (v3.py:570-573) -> optionally the final metric fit at LiDAR resolution (v3.py:768-778) and post_depth
 * (MetricFit.metal:200-211). One stream, no host synchronisation, one captured HIP graph per (buffers, stream).
 * ------------------------------------------------------------------------------------------------------------ */
typedef struct {
    int dh, dw;              /* LiDAR map size */
    int fit_iters;           /* trim rounds of each fit (0 .. 64) */
    float fit_trim;          /* 0.2 */
    int fit_min_points;      /* 32 */
    int use_prompt;          /* prompt fit + (residual, gate) through prompt_proj; 0: no prompt features */
    int soft_gate;           /* soft_residual_gate (v3.py:379-382) */
    int output_gate;         /* refiner_output_gate (v3.py:565-569) */
    float output_gate_floor; /* 0.1 */
    float anchor;            /* anchor_strength beta in [0, 1] (v3.py:570-573); 0 = off */
    int final_fit;           /* the metric fit of the refined depth at LiDAR resolution */
} pmg_unet_step_config;

/* Sets the step options and allocates the step's own workspace (the fits'); captured steps are dropped. Call it
 * before the first pmg_unet_step and again to change the options; pmg_unet_step itself allocates nothing. */
int pmg_unet_step_prepare(pmg_unet* u, const pmg_unet_step_config* cfg);
/* points: [B][H][W][3] (x/z, y/z, logz) fp32; points_out: the same map with the refined logz (may alias points:
 * the loop's `current_coord = cat(xy, refined_logz)`, v3.py:574); lidar, conf: [B][dh][dw] fp32;
 * encoder_feature [B][enc_channels][H/ds][W/ds], encoder_bias_map [B][C_{L-1}][H/ds][W/ds] or NULL (as for
 * pmg_unet_forward); st_prompt, st_final: [B][2] or NULL; depth: [B][H][W] fp32 post_depth of the refined map with
 * the final fit's (s, t) (+inf where not > 0), or NULL (needs final_fit). */
int pmg_unet_step(pmg_unet* u, const float* points, float* points_out, const float* lidar, const float* conf,
                  const float* encoder_feature, const float* encoder_bias_map, float* st_prompt, float* st_final,
                  float* depth, void* stream);
/* Synchronises `stream`; reports (PMG_E_DEVICE) and clears a device-wide wait of a step's metric fit that expired. */
int pmg_unet_check(pmg_unet* u, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PMG_H */
