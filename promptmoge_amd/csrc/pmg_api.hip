// Error plumbing and the fused refiner step (pmg_refiner_*).
//
// The step is the refine-loop body of MoGeModel.forward (moge/model/v3.py:547-576) for a single-level refiner,
// in the order of the reference's device engine (Refiner.swift:224-292): prompt fit, then one fused input kernel
// (voxel keys, prompt residual/gate, input/prompt projections, first LayerNorm), then two convolutions per residual
// block that derive the level-0 neighbourhood from the keys (the second one also normalises for the next block, or
// applies out_proj and the log-depth update after the last block), then the optional metric fit of the refined
// depth. Everything is enqueued on one stream with no host synchronisation:
// at level 0 the voxel count is B*H*W, known on the host, so every grid is sized without reading the device.
// The enqueue sequence is captured once into a HIP graph and replayed while the caller's buffers are unchanged.
#include <climits>
#include <cstring>
#include <string>
#include <vector>

#include "pmg_common.h"
#include "pmg_graph.h"
#include "pmg_internal.h"

namespace pmg {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
    set_error(msg);
    return code;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(PMG_E_HIP, std::string(what) + ": launch failed: " + hipGetErrorString(e));
    return PMG_OK;
}

int num_cus() {
    static int cached[64];
    static bool init[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!init[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
        init[dev] = true;
    }
    return cached[dev];
}

}  // namespace pmg

using namespace pmg;

struct pmg_refiner {
    pmg_refiner_config cfg{};
    int64_t M = 0;
    bool have_weights = false;
    pmg_refiner_weights w{};
    std::vector<pmg_block_weights> blocks;

    void* arena = nullptr;
    size_t arena_bytes = 0;
    int32_t* zq = nullptr;
    int32_t* zmin = nullptr;
    int32_t* zmax = nullptr;
    float* x = nullptr;
    float* rg = nullptr;  // [M][2] prompt features of the step, for the first block's recomputed skip
    void* q1 = nullptr;
    void* q2 = nullptr;
    float* st_scratch = nullptr;
    void* fit_ws[2] = {nullptr, nullptr};
    size_t fit_ws_bytes[2] = {0, 0};  // prompt fit, final fit

    // Captured steps and forwards, keyed by (kind, buffers..., stream); a ping-pong of two point buffers over K
    // steps uses two entries.
    GraphCache graphs;
};

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Whether the first block's conv2 recomputes the input stage's h from the level-0 inputs instead of reading it
// (the int8 neighbour-pixel-major kernel, C <= 64, with a next block: its LayerNorm epilogue): the input stage then
// stores no h, and the first residual epilogue reads 20 bytes per row instead of 4 C.
static bool recompute_x0(const pmg_refiner* r) {
    return r->cfg.precision != PMG_PREC_FP16 && r->cfg.C <= 64 && r->blocks.size() >= 2;
}

// Residual blocks: conv1 (bias, SiLU, requantise) then conv2 (bias, skip, and either the next block's
// LayerNorm/SiLU/quantise or, after the last block, out_proj and either the log-depth update of the point map or
// the module's (M, 1) output). Expects q1 and either x from the input stage or, with x0_feats (recompute_x0), the
// level-0 features (and prompt features x0_rg, or NULL) from which the first block's skip is formed.
static int enqueue_blocks(pmg_refiner* r, const float* points, float* points_out, float* delta_out, hipStream_t s,
                          const float* gate_lidar, const float* gate_conf, const float* x0_feats,
                          const float* x0_rg) {
    const pmg_refiner_config& c = r->cfg;
    const int prec = c.precision == PMG_PREC_FP16 ? PMG_PREC_FP16 : PMG_PREC_INT8;
    const int64_t M = r->M;
    const int C = c.C;
    const int nbk = (int)r->blocks.size();
    for (int k = 0; k < nbk; ++k) {
        const pmg_block_weights& bk = r->blocks[k];
        ColConvArgs a1{};
        a1.x = r->q1;
        a1.zq = r->zq;
        a1.w = bk.w1;
        a1.M = M;
        a1.H = c.H;
        a1.W = c.W;
        a1.a_scale = bk.a1_scale;
        a1.w_scale = bk.w1_scale;
        a1.bias = bk.b1;
        a1.out_mult = bk.q2_mult;
        a1.out = r->q2;
        if (int e = launch_conv_col(prec, a1, C, PMG_EPI_Q, s)) return e;
        ColConvArgs a2{};
        a2.x = r->q2;
        a2.zq = r->zq;
        a2.w = bk.w2;
        a2.M = M;
        a2.H = c.H;
        a2.W = c.W;
        a2.a_scale = bk.a2_scale;
        a2.w_scale = bk.w2_scale;
        a2.bias = bk.b2;
        a2.skip = r->x;
        a2.out = r->x;
        if (k == 0 && x0_feats) {
            a2.x0_feats = x0_feats;
            a2.x0_rg = x0_rg;
            a2.x0_in_w = r->w.in_w;
            a2.x0_in_b = r->w.in_b;
            a2.x0_pr_w = r->w.pr_w;
            a2.x0_pr_b = r->w.pr_b;
        }
        if (k + 1 < nbk) {
            const pmg_block_weights& bn = r->blocks[k + 1];
            a2.ln_gamma = bn.ln_gamma;
            a2.ln_beta = bn.ln_beta;
            a2.ln_eps = 1e-6f;
            a2.next_mult = bn.q1_mult;
            a2.next_q = r->q1;
            if (int e = launch_conv_col(prec, a2, C, PMG_EPI_RLN, s)) return e;
        } else {
            a2.out_w = r->w.out_w;
            a2.out_b = r->w.out_b;
            if (delta_out) {
                a2.out = delta_out;
            } else {
                a2.points = points;
                a2.points_out = points_out;
                if (c.output_gate && gate_lidar) {
                    a2.gate_lidar = gate_lidar;
                    a2.gate_conf = gate_conf;
                    a2.gate_dh = c.dh;
                    a2.gate_dw = c.dw;
                    // the reference's Python floats: floor + (1.0 - floor) * u, both constants rounded to fp32
                    a2.gate_floor = c.output_gate_floor;
                    a2.gate_scale = (float)(1.0 - (double)c.output_gate_floor);
                }
            }
            if (int e = launch_conv_col(prec, a2, C, PMG_EPI_ROUT, s)) return e;
        }
    }
    return PMG_OK;
}

static InputStage input_stage_args(pmg_refiner* r, const float* feats) {
    const pmg_refiner_config& c = r->cfg;
    const pmg_block_weights& b0 = r->blocks[0];
    InputStage in{};
    in.points = feats;
    in.B = c.B;
    in.H = c.H;
    in.W = c.W;
    in.C = c.C;
    in.dh = c.dh;
    in.dw = c.dw;
    in.soft_gate = c.soft_gate;
    in.in_w = r->w.in_w;
    in.in_b = r->w.in_b;
    in.pr_w = r->w.pr_w;
    in.pr_b = r->w.pr_b;
    in.x_out = r->x;
    in.gamma = b0.ln_gamma;
    in.beta = b0.ln_beta;
    in.eps = 1e-6f;
    in.out_mult = b0.q1_mult;
    in.q_out = r->q1;
    in.resolution = c.depth_resolution;
    in.zq_out = r->zq;
    return in;
}

// Enqueues one step on `s`.
static int enqueue_step(pmg_refiner* r, const float* points, float* points_out, const float* lidar,
                        const float* conf, float* st_prompt, float* st_final, hipStream_t s) {
    const pmg_refiner_config& c = r->cfg;
    const bool f16 = c.precision == PMG_PREC_FP16;
    float* st = st_prompt ? st_prompt : r->st_scratch;
    if (c.use_prompt) {
        FitLaunch f{};
        f.mode = 1;
        f.logz = points + 2;
        f.stride = 3;
        f.lidar = lidar;
        f.conf = conf;
        f.B = c.B;
        f.H = c.H;
        f.W = c.W;
        f.dh = c.dh;
        f.dw = c.dw;
        f.N = (int64_t)c.H * c.W;
        f.iters = c.fit_iters;
        f.trim = c.fit_trim;
        f.min_points = c.fit_min_points;
        f.st = st;
        f.info = nullptr;
        f.workspace = r->fit_ws[0];
        f.workspace_bytes = r->fit_ws_bytes[0];
        if (int e = launch_fit(f, s)) return e;
    }
    InputStage in = input_stage_args(r, points);
    in.lidar = lidar;
    in.conf = conf;
    in.st = st;
    in.use_prompt = c.use_prompt;
    const bool x0 = recompute_x0(r);
    if (x0) {
        in.x_out = nullptr;
        in.rg_out = c.use_prompt ? r->rg : nullptr;
    }
    if (int e = launch_input_stage(in, f16, s)) return e;
    if (int e = enqueue_blocks(r, points, points_out, nullptr, s, lidar, conf, x0 ? points : nullptr,
                               x0 && c.use_prompt ? r->rg : nullptr))
        return e;

    if (c.anchor > 0.0f) {
        // v3.py:570-573: _lidar_in_affine_frame on the refined logz (the prompt fit's inputs), then the pull
        float* st_a = r->st_scratch + 4 * c.B;
        FitLaunch f{};
        f.mode = 1;
        f.logz = points_out + 2;
        f.stride = 3;
        f.lidar = lidar;
        f.conf = conf;
        f.B = c.B;
        f.H = c.H;
        f.W = c.W;
        f.dh = c.dh;
        f.dw = c.dw;
        f.N = (int64_t)c.H * c.W;
        f.iters = c.fit_iters;
        f.trim = c.fit_trim;
        f.min_points = c.fit_min_points;
        f.st = st_a;
        f.info = nullptr;
        f.workspace = r->fit_ws[0];
        f.workspace_bytes = r->fit_ws_bytes[0];
        if (int e = launch_fit(f, s)) return e;
        if (int e = launch_anchor(points_out, c.B, c.H, c.W, lidar, conf, c.dh, c.dw, st_a, c.anchor, s)) return e;
    }

    if (c.final_fit) {
        // v3.py:768-778: area-pool the refined depth to the LiDAR grid, mask, fit.
        FinalFit f{};
        f.logz = points_out + 2;
        f.stride = 3;
        f.lidar = lidar;
        f.conf = conf;
        f.mask_binary = nullptr;
        f.B = c.B;
        f.H = c.H;
        f.W = c.W;
        f.dh = c.dh;
        f.dw = c.dw;
        f.iters = c.fit_iters;
        f.trim = c.fit_trim;
        f.min_points = c.fit_min_points;
        f.st = st_final ? st_final : r->st_scratch + 2 * c.B;
        f.info = nullptr;
        f.workspace = r->fit_ws[1];
        f.workspace_bytes = r->fit_ws_bytes[1];
        if (int e = launch_final_fit(f, s)) return e;
    }
    return PMG_OK;
}

// Enqueues the refiner module's forward (Sparse3DUNet.forward, sparse_unet.py:176-258, single level): input_proj
// (+ prompt_proj of the given prompt features), the residual blocks, out_proj into delta_out [M].
static int enqueue_forward(pmg_refiner* r, const float* feats, const int32_t* coords, const float* prompt_feats,
                           float* delta_out, hipStream_t s) {
    InputStage in = input_stage_args(r, feats);
    in.prompt_in = prompt_feats;
    in.use_prompt = prompt_feats != nullptr;
    in.zkeys = coords ? coords + 3 : nullptr;
    in.zkey_stride = 4;
    const bool x0 = recompute_x0(r);
    if (x0) in.x_out = nullptr;
    if (int e = launch_input_stage(in, r->cfg.precision == PMG_PREC_FP16, s)) return e;
    return enqueue_blocks(r, nullptr, nullptr, delta_out, s, nullptr, nullptr, x0 ? feats : nullptr,
                          x0 ? prompt_feats : nullptr);
}

extern "C" {

const char* pmg_last_error(void) { return g_last_error.c_str(); }

int pmg_version(void) { return 5; }

pmg_refiner* pmg_refiner_create(const pmg_refiner_config* cfg) {
    if (!cfg) {
        set_error("pmg_refiner_create: null config");
        return nullptr;
    }
    const pmg_refiner_config& c = *cfg;
    if (c.B < 1 || c.H < 1 || c.W < 1 || (int64_t)c.B * c.H * c.W > INT_MAX / 27 || !supported_width(c.C) ||
        c.n_blocks < 1 || (c.precision != PMG_PREC_INT8 && c.precision != PMG_PREC_FP16) || c.dh < 1 || c.dw < 1 ||
        c.fit_iters < 0 || c.fit_iters > 64 || c.fit_min_points < 1 || !(c.fit_trim >= 0.0f && c.fit_trim < 1.0f) ||
        (int64_t)c.H * c.W > ((int64_t)1 << 22) || !(c.output_gate_floor >= 0.0f && c.output_gate_floor <= 1.0f) ||
        !(c.anchor >= 0.0f && c.anchor <= 1.0f)) {
        set_error("pmg_refiner_create: unsupported configuration");
        return nullptr;
    }
    // the metric fit holds at most 2^21 elements per batch item: the prompt fit and the anchor's re-fit run on the
    // H x W map, the final fit on the dh x dw LiDAR grid
    if ((c.use_prompt || c.anchor > 0.0f) && (int64_t)c.H * c.W > kFitMaxElements) {
        set_error("pmg_refiner_create: H*W = " + std::to_string((int64_t)c.H * c.W) +
                  " exceeds the metric fit's 2^21 elements (use_prompt / anchor)");
        return nullptr;
    }
    if (c.final_fit && (int64_t)c.dh * c.dw > kFitMaxElements) {
        set_error("pmg_refiner_create: dh*dw = " + std::to_string((int64_t)c.dh * c.dw) +
                  " exceeds the metric fit's 2^21 elements (final_fit)");
        return nullptr;
    }
    pmg_refiner* r = new pmg_refiner();
    r->cfg = c;
    r->M = (int64_t)c.B * c.H * c.W;
    const int64_t M = r->M;
    const size_t elt = c.precision == PMG_PREC_FP16 ? 2 : 1;
    r->fit_ws_bytes[0] = align_up(fit_workspace_bytes((int64_t)c.H * c.W, c.fit_iters), 256);
    r->fit_ws_bytes[1] = c.final_fit ? align_up(final_fit_workspace_bytes(c.B, c.dh, c.dw, c.fit_iters), 256) : 256;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align_up(off + bytes, 256);
        return o;
    };
    const size_t o_zq = take(M * 4), o_zmin = take(c.B * 4), o_zmax = take(c.B * 4);
    const size_t o_x = take(M * c.C * 4), o_q1 = take(M * c.C * elt), o_q2 = take(M * c.C * elt);
    const size_t o_rg = take(M * 2 * 4);
    const size_t o_st = take(6 * c.B * 4), o_f0 = take(r->fit_ws_bytes[0]), o_f1 = take(r->fit_ws_bytes[1]);
    r->arena_bytes = off;
    if (hipMalloc(&r->arena, r->arena_bytes) != hipSuccess) {
        set_error("pmg_refiner_create: hipMalloc of " + std::to_string(r->arena_bytes) + " bytes failed");
        delete r;
        return nullptr;
    }
    if (hipMemset(r->arena, 0, r->arena_bytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        set_error("pmg_refiner_create: clearing the workspace failed");
        hipFree(r->arena);
        delete r;
        return nullptr;
    }
    uint8_t* a = (uint8_t*)r->arena;
    r->zq = (int32_t*)(a + o_zq);
    r->zmin = (int32_t*)(a + o_zmin);
    r->zmax = (int32_t*)(a + o_zmax);
    r->x = (float*)(a + o_x);
    r->rg = (float*)(a + o_rg);
    r->q1 = a + o_q1;
    r->q2 = a + o_q2;
    r->st_scratch = (float*)(a + o_st);
    r->fit_ws[0] = a + o_f0;
    r->fit_ws[1] = a + o_f1;
    return r;
}

void pmg_refiner_destroy(pmg_refiner* r) {
    if (!r) return;
    r->graphs.clear();
    if (r->arena) hipFree(r->arena);
    delete r;
}

int pmg_refiner_set_weights(pmg_refiner* r, const pmg_refiner_weights* w) {
    PMG_REQUIRE(r && w, "null argument");
    PMG_REQUIRE(w->n_blocks == r->cfg.n_blocks && w->blocks, "block count mismatch");
    PMG_REQUIRE(w->in_w && w->in_b && w->out_w && w->out_b, "missing projection weights");
    PMG_REQUIRE(!r->cfg.use_prompt || (w->pr_w && w->pr_b), "use_prompt needs prompt_proj weights");
    const bool i8 = r->cfg.precision == PMG_PREC_INT8;
    for (int k = 0; k < w->n_blocks; ++k) {
        const pmg_block_weights& b = w->blocks[k];
        PMG_REQUIRE(b.ln_gamma && b.ln_beta && b.w1 && b.b1 && b.w2 && b.b2, "missing block weights");
        PMG_REQUIRE(aligned16(b.w1) && aligned16(b.w2), "conv weights must be 16-byte aligned");
        if (i8)
            PMG_REQUIRE(b.w1_scale && b.w2_scale && b.a1_scale > 0.0f && b.a2_scale > 0.0f && b.q1_mult > 0.0f &&
                            b.q2_mult > 0.0f,
                        "int8 blocks need weight and activation scales");
    }
    r->w = *w;
    r->blocks.assign(w->blocks, w->blocks + w->n_blocks);
    r->w.blocks = nullptr;
    r->have_weights = true;
    r->graphs.clear();
    return PMG_OK;
}

int pmg_refiner_step(pmg_refiner* r, const float* points, float* points_out, const float* lidar, const float* conf,
                     float* st_prompt, float* st_final, void* stream) {
    PMG_REQUIRE(r && r->have_weights, "weights not set");
    PMG_REQUIRE(points && points_out, "null points");
    PMG_REQUIRE((!r->cfg.use_prompt && !r->cfg.final_fit) || (lidar && conf), "LiDAR inputs required");
    hipStream_t s = (hipStream_t)stream;
    const void* const key[kGraphKey] = {(const void*)1, points, points_out, lidar, conf, st_prompt, st_final, stream};
    return r->graphs.run(key, s, r->cfg.use_graph, [&] { return enqueue_step(r, points, points_out, lidar, conf, st_prompt, st_final, s); });
}

int pmg_refiner_forward(pmg_refiner* r, const float* feats, const int32_t* coords, const float* prompt_feats,
                        float* out, void* stream) {
    PMG_REQUIRE(r && r->have_weights, "weights not set");
    PMG_REQUIRE(feats && out, "null buffer");
    PMG_REQUIRE(!prompt_feats || (r->w.pr_w && r->w.pr_b), "prompt_feats given but the refiner has no prompt_proj");
    hipStream_t s = (hipStream_t)stream;
    const void* const key[kGraphKey] = {(const void*)2, feats, coords, prompt_feats, out, nullptr, nullptr, stream};
    return r->graphs.run(key, s, r->cfg.use_graph, [&] { return enqueue_forward(r, feats, coords, prompt_feats, out, s); });
}

int pmg_refiner_check(pmg_refiner* r, void* stream) {
    PMG_REQUIRE(r, "null refiner");
    PMG_CHECK_HIP(hipStreamSynchronize((hipStream_t)stream));
    // each fit launch whose bounded wait expired has already restored its workspace and written NaN (s, t); the
    // count it left in the workspace is reported once here and cleared
    // (a context without a final fit holds only a stub there)
    unsigned seen[2] = {0, 0};
    const bool has[2] = {r->fit_ws_bytes[0] > kFitErrSeenOffset, r->fit_ws_bytes[1] > kFitErrSeenOffset};
    for (int k = 0; k < 2; ++k)
        if (has[k])
            PMG_CHECK_HIP(hipMemcpy(&seen[k], (uint8_t*)r->fit_ws[k] + kFitErrSeenOffset, sizeof(unsigned),
                                    hipMemcpyDeviceToHost));
    if (seen[0] || seen[1]) {
        for (int k = 0; k < 2; ++k)
            if (has[k]) PMG_CHECK_HIP(hipMemset((uint8_t*)r->fit_ws[k] + kFitErrSeenOffset, 0, sizeof(unsigned)));
        PMG_CHECK_HIP(hipDeviceSynchronize());
        return fail(PMG_E_DEVICE, "pmg_refiner_check: a device-wide wait in the metric fit expired (" +
                                      std::to_string(seen[0] + seen[1]) + " launches)");
    }
    return PMG_OK;
}

const void* pmg_refiner_buffer(pmg_refiner* r, int id) {
    if (!r) return nullptr;
    switch (id) {
        case 0: return r->zq;
        case 3: return r->x;
        case 4: return r->q1;
        case 5: return r->q2;
        default: return nullptr;
    }
}

}  // extern "C"
