// Launchers shared between translation units (not part of the C ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pmg {

bool supported_width(int C);

int launch_ln_silu(const float* x, int64_t M, int C, const float* gamma, const float* beta, float eps,
                   float out_mult, void* out, bool f16, hipStream_t s);

struct InputStage {
    const float* points;
    int B, H, W, C;
    const float* lidar;
    const float* conf;
    int dh, dw;
    const float* st;
    int use_prompt, soft_gate;
    const float* in_w;
    const float* in_b;
    const float* pr_w;
    const float* pr_b;
    float* x_out;
    const float* gamma;
    const float* beta;
    float eps;
    float out_mult;
    void* q_out;
    float resolution;
    int32_t* zq_out;
    const float* prompt_in;  // [M][2] given prompt features, or NULL (computed from the LiDAR when use_prompt)
    const int32_t* zkeys;    // given z keys (coords[:, 3]) with element stride zkey_stride, or NULL
    int64_t zkey_stride;
    float* rg_out;  // [M][2] prompt features (residual, gate) written for a conv that recomputes h, or NULL
};
int launch_input_stage(const InputStage& in, bool f16, hipStream_t s);

struct FitLaunch {
    int mode;
    const float* z;
    const float* tg;
    const uint8_t* mask;
    const float* logz;
    int64_t stride;
    const float* lidar;
    const float* conf;
    int B, H, W, dh, dw;
    int64_t N;
    int iters;
    float trim;
    int min_points;
    float* st;
    int32_t* info;
    void* workspace;
    size_t workspace_bytes;
};
size_t fit_workspace_bytes(int64_t N, int iters);
int launch_fit(const FitLaunch& f, hipStream_t s);
// Byte offset, in a fit workspace, of the count of launches whose bounded wait expired (sticky until cleared).
constexpr size_t kFitErrSeenOffset = 3968;
// Elements per batch item the fit holds (256 blocks x 8192).
constexpr int64_t kFitMaxElements = (int64_t)1 << 21;

// The final metric fit at LiDAR resolution (v3.py:768-778): area-pooled depth, LiDAR mask, then the fit. The
// workspace starts with the fit's own (error flag at byte 64), followed by the pooled depth and mask.
struct FinalFit {
    const float* logz;
    int64_t stride;
    const float* lidar;
    const float* conf;
    const uint8_t* mask_binary;
    int B, H, W, dh, dw;
    int iters;
    float trim;
    int min_points;
    float* st;
    int32_t* info;
    void* workspace;
    size_t workspace_bytes;
};
size_t final_fit_workspace_bytes(int B, int dh, int dw, int iters);
int launch_final_fit(const FinalFit& f, hipStream_t s);

struct ColConvArgs {
    const void* x;
    const int32_t* zq;
    const void* w;
    int64_t M;
    int H, W;
    float a_scale;
    const float* w_scale;
    const float* bias;
    float out_mult;
    const float* skip;
    void* out;
    const float* ln_gamma;
    const float* ln_beta;
    float ln_eps;
    float next_mult;
    void* next_q;
    const float* out_w;
    const float* out_b;
    const float* points;
    float* points_out;
    // PMG_EPI_ROUT with points: the refiner output gate (v3.py:565-569) when gate_lidar is set -- the update is
    // scaled by g = gate_floor + gate_scale * u, u the LiDAR uncertainty of the pixel (lidar, conf [B][dh][dw])
    const float* gate_lidar;
    const float* gate_conf;
    int gate_dh, gate_dw;
    float gate_floor, gate_scale;
    // Residual epilogues of the first block: with x0_feats set, the skip is not read from `skip` but recomputed per
    // row as the input stage's h = input_proj(x0_feats[m]) (+ prompt_proj(x0_rg[m]) when x0_rg is set), so h is never
    // stored (x0_feats [M][3]; x0_rg [M][2]; x0_in_w [C][3], x0_in_b, x0_pr_w [C][2], x0_pr_b).
    const float* x0_feats;
    const float* x0_rg;
    const float* x0_in_w;
    const float* x0_in_b;
    const float* x0_pr_w;
    const float* x0_pr_b;
};
int launch_conv_col(int precision, const ColConvArgs& a, int C, int epi, hipStream_t s);

// The elastic anchor (v3.py:570-573): logz of points [B][H][W][3] moves by beta * gate * (log_d_aff - logz), with
// (log_d_aff, gate) the LiDAR in the affine frame of st [B][2] (hard gate, v3.py:376-380).
int launch_anchor(float* points, int B, int H, int W, const float* lidar, const float* conf, int dh, int dw,
                  const float* st, float beta, hipStream_t s);

// int8 submanifold conv on a device-sized level (generic map): rows m < *m_dev of a capacity-`cap` level; nmap_t is
// [27][cap] and tile_mask covers the rows. Epilogues ACC, BIAS, Q (SiLU requantise), R (+ skip). With a partials
// buffer of conv_split_bytes(C) bytes (C = 128, 256), a level with few rows splits its taps over more blocks and a
// second launch adds the partial sums (launches on one stream may share the buffer).
struct DevConv {
    const int8_t* x;
    const int32_t* nmap_t;
    const uint32_t* tile_mask;
    int64_t cap;
    const int64_t* m_dev;
    int Ci, Co;
    const int8_t* w;  // [Co][27][Ci]
    int epilogue;
    float a_scale;
    const float* w_scale;
    const float* bias;
    float out_mult;
    const float* skip;
    void* out;
    int32_t* part;       // tap-split partial sums, or NULL
    int64_t part_bytes;
};
int launch_conv_i8_dev(const DevConv& d, hipStream_t s);
// The same for the fp16 teacher: x, w fp16 (the int8_t pointers hold fp16 data), fp32 accumulation, epilogues SILU
// (bias + SiLU to fp16), R, BIAS, ACC; no tap split.
int launch_conv_f16_dev(const DevConv& d, hipStream_t s);
int64_t conv_split_bytes(int C);  // partials buffer of a width's tap split (0: no split at that width)

// Stable LSD radix sort of (uint64 key, int32 value) pairs over the keys' low `bits` bits, 8 bits per pass
// (pmg_pool.hip): the caller writes the keys into keys[0]; the first pass takes value i for key i; the sorted
// values go to vals_final and the sorted keys are in keys[sorted]. Workspace: radix_sort_workspace_bytes(M).
struct RadixBufs {
    uint64_t* keys[2];
    int32_t* vals[2];
    uint32_t* hist;
    uint32_t* tcnt;
    uint32_t* ctot;
    int sorted;
};
size_t radix_sort_workspace_bytes(int64_t M);
RadixBufs radix_bufs(void* workspace, int64_t M);
int radix_sort_pairs(RadixBufs& r, int64_t M, int bits, int32_t* vals_final, hipStream_t s);

}  // namespace pmg
