// Bit-reproducible fp32 arithmetic shared by every kernel whose result is rounded into an integer.
//
// The int8 refiner requantises after non-linearities (SiLU, LayerNorm, log), and a single ulp of difference
// in front of rint() flips an int8 code at a .5 tie. So every function here is written from IEEE-754
// basic operations only (+, -, *, /, sqrt, rint, ldexp by exponent-field construction), each of which is
// correctly rounded on gfx950 and on the host. The library is compiled with -ffp-contract=off (no fused
// multiply-add is formed) and with correctly rounded fp32 division and square root, so the same source
// gives the same bits on the GPU, on the host CPU, and in a NumPy float32 restatement of the same steps.
//
//   exp_f32   Cody-Waite reduction x = k*ln2 + r, |r| <= ln2/2, degree-7 Taylor polynomial in Horner form,
//             scaling by 2^k through the exponent field. Domain: exp(x) = 0 for x < -87, +inf for x > 88.8.
//             (Results stay normal on the whole non-zero range, so no denormal handling is needed.)
//   log_f32   x = 2^e * m, m in [sqrt(2)/2, sqrt(2)], log(m) = 2 atanh(s), s = (m-1)/(m+1), odd series to s^9.
//             Domain: positive normal x (callers clamp to >= 1e-4).
//   silu_f32  y / (1 + exp(-y)), as in the reference's deployed epilogue (SparseConvInt8.metal:108).
//   quant_i8  clamp(rint(y * mult), -127, 127) with mult = 127/clip: the requantisation of the reference's
//             deployed int8 kernels (SparseConvInt8.metal:109, Refiner.metal:120; mult from Refiner.swift:148),
//             round-half-to-even as torch.round and Metal rint.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define PMG_HD __host__ __device__ inline

namespace pmg {

PMG_HD uint32_t f2u(float x) { return __builtin_bit_cast(uint32_t, x); }
PMG_HD float u2f(uint32_t x) { return __builtin_bit_cast(float, x); }
PMG_HD float rne(float x) { return __builtin_rintf(x); }
PMG_HD float fmin_(float a, float b) { return a < b ? a : b; }
PMG_HD float fmax_(float a, float b) { return a > b ? a : b; }

// fp32 constants by bit pattern so that the NumPy restatement uses the identical values.
#define PMG_F(bits) ::pmg::u2f(bits##u)
#define PMG_LOG2E PMG_F(0x3fb8aa3b)
#define PMG_LN2_HI PMG_F(0x3f317200)
#define PMG_LN2_LO PMG_F(0x35bfbe8e)
#define PMG_I6 PMG_F(0x3e2aaaab)
#define PMG_I24 PMG_F(0x3d2aaaab)
#define PMG_I120 PMG_F(0x3c088889)
#define PMG_I720 PMG_F(0x3ab60b61)
#define PMG_I5040 PMG_F(0x39500d01)
#define PMG_C3 PMG_F(0x3eaaaaab)
#define PMG_C5 PMG_F(0x3e4ccccd)
#define PMG_C7 PMG_F(0x3e124925)
#define PMG_C9 PMG_F(0x3de38e39)
#define PMG_SQRT2 PMG_F(0x3fb504f3)

PMG_HD float exp_f32(float x) {
    // Branch-free: the polynomial runs on x clamped into the domain (identical to x inside it), and selects
    // produce the special values, so a wave never diverges here.
    const float xc = fmin_(fmax_(x, -87.0f), 88.8f);
    const float kf = rne(xc * PMG_LOG2E);
    float r = xc - kf * PMG_LN2_HI;
    r = r - kf * PMG_LN2_LO;
    float p = PMG_I5040;
    p = p * r + PMG_I720;
    p = p * r + PMG_I120;
    p = p * r + PMG_I24;
    p = p * r + PMG_I6;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    const int k = (int)kf;  // in [-126, 128]
    const float big = (p * u2f(254u << 23)) * 2.0f;
    const float val = k > 127 ? big : p * u2f((uint32_t)(k + 127 > 0 ? k + 127 : 0) << 23);
    const float out = x > 88.8f ? u2f(0x7f800000u) : (x < -87.0f ? 0.0f : val);
    return x != x ? x : out;
}

PMG_HD float log_f32(float x) {
    const uint32_t u = f2u(x);
    const float m0 = u2f((u & 0x007fffffu) | 0x3f800000u);
    const bool hi = m0 > PMG_SQRT2;
    const float m = hi ? m0 * 0.5f : m0;
    const int e = (int)(u >> 23) - 127 + (hi ? 1 : 0);
    const float f = m - 1.0f;
    const float s = f / (2.0f + f);
    const float z = s * s;
    float R = PMG_C9;
    R = R * z + PMG_C7;
    R = R * z + PMG_C5;
    R = R * z + PMG_C3;
    R = R * z;
    const float t = s + s * R;
    const float logm = t + t;
    const float ef = (float)e;
    return ef * PMG_LN2_HI + (ef * PMG_LN2_LO + logm);
}

PMG_HD float silu_f32(float y) { return y / (1.0f + exp_f32(-y)); }

PMG_HD float quant_f32(float y, float mult) { return fmin_(fmax_(rne(y * mult), -127.0f), 127.0f); }

PMG_HD int8_t quant_i8(float y, float mult) { return (int8_t)(int)quant_f32(y, mult); }

}  // namespace pmg
