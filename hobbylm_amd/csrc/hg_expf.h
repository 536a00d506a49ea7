// hg_expf.h -- binary32 exp() reproducing, bit for bit, the expf of the GNU C library
// (glibc >= 2.27, x86-64 FMA build) that Rust's f32::exp calls on linux-gnu.
//
// Method (Szabolcs Nagy, ARM optimized-routines; glibc sysdeps/ieee754/flt-32/e_expf.c):
//   x*32/ln2 = k + r, r in [-1/2, 1/2], k integer (round-to-nearest via the 1.5*2^52 shift);
//   exp(x) = 2^(k/32) * 2^(r/32), with 2^(k/32) from a 32-entry table of correctly
//   rounded 2^(i/32) whose exponent field is pre-biased, and 2^(r/32) from a cubic in r
//   evaluated in double precision; one final double -> float rounding.
// glibc's x86-64 multiarch selects a build of that source compiled with -mfma, in which the
// compiler fuses the three polynomial multiply-adds and both uses of z = x*32/ln2
// (k = rint(z) via z + shift, and r = z - k); the fma() calls below reproduce that.
// The table entries are bits(2^(i/32)) - (i << 47), computed to 80 digits and rounded.
// Equality with the host glibc over every binary32 input is checked by
// tests/test_expf.py.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define HG_HD __host__ __device__
#else
#define HG_HD
#endif

namespace hg {

HG_HD inline uint64_t hg_exp2_bits(uint32_t i) {
    // 2^(i/32) with i<<47 subtracted from its bit pattern; indexed by k mod 32
    constexpr uint64_t T[32] = {
        0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
        0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
        0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
        0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
        0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
        0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
        0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
        0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
    };
    return T[i & 31];
}

#ifndef HG_EXPF_VARIANT
#define HG_EXPF_VARIANT 2  // 0: no fusion, 1: fused polynomial, 2: fused polynomial + range reduction
#endif

// expf with the table read through `lookup(i)` (i < 32 -> hg_exp2_bits(i)).  The main path
// runs for every input and the special cases are selected afterwards, so a lookup that
// exchanges values between lanes is reached by every lane of a uniform call.
template <class Lookup>
HG_HD inline float hg_expf_l(float x, const Lookup &lookup) {
    const uint32_t ix = __builtin_bit_cast(uint32_t, x);
    const uint32_t abstop = (ix >> 20) & 0x7ff;
    const double InvLn2N = 0x1.71547652b82fep+0 * 32;
    const double SHIFT = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
#if HG_EXPF_VARIANT == 2
    double kd = __builtin_fma(InvLn2N, xd, SHIFT);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= SHIFT;
    const double r = __builtin_fma(InvLn2N, xd, -kd);
#else
    const double z0 = InvLn2N * xd;
    double kd = z0 + SHIFT;
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= SHIFT;
    const double r = z0 - kd;
#endif
    uint64_t t = lookup((uint32_t)(ki % 32));
    t += ki << 47;
    const double s = __builtin_bit_cast(double, t);
#if HG_EXPF_VARIANT >= 1
    const double z = __builtin_fma(C0, r, C1);
    const double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
#else
    const double z = C0 * r + C1;
    const double r2 = r * r;
    double y = C2 * r + 1.0;
    y = z * r2 + y;
#endif
    y = y * s;
    float res = (float)y;
    if (abstop >= 0x42b) {                                       // |x| >= 88 or x is NaN
        if (ix == 0xff800000u) res = 0.0f;                       // -inf
        else if (abstop >= 0x7f8) res = x + x;                   // +inf or NaN
        else if (x > 0x1.62e42ep6f) res = __builtin_huge_valf(); // overflow
        else if (x < -0x1.9fe368p6f) res = 0.0f;                 // underflow
    }
    return res;
}

struct Exp2Const {
    HG_HD uint64_t operator()(uint32_t i) const { return hg_exp2_bits(i); }
};

HG_HD inline float hg_expf(float x) { return hg_expf_l(x, Exp2Const{}); }

// 1/(1+exp(-x)) and x*sigmoid(x) as ops.rs:75-82 write them, with the reference expf.
template <class Lookup>
HG_HD inline float hg_sigmoid_l(float x, const Lookup &lookup) { return 1.0f / (1.0f + hg_expf_l(-x, lookup)); }
template <class Lookup>
HG_HD inline float hg_silu_l(float x, const Lookup &lookup) { return x * hg_sigmoid_l(x, lookup); }
HG_HD inline float hg_sigmoid(float x) { return hg_sigmoid_l(x, Exp2Const{}); }
HG_HD inline float hg_silu(float x) { return hg_silu_l(x, Exp2Const{}); }

}  // namespace hg
