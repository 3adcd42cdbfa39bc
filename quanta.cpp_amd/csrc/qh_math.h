// Scalar math shared by the decoder kernels, written to give the same bits as the reference's CPU build.
//
// qh_expf: exp(x) in binary32 as glibc computes it on x86-64 hosts with FMA (the engine's std::exp(float) calls,
// reference engine/src/ops_ref.cpp:221 softmax and :246 swiglu). The method is the published one of ARM's
// optimized-routines expf, which glibc uses since 2.28:
//   k = round(x * 32/ln2) (ties to even, through the 1.5 * 2^52 shift), r = x * 32/ln2 - k,
//   2^(k/32) from a 32-entry table of 2^(i/32) with the exponent added as an integer,
//   exp(x) ~= 2^(k/32) * (1 + C2 r + C1 r^2 + C0 r^3), all in binary64, one rounding to binary32 at the end.
// The table entries are bits(2^(i/32) rounded to nearest binary64) - (i << 47). The polynomial coefficients are
// the method's published ones (relative error 1.69 * 2^-34), pre-divided by 32, 32^2 and 32^3. Which products the
// host build fuses into multiply-adds is selected by QH_EXPF_FUSED (see tests/cpp/expf_exhaustive.cpp, which
// compares every one of the 2^32 inputs with the host's expf).
// Source of the method: ARM optimized-routines (github.com/ARM-software/optimized-routines, math/expf.c and
// math/exp2f_data.c), licensed MIT OR Apache-2.0 WITH LLVM-exception; the code here is written from that published
// description, and the table holds the values 2^(i/32) themselves.
#pragma once

#include <stdint.h>
#include <string.h>

#ifndef QH_HD
#define QH_HD __host__ __device__
#endif

namespace qh {

namespace expf_detail {

constexpr uint64_t kTab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};
constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;
constexpr double kShift = 0x1.8p+52;
constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32;

QH_HD inline uint32_t bits_f32(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
QH_HD inline uint64_t bits_f64(double d) {
    uint64_t u;
    memcpy(&u, &d, 8);
    return u;
}
QH_HD inline double from_bits_f64(uint64_t u) {
    double d;
    memcpy(&d, &u, 8);
    return d;
}

}  // namespace expf_detail

// FUSED: 0 = no multiply-add fused, 1 = the polynomial's three multiply-adds fused, 2 = also x * 32/ln2 fused
// into the rounding shift and the reduction.
// tab: the 32-entry table (kTab, or a copy of it, e.g. in LDS).
template <int FUSED>
QH_HD inline float expf_variant(float x, const uint64_t* tab = expf_detail::kTab) {
    using namespace expf_detail;
    const uint32_t abstop = (bits_f32(x) >> 20) & 0x7ffu;
    if (abstop >= (bits_f32(88.0f) >> 20)) {
        if (bits_f32(x) == 0xff800000u) return 0.0f;           // -inf
        if (abstop >= (bits_f32(__builtin_inff()) >> 20)) return x + x;  // +inf, nan
        if (x > 0x1.62e42ep6f) return __builtin_inff();       // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;                   // underflow to +0
    }
    const double xd = (double)x;
    double kd, r;
    if (FUSED >= 2) {
        kd = __builtin_fma(kInvLn2N, xd, kShift);
    } else {
        kd = kInvLn2N * xd + kShift;
    }
    const uint64_t ki = bits_f64(kd);
    kd -= kShift;
    if (FUSED >= 2) {
        r = __builtin_fma(kInvLn2N, xd, -kd);
    } else {
        r = kInvLn2N * xd - kd;
    }
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    const double s = from_bits_f64(t);
    double z, y;
    const double r2 = r * r;
    if (FUSED >= 1) {
        z = __builtin_fma(kC0, r, kC1);
        y = __builtin_fma(kC2, r, 1.0);
        y = __builtin_fma(z, r2, y);
    } else {
        z = kC0 * r + kC1;
        y = kC2 * r + 1.0;
        y = z * r2 + y;
    }
    y = y * s;
    return (float)y;
}

}  // namespace qh
