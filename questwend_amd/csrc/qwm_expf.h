// qwm_expf.h -- expf as ggml-CPU's x86-64 libm computes it, bit for bit on
// every float input, for the GPU and the host.
//
// ggml-CPU calls the C library's scalar expf in the sigmoid (ggml-cpu/
// unary-ops.cpp:31-33, the shared-expert gate and sigmoid routing) and in the
// scalar tails of soft_max and silu (vec.cpp:531-560, vec.h:936).  glibc
// 2.28 and later (this image has 2.35) implements expf with the algorithm of
// ARM's optimized-routines expf (Szabolcs Nagy): with N = 32,
//   k = round(x * N / ln2),  r = x * N / ln2 - k,
//   expf(x) = 2^(k/N) * (1 + C2 r + C1 r^2 + C0 r^3)   evaluated in double,
// where 2^(i/N) comes from a 32-entry table (the table below holds its bits
// minus i << 47, so that adding k << 47 scales it by 2^(k div N)), and the
// result is rounded to float once.  On x86-64 CPUs with FMA, glibc's ifunc
// picks the build compiled with FMA contraction: the rounding shift and the
// reduction r use fused multiply-adds, as restated here.
// tests/test_expf.py compares this restatement with the C library's expf on
// every float; the GPU tests compare the device copy with the host's.
#pragma once

#include <stdint.h>
#include <string.h>

#ifdef __HIPCC__
#define QWM_HD __host__ __device__ __forceinline__
#else
#define QWM_HD inline
#endif

namespace qwm {

// bits of 2^(i/32), rounded to the nearest double, minus i << 47
constexpr uint64_t EXP2F_TAB[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

QWM_HD uint32_t expf_f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
QWM_HD uint64_t expf_d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
QWM_HD double expf_u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

QWM_HD float libm_expf(float x) {
    const uint32_t ux = expf_f2u(x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                       // |x| >= 88 (top12 of 88.0f), inf or nan
        if (ux == 0xff800000u) return 0.0f;      // -inf
        if (abstop >= 0x7f8) return x + x;       // +inf, nan
        if (x > 0x1.62e42ep6f) return __builtin_inff();   // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;     // underflow
    }
    constexpr double InvLn2N = 0x1.71547652b82fep+0 * 32;
    constexpr double SHIFT = 0x1.8p+52;
    constexpr double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    constexpr double C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    constexpr double C2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = __builtin_fma(InvLn2N, xd, SHIFT);   // round(x N / ln2), ties to even, in the low bits
    const uint64_t ki = expf_d2u(kd);
    kd -= SHIFT;
    const double r = __builtin_fma(InvLn2N, xd, -kd);
    const uint64_t t = EXP2F_TAB[ki % 32] + (ki << 47);
    const double s = expf_u2d(t);
    const double z = __builtin_fma(C0, r, C1);
    const double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

// ggml-cpu's op_sigmoid (unary-ops.cpp:31-33): 1 / (1 + expf(-x))
QWM_HD float libm_sigmoid(float x) { return 1.0f / (1.0f + libm_expf(-x)); }

}  // namespace qwm
