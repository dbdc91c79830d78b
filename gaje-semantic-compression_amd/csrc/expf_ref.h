// Single-precision exponential with the exact results of the C library that
// the reference's f32::exp calls on x86-64 Linux.
//
// The reference computes every softmax and SiLU exponential with f32::exp
// (src/nn/attention.rs:106, src/compute/kernels/activation.rs:42-44), which
// lowers to glibc's expf.  On an FMA-capable x86-64 host glibc dispatches the
// FMA build of its table-driven expf (the ARM optimized-routines design:
// 2^(k/32) table, degree-3 polynomial, all intermediate work in binary64).  In
// that build the compiler fuses the scaling multiply into both of its uses, so
// the reduction is kd = fma(InvLn2N, x, SHIFT), r = fma(InvLn2N, x, -kd).
// Restated below from the published method; it agrees with the host libm's
// expf on all 2^32 single-precision inputs (tests/test_expf_ref.py sweeps
// them on the CPU, tests/test_gpu_ops.py checks the device build).
//
// Attribution: the algorithm, its 2^(i/32) table and its polynomial
// coefficients are those of Arm's optimized-routines expf (Copyright (c) Arm
// Limited; MIT OR Apache-2.0 WITH LLVM-exception), the implementation glibc
// adopted for expf.
//
// Usable from host C++ (the CPU sweep) and from HIP device code.
#pragma once

#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define GAJE_HD __host__ __device__
#else
#define GAJE_HD
#endif

namespace gaje {

// tab[i] = bits(2^(i/32) rounded to binary64) - (i << 47)
#define GAJE_EXP2_TAB                                                                              \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

#if defined(__HIP_DEVICE_COMPILE__)
__constant__ static const uint64_t kExp2Tab[32] = GAJE_EXP2_TAB;
#else
static const uint64_t kExp2Tab[32] = GAJE_EXP2_TAB;
#endif

GAJE_HD inline uint32_t ref_f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

// tab: the 32 table words above (kExp2Tab, or a copy of it in LDS).
GAJE_HD inline float expf_ref_t(float x, const uint64_t *tab) {
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double Shift = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const uint32_t ux = ref_f32_bits(x);
    const uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88 (top 12 bits of 88.0f), inf or nan
        if (ux == 0xff800000u) return 0.0f;      // -inf
        if (abstop >= 0x7f8u) return x + x;      // inf or nan
        if (x > 0x1.62e42ep6f) return __builtin_huge_valf();  // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;     // underflow
    }
    const double xd = (double)x;
    double kd = __builtin_fma(InvLn2N, xd, Shift);
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= Shift;
    const double r = __builtin_fma(InvLn2N, xd, -kd);
    uint64_t t = tab[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    const double z = __builtin_fma(C0, r, C1);
    const double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

GAJE_HD inline float expf_ref(float x) { return expf_ref_t(x, kExp2Tab); }

}  // namespace gaje
