// expf as the host C library computes it, for the softmax gradients and the
// logistic loss's scalar rows.
//
// hessboost calls f32::exp there (simd/mod.rs:425-427, 580-600), i.e. the
// host libm's expf. glibc (2.28 and later, 2.35 here) implements it with the
// method of ARM's Optimized Routines (Szabolcs Nagy, 2017): with N = 32,
// k = round(x N / ln 2) and r = x N / ln 2 - k, exp(x) = 2^(k/N) 2^(r/N),
// 2^(k/N) from a table of 2^(i/N) with the exponent bits added, and
// 2^(r/N) from a cubic in r, all in f64, rounded to f32 once at the end.
// On CPUs with FMA, glibc's build fuses the reduction (r from the unrounded
// product x N / ln 2) and the cubic's multiply-adds; this restatement does
// the same and so returns glibc's bits for every f32 x (checked
// exhaustively against the host libm: tests/test_libm_expf.py). Softmax
// evaluates exp at x - max(x) <= 0, the logistic loss's scalar rows at
// min(-x, 88.7) (simd/mod.rs:425-427).
//
// The table (bits of 2^(i/32) minus i << 47, for i < 32) is computed by the
// caller with the host's exp2 and passed in.
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define HBR_LIBM_FN __host__ __device__ inline
#else
#define HBR_LIBM_FN static inline
#endif

HBR_LIBM_FN double hbr_bits_to_f64(uint64_t u) {
    double d;
    memcpy(&d, &u, sizeof d);
    return d;
}

HBR_LIBM_FN uint64_t hbr_f64_to_bits(double d) {
    uint64_t u;
    memcpy(&u, &d, sizeof u);
    return u;
}

HBR_LIBM_FN float hbr_expf_libm(float x, const uint64_t *tab) {
    uint32_t ux;
    memcpy(&ux, &x, sizeof ux);
    if (ux == 0xff800000u) return 0.0f;                   // -inf
    if ((ux & 0x7fffffffu) > 0x7f800000u) return x + x;   // NaN
    if (x < -0x1.9fe368p6f) return 0.0f;                 // below log(2^-150): rounds to +0
    if (x > 0x1.62e42ep6f) return __builtin_inff();       // above log(FLT_MAX): overflows (+inf too)
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32;  // N / ln 2
    const double shift = 0x1.8p+52;                      // rounds k to an integer in the low bits
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    const uint64_t ki = hbr_f64_to_bits(kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const double s = hbr_bits_to_f64(tab[ki % 32] + (ki << 47));
    const double p = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(p, r2, y);
    return (float)(y * s);
}
