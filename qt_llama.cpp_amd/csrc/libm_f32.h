// libm_f32.h -- f32 tanh, exp, sin and cos with the exact results of the C
// library the reference links.
//
// The reference's numerics go through crates/mrml-math/src/lib.rs, which
// binds glibc's tanhf, expf, sinf, cosf, powf and sqrtf.  A token step only
// reproduces the CPU path bit for bit if these return the same bits on the
// GPU, and glibc 2.35 is not correctly rounded (tanhf differs from the
// correctly rounded value on ~20% of inputs, expf on ~0.07%), so the device
// code evaluates the same published algorithms, operation for operation:
//
//  * tanhf: the Sun fdlibm algorithm (s_tanhf.c / s_expm1f.c, freely
//    distributable): tanh via expm1 of 2|x|, expm1 by reduction
//    x = k ln2 + r and a rational approximation of r in float arithmetic.
//  * expf: the table-driven algorithm of Szabolcs Nagy (Arm
//    optimized-routines, used by glibc since 2.27): k = round(x N / ln2),
//    2^(k/N) from a 32-entry table of doubles and a cubic in double.  glibc
//    selects a build compiled with FMA on x86-64 CPUs that have FMA and AVX2,
//    in which the reduction r = x N/ln2 - k and the three polynomial steps
//    are fused multiply-adds; `fused` picks that form.
//
//  * sinf, cosf: Arm optimized-routines as well (glibc since 2.28): a
//    double-precision polynomial after reduction by pi/2, Payne-Hanek for
//    large arguments.  RoPE's angles are cosf and sinf of
//    pos * freq_scale / powf(base, 2i/d); the powf values depend on i only
//    and come from the host's libm.
//
// powf is not here.  sqrtf and division are IEEE operations on both.
//
// Every function is usable from host code (checked against glibc over the
// float range) and device code.  Compile with contraction off: each
// product and sum must round separately unless fused on purpose.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MRML_HD __host__ __device__ __forceinline__
#else
#define MRML_HD static inline
#endif

namespace mrml_libm {

MRML_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
MRML_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
MRML_HD uint64_t d2u(double d) { return __builtin_bit_cast(uint64_t, d); }
MRML_HD double u2d(uint64_t u) { return __builtin_bit_cast(double, u); }

// ---- expm1f / tanhf (fdlibm) --------------------------------------------------
//
// expm1f and tanhf below follow fdlibm's s_expm1f.c and s_tanhf.c (float
// conversion by Ian Lance Taylor, Cygnus Support), whose notice is:
//
// ====================================================
// Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//
// Developed at SunPro, a Sun Microsystems, Inc. business.
// Permission to use, copy, modify, and distribute this
// software is freely granted, provided that this notice
// is preserved.
// ====================================================

// Both are written without data-dependent branches: every lane evaluates
// the argument reduction and the candidate results of fdlibm's cases, each
// with exactly the operations of its case, and selects the one its own
// argument picks.  A wave of GeGLU activations spans most of the cases, and
// as branches each taken case ran for the whole wave (about 1 us of the
// GeGLU kernel's tail).  k = 0 and k = +-1 reduce to fdlibm's generic
// formula exactly (t*ln2_hi and t*ln2_lo are exact for t = 0, +-1, and
// x - (-y) is x + y), so one reduction serves every case.
// fdlibm's expm1f cases below its overflow threshold, selected by k.
// TANH: only the arguments tanhf passes (2|y| for |y| >= 1, where k >= 3,
// and -2|y| for |y| < 1, where -3 <= k <= 0): the k = 1 case is left out,
// and the caller replaces the results of the arguments that fdlibm's
// special cases would catch (tiny, huge and non-finite y).
template <bool TANH>
MRML_HD float expm1f_cases(float x, uint32_t hx, bool neg)
{
    const float ln2_hi = 6.9313812256e-01f;   // 0x3f317180
    const float ln2_lo = 9.0580006145e-06f;   // 0x3717f7d1
    const float invln2 = 1.4426950216e+00f;   // 0x3fb8aa3b
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
                Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
    const bool red = hx > 0x3eb17218u;     // |x| > 0.5 ln2: reduce by k ln2
    const bool near1 = hx < 0x3f851592u;   // and |x| < 1.5 ln2: k = +-1
    // the generic k; the clamp only keeps the conversion defined for the
    // arguments whose result a special case replaces (|x| < 88.8 gives |k| < 129)
    float kf = invln2 * x + (neg ? -0.5f : 0.5f);
    kf = kf > -200.0f ? (kf < 200.0f ? kf : 200.0f) : -200.0f;
    // (the empty asm statements here and in tanhf make the compiler form
    // each candidate in every lane, so the selects stay selects: it would
    // otherwise put the conversion and the special cases behind branches)
    int32_t kg = (int32_t)kf;
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("" : "+v"(kg));
#endif
    int32_t k = red ? (near1 ? (neg ? -1 : 1) : kg) : 0;
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("" : "+v"(k));
#endif
    const float tk = (float)k;
    const float hi = x - tk * ln2_hi;  // exact
    const float lo = tk * ln2_lo;
    const float xr = hi - lo;
    const float c = red ? (hi - xr) - lo : 0.0f;
    const float hfx = 0.5f * xr;
    const float hxs = xr * hfx;
    const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    const float t = 3.0f - r1 * hfx;
    const float e = hxs * ((r1 - t) / (6.0f - xr * t));
    const float r_k0 = xr - (xr * e - hxs);
    float e2 = (xr * (e - c) - c);
    e2 -= hxs;
    const float r_km1 = 0.5f * (xr - e2) - 0.5f;
    const float r_k1 = TANH ? 0.0f : (xr < -0.25f ? -2.0f * (e2 - (xr + 0.5f)) : 1.0f + 2.0f * (xr - e2));
    const uint32_t ksh = (uint32_t)k << 23;
    const float r_far = u2f(f2u(1.0f - (e2 - xr)) + ksh) - 1.0f;  // k <= -2 or k > 56: exp(x) - 1 directly
    const int32_t kl = k < 0 ? 0 : (k > 31 ? 31 : k);            // shift counts in range for every lane
    const float r_lo = u2f(f2u(u2f(0x3f800000u - (0x1000000u >> kl)) - (e2 - xr)) + ksh);  // 2 <= k < 23
    const int32_t kh = k < 0 ? 0 : (k > 0x7e ? 0x7e : k);
    float y = xr - (e2 + u2f((uint32_t)(0x7f - kh) << 23));      // 23 <= k <= 56
    y += 1.0f;
    const float r_hi = u2f(f2u(y) + ksh);
    const float r_mid = (k <= -2 || k > 56) ? r_far : (k < 23 ? r_lo : r_hi);
    return k == 0 ? r_k0 : (k == -1 ? r_km1 : ((!TANH && k == 1) ? r_k1 : r_mid));
}

MRML_HD float expm1f(float x)
{
    const uint32_t hx = f2u(x) & 0x7fffffffu;
    const bool neg = (f2u(x) >> 31) != 0;
    const bool red = hx > 0x3eb17218u;
    float r = expm1f_cases<false>(x, hx, neg);
    const float tt = 1.0f + x;
    if (!red && hx < 0x33000000u) r = x - (tt - (1.0f + x));  // |x| < 2^-25
    if (hx >= 0x4195b844u && neg) r = -1.0f;                  // x < -27 ln2
    if (hx >= 0x42b17218u && !neg && x > 8.8721679688e+01f) r = __builtin_inff();
    if (hx == 0x7f800000u) r = neg ? -1.0f : x;
    if (hx > 0x7f800000u) r = x + x;
    return r;
}

MRML_HD float tanhf(float x)
{
    const uint32_t jx = f2u(x), ix = jx & 0x7fffffffu;
    const float ax = u2f(ix);
    const bool ge1 = ix >= 0x3f800000u;  // |x| >= 1: 1 - 2/(expm1(2|x|) + 2); else -t/(t + 2), t = expm1(-2|x|)
    const float a2 = ge1 ? 2.0f * ax : -2.0f * ax;
    const float t = expm1f_cases<true>(a2, f2u(a2) & 0x7fffffffu, !ge1);
    float q = (ge1 ? 2.0f : -t) / (t + 2.0f);
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("" : "+v"(q));  // formed in every lane: the selects below stay selects, not branches
#endif
    const float z = ix >= 0x41b00000u ? 1.0f : (ge1 ? 1.0f - q : q);  // |x| >= 22: 1 - tiny rounds to 1
    const bool sgn = (jx >> 31) != 0;
    // fdlibm's special cases, as selects: |x| < 2^-55 (x * (1 + x), which is
    // x itself for zeros too), +-inf (+-1), NaN (x + x)
    float xx = x + x;
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("" : "+v"(xx));
#endif
    const float r = ix < 0x24000000u ? x * (1.0f + x) : (sgn ? -z : z);
    return ix >= 0x7f800000u ? (ix == 0x7f800000u ? (sgn ? -1.0f : 1.0f) : xx) : r;
}

// ---- expf (Arm optimized-routines algorithm) -------------------------------------
//
// expf below follows math/expf.c and its 2^(i/32) table (math/exp2f_data.c)
// of Arm optimized-routines:
//
// Copyright (c) 2017-2018, Arm Limited.
// SPDX-License-Identifier: MIT

// T[i] = bits(2^(i/32)) - (i << 47): the correctly rounded doubles 2^(i/32)
// with the table index pre-subtracted from the exponent field.
struct ExpfTable {
    uint64_t t[32];
};
constexpr ExpfTable kExpfT = {{
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
}};

// expf with the table read from `tab` (kExpfT's 32 entries; a kernel may keep
// a copy in LDS, which a lane-indexed read reaches much sooner than the
// read-only global copy after a long weight stream has left the caches).
MRML_HD float expf_t(float x, bool fused, const uint64_t *tab)
{
    const double N = 32.0;
    const double invln2N = 0x1.71547652b82fep+0 * N;
    const double shift = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / N / N / N, C1 = 0x1.ebfce50fac4f3p-3 / N / N,
                 C2 = 0x1.62e42ff0c52d6p-1 / N;
    const uint32_t abstop = (f2u(x) >> 20) & 0x7ffu;
    if (abstop >= (f2u(88.0f) >> 20)) {
        if (f2u(x) == f2u(-__builtin_inff())) return 0.0f;
        if (abstop >= (f2u(__builtin_inff()) >> 20)) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double xd = (double)x;
    const double z = invln2N * xd;
    double kd = z + shift;
    const uint64_t ki = d2u(kd);
    kd -= shift;
    // The FMA build also fuses the reduction r = x N/ln2 - k.
    const double r = fused ? __builtin_fma(invln2N, xd, -kd) : z - kd;
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    const double s = u2d(t);
    const double r2 = r * r;
    double y;
    if (fused) {
        const double p = __builtin_fma(C0, r, C1);
        y = __builtin_fma(C2, r, 1.0);
        y = __builtin_fma(p, r2, y);
    } else {
        const double p = C0 * r + C1;
        y = C2 * r + 1.0;
        y = p * r2 + y;
    }
    return (float)(y * s);
}

MRML_HD float expf(float x, bool fused) { return expf_t(x, fused, kExpfT.t); }

// ---- sinf / cosf (Arm optimized-routines algorithm) ------------------------------
//
// sinf and cosf below follow math/sinf.c, math/cosf.c, math/sincosf.h and
// math/sincosf_data.c of Arm optimized-routines (the notice above applies):
// |x| < pi/4: a polynomial in double; |x| < 120: x - n pi/2 with n the
// rounded x 2/pi; larger: the Payne-Hanek reduction against 96 bits of 2/pi
// in integer arithmetic; then the sine or cosine polynomial in double,
// rounded once to float.  `fused` selects the FMA build that glibc picks on
// x86-64 CPUs with FMA and AVX2 (the same choice as for expf), in which
// each polynomial step and the fast reduction are fused multiply-adds.

struct SinCosTable {
    double sign[4];               // sign of the sine in quadrants 0..3
    double hpi_inv, hpi;          // 2/pi * 2^24, pi/2
    double c0, c1, c2, c3, c4;    // cosine polynomial
    double s1, s2, s3;            // sine polynomial
};
// Entry 1 negates the cosine polynomial (quadrants 2 and 3).
constexpr SinCosTable kSinCos[2] = {
    {{1.0, -1.0, -1.0, 1.0}, 0x1.45f306dc9c883p+23, 0x1.921fb54442d18p+0, 0x1p+0, -0x1.ffffffd0c621cp-2,
     0x1.55553e1068f19p-5, -0x1.6c087e89a359dp-10, 0x1.99343027bf8c3p-16, -0x1.555545995a603p-3,
     0x1.1107605230bc4p-7, -0x1.994eb3774cf24p-13},
    {{1.0, -1.0, -1.0, 1.0}, 0x1.45f306dc9c883p+23, 0x1.921fb54442d18p+0, -0x1p+0, 0x1.ffffffd0c621cp-2,
     -0x1.55553e1068f19p-5, 0x1.6c087e89a359dp-10, -0x1.99343027bf8c3p-16, -0x1.555545995a603p-3,
     0x1.1107605230bc4p-7, -0x1.994eb3774cf24p-13},
};
// Windows of the bits of 2/pi = 0.a2f9836e4e441529fc2757d1f534ddc0db62...:
// entry k holds hex digits 2k-6 .. 2k+1 of the fraction (fewer at the start).
struct InvPio4 {
    uint32_t w[24];
};
constexpr InvPio4 kInvPio4 = {{
    0xa2u, 0xa2f9u, 0xa2f983u, 0xa2f9836eu, 0xf9836e4eu, 0x836e4e44u, 0x6e4e4415u, 0x4e441529u,
    0x441529fcu, 0x1529fc27u, 0x29fc2757u, 0xfc2757d1u, 0x2757d1f5u, 0x57d1f534u, 0xd1f534ddu, 0xf534ddc0u,
    0x34ddc0dbu, 0xddc0db62u, 0xc0db6295u, 0xdb629599u, 0x6295993cu, 0x95993c43u, 0x993c4390u, 0x3c439041u,
}};

MRML_HD double madd(double a, double b, double c, bool fused) { return fused ? __builtin_fma(a, b, c) : a * b + c; }

// sin (n even) or cos (n odd) of the reduced argument x, x2 = x*x.
MRML_HD float sincos_poly(double x, double x2, const SinCosTable &p, int n, bool fused)
{
    if ((n & 1) == 0) {
        const double x3 = x * x2;
        const double s1 = madd(x2, p.s3, p.s2, fused);
        const double x7 = x3 * x2;
        const double s = madd(x3, p.s1, x, fused);
        return (float)madd(x7, s1, s, fused);
    }
    const double x4 = x2 * x2;
    const double c2 = madd(x2, p.c4, p.c3, fused);
    const double c1 = madd(x2, p.c1, p.c0, fused);
    const double x6 = x4 * x2;
    const double c = madd(x4, p.c2, c1, fused);
    return (float)madd(x6, c2, c, fused);
}

// x - n pi/2 for |x| < 120, n = round(x 2/pi).
MRML_HD double reduce_fast(double x, const SinCosTable &p, int &n, bool fused)
{
    const double r = x * p.hpi_inv;
    n = ((int32_t)r + 0x800000) >> 24;
    return madd(-(double)n, p.hpi, x, fused);
}

// Payne-Hanek: x mod pi/2 (scaled by 2^-62 * 2 pi) and the quadrant, from the
// float's bits.
MRML_HD double reduce_large(uint32_t xi, int &np)
{
    const uint32_t *arr = &kInvPio4.w[(xi >> 26) & 15];
    const int shift = (xi >> 23) & 7;
    xi = (xi & 0xffffffu) | 0x800000u;
    xi <<= shift;
    uint64_t res0 = (uint64_t)(uint32_t)(xi * arr[0]);
    const uint64_t res1 = (uint64_t)xi * arr[4];
    const uint64_t res2 = (uint64_t)xi * arr[8];
    res0 = (res2 >> 32) | (res0 << 32);
    res0 += res1;
    const uint64_t n = (res0 + (1ull << 61)) >> 62;
    res0 -= n << 62;
    np = (int)n;
    return (double)(int64_t)res0 * 0x1.921fb54442d18p-62;
}

// COS = false: sinf, true: cosf.
template <bool COS>
MRML_HD float sincosf1(float y, bool fused)
{
    const uint32_t top = (f2u(y) >> 20) & 0x7ffu;
    double x = y;
    if (top < ((f2u(0x1.921fb6p-1f) >> 20) & 0x7ffu)) {  // |y| < pi/4 (as a float)
        if (top < ((f2u(0x1p-12f) >> 20) & 0x7ffu)) return COS ? 1.0f : y;
        return sincos_poly(x, x * x, kSinCos[0], COS ? 1 : 0, fused);
    }
    int n;
    if (top < ((f2u(120.0f) >> 20) & 0x7ffu)) {
        x = reduce_fast(x, kSinCos[0], n, fused);
        const double s = kSinCos[0].sign[n & 3];
        const SinCosTable &p = kSinCos[(n & 2) ? 1 : 0];
        return sincos_poly(x * s, x * x, p, COS ? n ^ 1 : n, fused);
    }
    if (top < ((f2u(__builtin_inff()) >> 20) & 0x7ffu)) {
        const uint32_t xi = f2u(y);
        const int sign = (int)(xi >> 31);
        x = reduce_large(xi, n);
        const double s = kSinCos[0].sign[(n + sign) & 3];
        const SinCosTable &p = kSinCos[((n + sign) & 2) ? 1 : 0];
        return sincos_poly(x * s, x * x, p, COS ? n ^ 1 : n, fused);
    }
    return (y - y) / (y - y);  // inf or nan: nan
}

MRML_HD float sinf(float x, bool fused) { return sincosf1<false>(x, fused); }
MRML_HD float cosf(float x, bool fused) { return sincosf1<true>(x, fused); }

}  // namespace mrml_libm
