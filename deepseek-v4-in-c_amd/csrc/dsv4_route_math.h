/* SPDX-License-Identifier: Apache-2.0 */
/* dsv4_route_math.h - the router's score transform, bit for bit as the
 * reference computes it on its host:
 *
 *   orig = sqrtf(softplus(x)),  softplus(x) = x > 20 ? x : log1pf(expf(x))
 *
 * (src/10_compute/dsv4_ops.c:43-46, 121-122). expf, log1pf and sqrtf are the
 * host C library's (glibc 2.35 on x86-64), so the device restates the
 * library's published algorithms operation for operation; only IEEE-rounded
 * adds, multiplies, divides and fused multiply-adds appear, which give the
 * same bits on the GPU as on the host. Compiled for the GPU (the library) and
 * for the host (tests/test_route_math.py checks every fp32 input of the
 * router's range against the host's libm).
 *
 *   expf    the exp2f-table method of ARM's optimized-routines, which glibc
 *           ships since 2.27 (sysdeps/ieee754/flt-32/e_expf.c): x / ln2 * 32
 *           rounded to an integer k, r = the remainder, 2^(k / 32) from a
 *           32-entry table of 2^(i / 32) with the exponent of k folded into
 *           its bits, and 2^(r / 32) by a cubic; all in double, one final
 *           rounding to float. x86-64 glibc runs the build of it with fused
 *           multiply-adds on CPUs that have FMA (the reference's host and the
 *           GPU box's), where the compiler fuses every multiply-add of the
 *           source: x / ln2 * 32 + shift, its remainder and the three
 *           polynomial steps are FMAs here. (With the remainder unfused, one
 *           input of [-104, 20], -0x1.f8cbb2p+5, rounds differently.)
 *   log1pf  fdlibm's float log1p (Sun Microsystems; glibc
 *           sysdeps/ieee754/flt-32/s_log1pf.c): 1 + x = 2^k (1 + f) with
 *           sqrt(2)/2 <= 1 + f < sqrt(2), a rounding correction c for the
 *           1 + x, s = f / (2 + f), log(1 + f) = f - (hfsq - s (hfsq + R(s^2)))
 *           with a degree-7 polynomial R, and k ln2 in two parts; in float.
 *   sqrtf   correctly rounded; the double square root of a float rounded
 *           once to float is correctly rounded.
 * The inputs that reach log1pf here are expf results: zero, subnormal or
 * positive. */
#ifndef DSV4_ROUTE_MATH_H
#define DSV4_ROUTE_MATH_H

#include <math.h>
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#define DSV4_HD __host__ __device__ __forceinline__
#define DSV4_TABLE static __device__ __constant__
#else
#define DSV4_HD static inline
#define DSV4_TABLE static
#endif
/* Every multiply-add below that is not written as fma() must round twice, as
 * in the library's build. clang keeps that under its default contraction
 * modes (on, fast-honor-pragmas: the pragma), not under -ffp-contract=fast;
 * gcc needs -ffp-contract=off. */
#if defined(__clang__)
#define DSV4_UNFUSED _Pragma("clang fp contract(off)")
#else
#define DSV4_UNFUSED
#endif

namespace dsv4_route {

DSV4_HD uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
DSV4_HD float fof(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
DSV4_HD uint64_t dbits(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
DSV4_HD double dof(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

/* 2^(i / 32) rounded to double, minus i << 47 in its bits (the exponent of
 * k is added back as k << 47) */
DSV4_TABLE const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

/* expf for the router's arguments (finite, x <= 20 here; the overflow,
 * underflow and NaN branches follow the library's). */
DSV4_HD float expf_lib(float x)
{
    DSV4_UNFUSED
    const double N = 32.0;
    const uint32_t abstop = (fbits(x) >> 20) & 0x7ff;
    if (abstop >= ((fbits(88.0f) >> 20) & 0x7ff)) {
        if (fbits(x) == fbits(-INFINITY)) return 0.0f;
        if (abstop >= ((fbits(INFINITY) >> 20) & 0x7ff)) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;              /* overflow  */
        if (x < -0x1.9fe368p6f) return 0.0f;                 /* underflow */
    }
    const double xd = (double)x;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * N;
    const double shift = 0x1.8p+52;
    double kd = fma(inv_ln2_n, xd, shift);
    const uint64_t ki = dbits(kd);
    kd -= shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    double z;
    uint64_t t = kExp2Tab[ki % 32];
    t += ki << (52 - 5);
    const double s = dof(t);
    z = fma(0x1.c6af84b912394p-5 / N / N / N, r, 0x1.ebfce50fac4f3p-3 / N / N);
    const double r2 = r * r;
    double y = fma(0x1.62e42ff0c52d6p-1 / N, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return (float)y;
}

/* log1pf for x >= 0 (and NaN / +inf as the library returns them) */
DSV4_HD float log1pf_lib(float x)
{
    DSV4_UNFUSED
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f;
    const float Lp1 = 6.6666668653e-01f, Lp2 = 4.0000000596e-01f, Lp3 = 2.8571429849e-01f,
                Lp4 = 2.2222198546e-01f, Lp5 = 1.8183572590e-01f, Lp6 = 1.5313838422e-01f,
                Lp7 = 1.4798198640e-01f;
    const int32_t hx = (int32_t)fbits(x);
    const int32_t ax = hx & 0x7fffffff;
    int32_t k = 1, hu = 0;
    float f = 0.0f, c = 0.0f;
    if (hx < 0x3ed413d7) {                 /* x < 0.41422 */
        if (ax >= 0x3f800000) return x == -1.0f ? -INFINITY : (x - x) / (x - x);
        if (ax < 0x31000000) {             /* |x| < 2^-29 */
            if (ax < 0x24800000) return x; /* |x| < 2^-54 */
            return x - x * x * 0.5f;
        }
        if (hx > 0 || hx <= (int32_t)0xbe95f61f) {   /* -0.2929 < x < 0.41422 */
            k = 0;
            f = x;
            hu = 1;
        }
    } else if (hx >= 0x7f800000) {
        return x + x;
    }
    if (k != 0) {
        float u;
        if (hx < 0x5a000000) {
            u = 1.0f + x;
            hu = (int32_t)fbits(u);
            k = (hu >> 23) - 127;
            c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);   /* correction term */
            c /= u;
        } else {
            u = x;
            hu = (int32_t)fbits(u);
            k = (hu >> 23) - 127;
            c = 0.0f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = fof((uint32_t)hu | 0x3f800000u);              /* normalize u */
        } else {
            k += 1;
            u = fof((uint32_t)hu | 0x3f000000u);              /* normalize u / 2 */
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    const float hfsq = 0.5f * f * f;
    if (hu == 0) {                         /* |f| < 2^-20 */
        if (f == 0.0f) {
            if (k == 0) return 0.0f;
            c += (float)k * ln2_lo;
            return (float)k * ln2_hi + c;
        }
        const float R = hfsq * (1.0f - 0.66666666666666666f * f);
        if (k == 0) return f - R;
        return (float)k * ln2_hi - ((R - ((float)k * ln2_lo + c)) - f);
    }
    const float s = f / (2.0f + f);
    const float z = s * s;
    const float R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + R));
    return (float)k * ln2_hi - ((hfsq - (s * (hfsq + R) + ((float)k * ln2_lo + c))) - f);
}

/* sqrt(softplus(x)), softplus's threshold at 20 as torch's */
DSV4_HD float route_orig(float x)
{
    DSV4_UNFUSED
    const float sp = x > 20.0f ? x : log1pf_lib(expf_lib(x));
    return (float)sqrt((double)sp);
}

} // namespace dsv4_route

#endif /* DSV4_ROUTE_MATH_H */
