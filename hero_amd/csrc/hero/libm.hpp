// libm.hpp -- single-precision exp, log1p, expm1 and tanh for host and device
// that return exactly what the x86-64 glibc 2.35 expf / log1pf / expm1f / tanhf
// return, for every input.
//
// The reference calls std::exp and std::log1p on floats, i.e. glibc's expf
// and log1pf, and neither is correctly rounded; a last-bit difference in one
// of them can flip an int8 activation quantization several layers later. So
// the device evaluates the same published methods with the same operation
// order:
//   expf   -- the table-driven method of ARM's optimized-routines (the one in
//             glibc): x*N/ln2 = k + r with N = 32 and round-to-nearest k,
//             2^(k/N) from a 32-entry table of 2^(i/32), and 2^(r/N) from a
//             degree-3 polynomial, all in fp64; glibc's x86-64 build fuses
//             the reduction r = x*N/ln2 - k into one fma, and so does this.
//   log1pf -- fdlibm's log1p (Sun Microsystems, freely distributable) in its
//             single-precision form: 1+x = 2^k (1+f) with a correction term,
//             then log(1+f) = f - s(f - R) with s = f/(2+f) and a degree-7
//             polynomial R in s^2, in fp32.
//   expm1f -- fdlibm's expm1 in single precision: x = k ln2 + r (ln2 split in
//             hi/lo parts, with the rounding error c of the reduction), a
//             degree-5 rational correction in r^2/2, and the scaling by 2^k
//             folded into the exponent bits.
//   tanhf  -- fdlibm's tanh: 1 - 2/(expm1(2|x|) + 2) for |x| >= 1,
//             -t/(t + 2) with t = expm1(-2|x|) below, +-1 from |x| >= 22.
// All four were checked against glibc on all 2^32 inputs (0 differences); the
// tests repeat that check on a dense sample and on the hard cases.
// Build with -ffp-contract=off: every operation below rounds once.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "hero/fp16.hpp"

namespace hero {

__host__ __device__ inline double bits_f64(uint64_t u) {
    union {
        uint64_t u;
        double d;
    } v{u};
    return v.d;
}
__host__ __device__ inline uint64_t f64_bits(double d) {
    union {
        double d;
        uint64_t u;
    } v{d};
    return v.u;
}

// bits of 2^(i/32) (correctly rounded) minus (i << 47)
__host__ __device__ inline uint64_t exp2_table(int i) {
    constexpr uint64_t t[32] = {
        0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
        0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
        0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
        0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
        0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
        0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
        0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
        0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
    };
    return t[i];
}

// `tab(i)` returns exp2_table(i); kernels that cannot afford a global-memory
// read per call (one in flight behind other loads waits for all of them) pass
// a copy of the table held in shared memory
//
// Branch-free: the table path runs for every input (for |x| >= 88, inf and nan
// its value is discarded) and the special cases are selected afterwards, so a
// wave never splits and independent calls interleave.
template <class Tab>
__host__ __device__ inline float expf_glibc_with(float x, const Tab& tab) {
    const uint32_t ix = f32_bits(x);
    const uint32_t abstop = (ix >> 20) & 0x7ff;
    constexpr double inv_ln2_n = 0x1.71547652b82fep0 * 32;
    constexpr double shift = 0x1.8p+52;
    constexpr double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32, c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = double(x);
    const double z = inv_ln2_n * xd;
    double kd = z + shift;
    const uint64_t ki = f64_bits(kd);
    kd -= shift;
    const double r = ::fma(inv_ln2_n, xd, -kd);
    const double s = bits_f64(tab(int(ki % 32)) + (ki << 47));
    const double p = c0 * r + c1;
    const double r2 = r * r;
    double y = c2 * r + 1.0;
    y = p * r2 + y;
    y = y * s;
    const float main = float(y);
    // |x| >= 88, inf or nan: exp(-inf) = 0; +inf and nan give x + x; overflow
    // to +inf; underflow to 0; otherwise the table path's value
    const float special = ix == 0xff800000u ? 0.f
                          : abstop >= 0x7f8 ? x + x
                          : x > 0x1.62e42ep6f ? bits_f32(0x7f800000u)
                          : x < -0x1.9fe368p6f ? 0.f
                          : main;
    return abstop >= 0x42b ? special : main;
}

__host__ __device__ inline float expf_glibc(float x) {
    return expf_glibc_with(x, [](int i) { return exp2_table(i); });
}

// log1pf below restates fdlibm's single-precision log1p (s_log1pf.c, the
// algorithm glibc uses), whose permission notice follows:
//
// ====================================================
// Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//
// Developed at SunPro, a Sun Microsystems, Inc. business.
// Permission to use, copy, modify, and distribute this
// software is freely granted, provided that this notice
// is preserved.
// ====================================================
__host__ __device__ inline float log1pf_glibc(float x) {
    const float ln2_hi = bits_f32(0x3f317180u), ln2_lo = bits_f32(0x3717f7d1u);
    const float lp1 = bits_f32(0x3f2aaaabu), lp2 = bits_f32(0x3ecccccdu), lp3 = bits_f32(0x3e924925u), lp4 = bits_f32(0x3e638e29u),
                lp5 = bits_f32(0x3e3a3325u), lp6 = bits_f32(0x3e1cd04fu), lp7 = bits_f32(0x3e178897u);
    const int32_t hx = int32_t(f32_bits(x));
    const int32_t ax = hx & 0x7fffffff;
    float f = 0.f, c = 0.f, u;
    int32_t k = 1, hu = 0;
    if (hx < 0x3ed413d7) {  // x < 0.41422
        if (ax >= 0x3f800000) return x == -1.f ? bits_f32(0xff800000u) : bits_f32(0x7fc00000u);  // -inf, nan
        if (ax < 0x31000000) return ax < 0x24800000 ? x : x - x * x * 0.5f;  // |x| < 2^-29
        if (hx > 0 || hx <= int32_t(0xbe95f61fu)) {  // -0.2929 < x < 0.41422
            k = 0;
            f = x;
            hu = 1;
        }
    } else if (hx >= 0x7f800000) {
        return x + x;
    }
    if (k != 0) {
        if (hx < 0x5a000000) {
            u = 1.f + x;
            hu = int32_t(f32_bits(u));
            k = (hu >> 23) - 127;
            c = k > 0 ? 1.f - (u - x) : x - (u - 1.f);  // the rounding error of 1+x
            c /= u;
        } else {
            u = x;
            hu = int32_t(f32_bits(u));
            k = (hu >> 23) - 127;
            c = 0.f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = bits_f32(uint32_t(hu) | 0x3f800000u);
        } else {
            k += 1;
            u = bits_f32(uint32_t(hu) | 0x3f000000u);
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.f;
    }
    const float hfsq = 0.5f * f * f;
    if (hu == 0) {  // |f| < 2^-20
        if (f == 0.f) {
            if (k == 0) return 0.f;
            c += float(k) * ln2_lo;
            return float(k) * ln2_hi + c;
        }
        const float R = hfsq * (1.f - 0.66666666666666666f * f);
        if (k == 0) return f - R;
        return float(k) * ln2_hi - ((R - (float(k) * ln2_lo + c)) - f);
    }
    const float s = f / (2.f + f);
    const float z = s * s;
    const float R = z * (lp1 + z * (lp2 + z * (lp3 + z * (lp4 + z * (lp5 + z * (lp6 + z * lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + R));
    return float(k) * ln2_hi - ((hfsq - (s * (hfsq + R) + (float(k) * ln2_lo + c))) - f);
}

// expm1f and tanhf below restate fdlibm's single-precision expm1 and tanh
// (s_expm1f.c, s_tanhf.c; the algorithms glibc 2.35 uses), under the same Sun
// Microsystems permission notice as log1pf above.
__host__ __device__ inline float expm1f_glibc(float x) {
    const float o_threshold = bits_f32(0x42b17180u), ln2_hi = bits_f32(0x3f317180u), ln2_lo = bits_f32(0x3717f7d1u),
                invln2 = bits_f32(0x3fb8aa3bu);
    const float q1 = bits_f32(0xbd088889u), q2 = bits_f32(0x3ad00d01u), q3 = bits_f32(0xb8a670cdu), q4 = bits_f32(0x36867e54u),
                q5 = bits_f32(0xb457edbbu);
    uint32_t hx = f32_bits(x);
    const uint32_t xsb = hx & 0x80000000u;
    hx &= 0x7fffffffu;
    float hi, lo, c = 0.f, t, e, y;
    int32_t k;
    if (hx >= 0x4195b844u) {  // |x| >= 27 ln2
        if (hx >= 0x42b17218u) {  // |x| >= 88.72
            if (hx > 0x7f800000u) return x + x;  // nan
            if (hx == 0x7f800000u) return xsb == 0 ? x : -1.f;
            if (x > o_threshold) return bits_f32(0x7f800000u);  // overflow
        }
        if (xsb != 0) return -1.f;
    }
    if (hx > 0x3eb17218u) {  // |x| > ln2 / 2: reduce
        if (hx < 0x3f851592u) {  // and < 1.5 ln2
            if (xsb == 0) {
                hi = x - ln2_hi;
                lo = ln2_lo;
                k = 1;
            } else {
                hi = x + ln2_hi;
                lo = -ln2_lo;
                k = -1;
            }
        } else {
            k = int32_t(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
            t = float(k);
            hi = x - t * ln2_hi;  // exact
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {  // |x| < 2^-25
        return x;
    } else {
        k = 0;
    }
    const float hfx = 0.5f * x, hxs = x * hfx;
    const float r1 = 1.f + hxs * (q1 + hxs * (q2 + hxs * (q3 + hxs * (q4 + hxs * q5))));
    t = 3.f - r1 * hfx;
    e = hxs * ((r1 - t) / (6.f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = x * (e - c) - c;
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) return x < -0.25f ? -2.f * (e - (x + 0.5f)) : 1.f + 2.f * (x - e);
    if (k <= -2 || k > 56) {  // exp(x) - 1 is exp(x) to working precision
        y = 1.f - (e - x);
        y = k == 128 ? y * 2.f * bits_f32(0x7f000000u) : bits_f32(f32_bits(y) + (uint32_t(k) << 23));
        return y - 1.f;
    }
    if (k < 23) {
        t = bits_f32(0x3f800000u - (0x1000000u >> k));  // 1 - 2^-k
        y = t - (e - x);
    } else {
        t = bits_f32(uint32_t(0x7f - k) << 23);  // 2^-k
        y = x - (e + t);
        y += 1.f;
    }
    return bits_f32(f32_bits(y) + (uint32_t(k) << 23));
}

__host__ __device__ inline float tanhf_glibc(float x) {
    const int32_t jx = int32_t(f32_bits(x)), ix = jx & 0x7fffffff;
    if (ix >= 0x7f800000) return jx >= 0 ? 1.f / x + 1.f : 1.f / x - 1.f;  // +-inf -> +-1, nan -> nan
    float z;
    if (ix < 0x41b00000) {  // |x| < 22
        if (ix == 0) return x;
        if (ix < 0x24000000) return x * (1.f + x);  // |x| < 2^-55
        const float ax = jx >= 0 ? x : -x;
        if (ix >= 0x3f800000) {
            const float t = expm1f_glibc(2.f * ax);
            z = 1.f - 2.f / (t + 2.f);
        } else {
            const float t = expm1f_glibc(-2.f * ax);
            z = -t / (t + 2.f);
        }
    } else {
        z = 1.f;
    }
    return jx >= 0 ? z : -z;
}

}  // namespace hero
