// zi_expf.hpp -- the reference's f32 exponential, for host and device code.
//
// The reference builds without libc (build.zig:14, link_libc = false), so
// every f32 @exp it evaluates on the sampling path (src/sampler.zig:219, 222,
// 230, 240; the softcap body, src/model.zig:2505) is a call to the compiler
// runtime's expf, a port of musl's expf (itself FreeBSD's e_expf.c).  That
// algorithm is restated here from its published form, in f32 throughout:
//   |x| > ln2/2:  k = trunc(x/ln2 +- 1/2) (k = +-1 below 1.5 ln2),
//                 hi = x - k*ln2hi (exact), lo = k*ln2lo, r = hi - lo;
//   |x| > 2^-13:  k = 0, r = x;   otherwise 1 + x.
//   c = r - r^2 (P1 + r^2 P2),  y = 1 + (r c / (2 - c) - lo + hi),
//   result y * 2^k (one rounding, as scalbnf).
// It is within 1 ulp of exp(x) but not correctly rounded: it differs from the
// correctly rounded value on about 0.8% of arguments in [-20, 0].  Compile
// without floating-point contraction: every step rounds to f32 on its own.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

namespace zi {

__host__ __device__ inline float zf_from_bits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
__host__ __device__ inline uint32_t zf_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

// y * 2^n with a single rounding (scalbnf's steps).
__host__ __device__ inline float zscalbnf(float y, int n) {
    if (n > 127) {
        y *= 0x1p127f;
        n -= 127;
        if (n > 127) {
            y *= 0x1p127f;
            n -= 127;
            if (n > 127) n = 127;
        }
    } else if (n < -126) {
        y *= 0x1p-102f;  // 2^-126 * 2^24
        n += 102;
        if (n < -126) {
            y *= 0x1p-102f;
            n += 102;
            if (n < -126) n = -126;
        }
    }
    return y * zf_from_bits((uint32_t)(0x7f + n) << 23);
}

__host__ __device__ inline float zexpf(float x) {
    const float ln2hi = zf_from_bits(0x3f317200u);   // 6.9314575195e-1
    const float ln2lo = zf_from_bits(0x35bfbe8eu);   // 1.4286067653e-6
    const float invln2 = zf_from_bits(0x3fb8aa3bu);  // 1.4426950216e+0
    const float P1 = 11184783.0f * 0x1p-26f;         // 0xaaaa8f.0p-26 = 1.6666625440e-1
    const float P2 = -11883029.0f * 0x1p-32f;        // -0xb55215.0p-32 = -2.7667332906e-3
    uint32_t hx = zf_bits(x);
    const int sign = (int)(hx >> 31);
    hx &= 0x7fffffffu;
    if (hx >= 0x42aeac50u) {  // |x| >= 87.33655 or NaN
        if (hx > 0x7f800000u) return x;                       // NaN
        if (hx >= 0x42b17218u && !sign) return x * 0x1p127f;  // x >= 88.722839: overflow
        if (sign && hx >= 0x42cff1b5u) return 0.0f;           // x <= -103.972084: underflow
    }
    int k;
    float hi, lo;
    if (hx > 0x3eb17218u) {  // |x| > ln2 / 2
        if (hx > 0x3f851592u) k = (int)(invln2 * x + (sign ? -0.5f : 0.5f));  // |x| > 1.5 ln2
        else k = 1 - sign - sign;
        const float fk = (float)k;
        hi = x - fk * ln2hi;
        lo = fk * ln2lo;
        x = hi - lo;
    } else if (hx > 0x39000000u) {  // |x| > 2^-13
        k = 0;
        hi = x;
        lo = 0.0f;
    } else {
        return 1.0f + x;
    }
    const float xx = x * x;
    const float c = x - xx * (P1 + xx * P2);
    const float y = 1.0f + (x * c / (2.0f - c) - lo + hi);
    return k == 0 ? y : zscalbnf(y, k);
}

// The same function without branches, for per-element use on the device
// (the branches above diverge within a wave).  Every input gives zexpf's bits:
//  - k = 0 (|x| <= ln2/2) is the general reduction with fk = 0: x - 0*ln2hi
//    = x and 0*ln2lo = 0 exactly, so hi = x, lo = 0, r = x;
//  - y * 2^k with k in [-150, 128] as y * 2^(k>>1) * 2^(k - (k>>1)): the first
//    product is exact (|y| in [0.7, 1.5], the scale within 2^+-75), so the
//    second rounds once, as scalbnf does;
//  - the tiny and special cases are selected at the end.
// Checked equal to zexpf on all 2^32 inputs.
__host__ __device__ inline float zexpf_nb(float x0) {
    const float ln2hi = zf_from_bits(0x3f317200u);
    const float ln2lo = zf_from_bits(0x35bfbe8eu);
    const float invln2 = zf_from_bits(0x3fb8aa3bu);
    const float P1 = 11184783.0f * 0x1p-26f;
    const float P2 = -11883029.0f * 0x1p-32f;
    const uint32_t ux = zf_bits(x0);
    const uint32_t hx = ux & 0x7fffffffu;
    const int sign = (int)(ux >> 31);
    float t = invln2 * x0 + (sign ? -0.5f : 0.5f);
    t = fminf(fmaxf(t, -200.0f), 200.0f);  // only |x| < 104 keeps its k; NaN -> a bound
    int k = (int)t;
    k = hx > 0x3f851592u ? k : (hx > 0x3eb17218u ? 1 - sign - sign : 0);
    const float fk = (float)k;
    const float hi = x0 - fk * ln2hi;
    const float lo = fk * ln2lo;
    const float x = hi - lo;
    const float xx = x * x;
    const float c = x - xx * (P1 + xx * P2);
    const float y = 1.0f + (x * c / (2.0f - c) - lo + hi);
    const int k1 = k >> 1, k2 = k - k1;
    float r = (y * zf_from_bits((uint32_t)(0x7f + k1) << 23)) * zf_from_bits((uint32_t)(0x7f + k2) << 23);
    r = hx > 0x39000000u ? r : 1.0f + x0;
    r = (hx >= 0x42b17218u && !sign) ? x0 * 0x1p127f : r;
    r = (sign && hx >= 0x42cff1b5u) ? 0.0f : r;
    return hx > 0x7f800000u ? x0 : r;
}

}  // namespace zi
