// zi_pow.hpp -- f32 pow as Zig's std.math.pow computes it, shared by the host
// and the device so that DRY penalties agree bit for bit.
//
// src/sampler.zig:182 takes the DRY penalty as std.math.pow(f32, base, e).
// Zig's std.math.pow (lib/std/math/pow.zig, Zig 0.17.1; not in the reference
// tree) follows Go's math.Pow: the special cases, then x^yf through
// exp(yf * log(x)) for the fractional part and x^yi by repeated squaring of
// frexp(x)'s significand with the exponent carried apart, each product
// rounded to f32, and a final scalbn.  exp and log are taken as f64 results
// rounded to f32 (exp32 / log32).
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace zi {

__host__ __device__ inline float exp32_hd(float x) { return (float)exp((double)x); }
__host__ __device__ inline float log32_hd(float x) { return (float)log((double)x); }

__host__ __device__ inline bool pow_odd_integer(float y) {
    if (!(fabsf(y) < 16777216.0f)) return false;  // every f32 from 2^24 on is even
    const float t = truncf(y);
    return t == y && fmodf(t, 2.0f) != 0.0f;
}

__host__ __device__ inline float pow_zig(float x, float y) {
    const float inf = __builtin_inff();
    if (y == 0.0f || x == 1.0f) return 1.0f;
    if (x != x || y != y) return __builtin_nanf("");
    if (y == 1.0f) return x;
    if (x == 0.0f) {
        if (y < 0.0f) return pow_odd_integer(y) ? copysignf(inf, x) : inf;
        return pow_odd_integer(y) ? x : 0.0f;
    }
    if (y == inf || y == -inf) {
        if (x == -1.0f) return 1.0f;
        return ((fabsf(x) < 1.0f) == (y > 0.0f)) ? 0.0f : inf;
    }
    if (x == inf || x == -inf) {
        if (x < 0.0f) return pow_zig(1.0f / x, -y);
        return y < 0.0f ? 0.0f : inf;
    }
    if (y == 0.5f) return sqrtf(x);
    if (y == -0.5f) return 1.0f / sqrtf(x);
    float yi;
    float yf = modff(fabsf(y), &yi);
    if (yf != 0.0f && x < 0.0f) return __builtin_nanf("");
    if (yi >= 2147483648.0f) {  // a large even integer: overflow or underflow except for x = -1
        if (x == -1.0f) return 1.0f;
        return ((fabsf(x) < 1.0f) == (y > 0.0f)) ? 0.0f : inf;
    }
    float a1 = 1.0f;
    int ae = 0;
    if (yf != 0.0f) {
        if (yf > 0.5f) {
            yf -= 1.0f;
            yi += 1.0f;
        }
        a1 = exp32_hd(yf * log32_hd(x));
    }
    int xe;
    float x1 = frexpf(x, &xe);
    for (int32_t i = (int32_t)yi; i != 0; i >>= 1) {
        if (xe < -(1 << 9) || (1 << 9) < xe) {  // catastrophic overflow: scalbn settles it
            ae += xe;
            break;
        }
        if (i & 1) {
            a1 *= x1;
            ae += xe;
        }
        x1 *= x1;
        xe <<= 1;
        if (x1 < 0.5f) {
            x1 += x1;
            xe -= 1;
        }
    }
    if (y < 0.0f) {
        a1 = 1.0f / a1;
        ae = -ae;
    }
    return ldexpf(a1, ae);
}

// The DRY penalty of a repeat of length rlen (src/sampler.zig:178-184):
// mult * pow(base, min(rlen - allowed, max_exp)), max_exp = 88 / log(base)
// for base > 1.0001, else 100.
__host__ __device__ inline float dry_penalty(uint32_t rlen, float mult, float base, uint32_t allowed) {
    const float max_exp = (base > 1.0001f) ? 88.0f / log32_hd(base) : 100.0f;
    const float rexp = (float)(rlen - allowed);
    const float e = rexp < max_exp ? rexp : max_exp;
    return mult * pow_zig(base, e);
}

}  // namespace zi
