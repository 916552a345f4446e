// zi_common.hpp -- device helpers shared by the gfx950 sampling kernels.
//
// Layout conventions used by every kernel:
//  * One row of V logits is split into G chunks of CH elements (CH a multiple
//    of 64); chunk g covers ids [g*CH, min(V, (g+1)*CH)) and is handled by one
//    256-thread workgroup (4 wave64s).
//  * Thread t of a workgroup loads NV 16-byte vectors: vector j holds the
//    VEC = 16/sizeof(T) consecutive ids starting at c0 + (j*256 + t)*VEC, so
//    each wave's load instruction reads 1 KiB of contiguous memory.
//  * Ordering keys: okey() maps a float to a uint32 whose unsigned order is
//    the float order with -0 == +0; ckey() appends ~id so that larger 64-bit
//    keys mean (value desc, id asc), the order of the reference's top-k
//    (src/sampler.zig:203-209).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zi {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr uint32_t kNegInfKey = 0x007FFFFFu;  // okey(-inf)

__device__ __forceinline__ uint32_t okey(float v) {
    uint32_t b = __float_as_uint(v);
    b = (b == 0x80000000u) ? 0u : b;  // -0 ranks equal to +0
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float okey_inv(uint32_t k) {
    uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __uint_as_float(b);
}

__device__ __forceinline__ uint64_t ckey(float v, uint32_t id) {
    return ((uint64_t)okey(v) << 32) | (uint64_t)(~id);
}

__device__ __forceinline__ uint32_t ckey_id(uint64_t k) { return ~(uint32_t)(k & 0xFFFFFFFFull); }

// Correctly rounded in practice: f64 exp rounded once to f32.  Used wherever a
// result must agree bit-for-bit with the CPU oracle (oracle/or_exp32).
__device__ __forceinline__ float exp32(float x) { return (float)exp((double)x); }

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0)); }

// Number of set bits of `m` below this lane.
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// Largest T such that at least r lanes of the wave hold key >= T (0 if fewer
// than r lanes have a nonzero key).  32-step bisection on ballot counts; T is
// wave-uniform.
__device__ __forceinline__ uint32_t wave_kth_largest(uint32_t key, int r) {
    uint32_t T = 0;
#pragma unroll
    for (int b = 31; b >= 0; --b) {
        uint32_t cand = T | (1u << b);
        if (__popcll(ballot(key >= cand)) >= r) T = cand;
    }
    return T;
}

// wave_shr:1 with `fill` entering lane 0.
__device__ __forceinline__ float shr1(float v, float fill) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(v), 0x138, 0xF, 0xF, false));
}

// Exact sequential f32 prefix over lanes: returns
//   P_i = fl(...fl(fl(carry + x_0) + x_1) ... + x_i)   (SUB=false)
//   P_i = fl(...fl(fl(carry - x_0) - x_1) ... - x_i)   (SUB=true)
// for lanes i < steps (lanes >= steps hold unspecified values).  Each step
// shifts the running values one lane up and applies one IEEE operation, so
// after s steps lanes < s hold their final sequential value; no reassociation
// happens.  All 64 lanes of the wave must be active.
template <bool SUB>
__device__ __forceinline__ float wave_serial_chain(float x, float carry, int steps) {
    float p = x;
    for (int s = 0; s < steps; ++s) {
        float prev = shr1(p, carry);
        p = SUB ? (prev - x) : (prev + x);
    }
    return p;
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    uint32_t lo = __shfl_xor((uint32_t)v, m), hi = __shfl_xor((uint32_t)(v >> 32), m);
    return ((uint64_t)hi << 32) | lo;
}

template <typename T>
struct VecTraits;
template <>
struct VecTraits<float> {
    static constexpr int VEC = 4;
};
template <>
struct VecTraits<uint16_t> {  // bf16 stored as raw 16-bit words
    static constexpr int VEC = 8;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Unpack one 16-byte vector into VEC floats.
template <typename T>
__device__ __forceinline__ void unpack(const uint4 &r, float *out);
template <>
__device__ __forceinline__ void unpack<float>(const uint4 &r, float *out) {
    out[0] = __uint_as_float(r.x);
    out[1] = __uint_as_float(r.y);
    out[2] = __uint_as_float(r.z);
    out[3] = __uint_as_float(r.w);
}
template <>
__device__ __forceinline__ void unpack<uint16_t>(const uint4 &r, float *out) {
    out[0] = bf16_lo(r.x); out[1] = bf16_hi(r.x);
    out[2] = bf16_lo(r.y); out[3] = bf16_hi(r.y);
    out[4] = bf16_lo(r.z); out[5] = bf16_hi(r.z);
    out[6] = bf16_lo(r.w); out[7] = bf16_hi(r.w);
}

}  // namespace zi
