// zi_common.hpp -- device helpers shared by the gfx950 sampling kernels.
//
// Layout conventions used by every kernel:
//  * One row of V logits is split into G chunks of CH elements (CH a multiple
//    of 64); chunk g covers ids [g*CH, min(V, (g+1)*CH)) and is handled by one
//    512-thread workgroup (8 wave64s).
//  * Thread t of a workgroup loads NV 16-byte vectors: vector j holds the
//    VEC = 16/sizeof(T) consecutive ids starting at c0 + (j*512 + t)*VEC, so
//    each wave's load instruction reads 1 KiB of contiguous memory.
//  * Ordering keys: okey() maps a float to a uint32 whose unsigned order is
//    the float order with -0 == +0; ckey() appends ~id so that larger 64-bit
//    keys mean (value desc, id asc), the order of the reference's top-k
//    (src/sampler.zig:203-209).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "zi_expf.hpp"

namespace zi {

constexpr int kThreads = 512;
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

// The reference's f32 exp (its compiler runtime's expf, zi_expf.hpp), used
// wherever the reference evaluates @exp on f32: the sampler's terms and
// weights and the softcap body.  The branch-free form, which gives the same
// bits for every input; the CPU oracle evaluates the published steps
// (oracle/or_zexpf).
__device__ __forceinline__ float exp32(float x) { return zexpf_nb(x); }

// Final-logit softcap, the vectorized body of src/model.zig:2492-2510:
// z = l * (1/cap) clamped to [-9, 9], tanh = (e - 1) / (e + 1) with e = exp(2z),
// l = cap * tanh, every step rounded to f32.
__device__ __forceinline__ float softcap_f(float l, float cap, float inv_cap) {
    const float z = fminf(fmaxf(l * inv_cap, -9.0f), 9.0f);
    const float e2z = exp32(z * 2.0f);
    return cap * ((e2z - 1.0f) / (e2z + 1.0f));
}

// The softcap's scalar tail (src/model.zig:2511-2513), ids >= 32*floor(V/32):
// l = cap * tanh(l / cap) with a true division and no clamp; tanh is the f64
// tanh rounded once to f32, as in the CPU oracle.
__device__ __forceinline__ float softcap_tail_f(float l, float cap) { return cap * (float)tanh((double)(l / cap)); }

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0)); }

// Number of set bits of `m` below this lane.
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

// Largest T such that at least r of the wave's keys (N per lane) are >= T
// (0 if fewer than r keys are nonzero).  32-step bisection on ballot counts;
// T is wave-uniform.
template <int N>
__device__ __forceinline__ uint32_t wave_kth_largest(const uint32_t (&key)[N], int r) {
    uint32_t T = 0;
#pragma unroll
    for (int b = 31; b >= 0; --b) {
        const uint32_t cand = T | (1u << b);
        int c = 0;
#pragma unroll
        for (int i = 0; i < N; ++i) c += __popcll(ballot(key[i] >= cand));
        if (c >= r) T = cand;
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

// Orders this wave's LDS writes before its later LDS reads by other lanes
// (cross-lane exchange through LDS within one wave).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
    return v;
}

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    uint32_t lo = __shfl_xor((uint32_t)v, m), hi = __shfl_xor((uint32_t)(v >> 32), m);
    return ((uint64_t)hi << 32) | lo;
}

// Value of `v` held by lane (this lane XOR D), D a power of two below 64,
// without going through LDS: quad_perm DPP for 1 and 2, row shifts for 4,
// row_ror:8 for 8, and the gfx950 permlane swaps for 16 and 32.
template <int D>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
    static_assert(D == 1 || D == 2 || D == 4 || D == 8 || D == 16 || D == 32, "lane_xor distance");
    if constexpr (D == 1) {
        return __builtin_amdgcn_update_dpp(0u, v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (D == 2) {
        return __builtin_amdgcn_update_dpp(0u, v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (D == 4) {
        const uint32_t up = __builtin_amdgcn_update_dpp(0u, v, 0x104, 0xF, 0xF, false);  // lane + 4
        const uint32_t dn = __builtin_amdgcn_update_dpp(0u, v, 0x114, 0xF, 0xF, false);  // lane - 4
        return (lane_id() & 4) ? dn : up;
    } else if constexpr (D == 8) {
        return __builtin_amdgcn_update_dpp(0u, v, 0x128, 0xF, 0xF, false);  // row_ror:8
    } else if constexpr (D == 16) {
        // r[0] = rows (0,0,2,2), r[1] = rows (1,1,3,3) of v
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane_id() & 16) ? r[0] : r[1];
    } else {
        // r[0] = halves (lo,lo), r[1] = halves (hi,hi) of v
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane_id() & 32) ? r[0] : r[1];
    }
}

// Bitonic sort of one 32-bit key per lane, descending over the wave (all 64
// lanes active); every exchange is a DPP / permlane move.
template <int D, int SIZE>
__device__ __forceinline__ uint32_t sort_step_u32(uint32_t x) {
    const int lane = lane_id();
    const uint32_t p = lane_xor<D>(x);
    const bool keep_max = ((lane & D) == 0) == ((lane & SIZE) == 0);
    return keep_max ? max(x, p) : min(x, p);
}

template <int D, int SIZE>
__device__ __forceinline__ uint32_t sort_clean_u32(uint32_t x) {
    x = sort_step_u32<D, SIZE>(x);
    if constexpr (D > 1) x = sort_clean_u32<D / 2, SIZE>(x);
    return x;
}

template <int SIZE>
__device__ __forceinline__ uint32_t sort_from_u32(uint32_t x) {
    x = sort_clean_u32<SIZE / 2, SIZE>(x);
    if constexpr (SIZE < 64) x = sort_from_u32<SIZE * 2>(x);
    return x;
}

__device__ __forceinline__ uint32_t wave_sort_desc_u32(uint32_t x) { return sort_from_u32<2>(x); }

// Sequential f32 sum over s[i0, i1), added in index order onto `acc`, by the
// one calling lane: the reference's loop order exactly, at one dependent add
// per term (4 terms per LDS read).
__device__ __forceinline__ float lane_sum(const float *s, int i0, int i1, float acc) {
    int i = i0;
    for (; i < i1 && (i & 3); ++i) acc = acc + s[i];
    for (; i + 4 <= i1; i += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(s + i);
        acc = acc + v.x;
        acc = acc + v.y;
        acc = acc + v.z;
        acc = acc + v.w;
    }
    for (; i < i1; ++i) acc = acc + s[i];
    return acc;
}

// 1 + the first i < end whose prefix sum fl(...fl(0 + s_0) ... + s_i) is
// >= thr (`none` if there is none).  The terms are >= 0, so the rounded
// prefixes never decrease and a block of four can be tested by its last.
__device__ __forceinline__ int first_reach(const float *s, int end, float thr, int none) {
    float acc = 0.0f;
    int i = 0;
    for (; i + 4 <= end; i += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(s + i);
        const float p0 = acc + v.x, p1 = p0 + v.y, p2 = p1 + v.z, p3 = p2 + v.w;
        if (p3 >= thr) return i + (p0 >= thr ? 1 : p1 >= thr ? 2 : p2 >= thr ? 3 : 4);
        acc = p3;
    }
    for (; i < end; ++i) {
        acc = acc + s[i];
        if (acc >= thr) return i + 1;
    }
    return none;
}

// The first i in [start, end) at which r = fl(r - s_i), applied in order
// from i = start, is <= 0, else end - 1 (the draw's fallback).  The terms are
// >= 0, so r never increases and a block of four is tested by its last.
__device__ __forceinline__ int first_drop(const float *s, int start, int end, float r) {
    int i = start;
    for (; i < end && (i & 3); ++i) {
        r = r - s[i];
        if (r <= 0.0f) return i;
    }
    for (; i + 4 <= end; i += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(s + i);
        const float d0 = r - v.x, d1 = d0 - v.y, d2 = d1 - v.z, d3 = d2 - v.w;
        if (d3 <= 0.0f) return i + (d0 <= 0.0f ? 0 : d1 <= 0.0f ? 1 : d2 <= 0.0f ? 2 : 3);
        r = d3;
    }
    for (; i < end; ++i) {
        r = r - s[i];
        if (r <= 0.0f) return i;
    }
    return end - 1;
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
