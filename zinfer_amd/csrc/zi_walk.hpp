// zi_walk.hpp -- the reference's sequential f32 sums over a sorted row, exactly,
// in O(groups + binades) instead of one dependent addition per entry.
//
// The sums of src/sampler.zig:217-275 run entry by entry in the sorted order:
//   total = fl(total + t_i)   (:219, :236-242)   acc = fl(acc + t_i) until acc >= thr (:221-226)
//   r = fl(r - w_i) until r <= 0 (:270-275)
// with t_i >= 0.  A row here is a list of groups (value, count): count equal
// entries, whose terms are equal.  While the running value v stays in one
// binade, every f32 addition is an integer addition on v's grid: v = m*q with
// q = ulp(v) (2^-149 below 2^-125) and m < 2^24, and
//   fl(v + t) = (m + d) q,  d = t/q rounded to nearest, ties to an even m + d,
// as long as m + d < 2^24 (at 2^24 the grid coarsens).  A subtraction is the
// same with m - d, as long as the exact difference stays in the binade.  So a
// group of c copies adds c*d at once, except at a tie (t/q = n + 1/2), where
// the first copy's d depends on m's parity and every later one is the even
// choice.  A group is therefore a map from m's parity to (increment, parity);
// the maps compose associatively, so a wave scans 64 groups at once and only
// the group at which v leaves its binade (or reaches a threshold) is walked
// copy-run by copy-run, with that one crossing copy evaluated in f32.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "zi_expf.hpp"

namespace zi {

constexpr uint64_t kWalkSat = 1ull << 40;  // increments saturate here (any crossing is far below)

// v = m * 2^(qe - 150) with m < 2^24, qe >= 1 (v >= 0 finite).
struct WalkGrid {
    uint32_t m;
    int qe;
};
__host__ __device__ inline WalkGrid walk_grid(float v) {
    const uint32_t b = zf_bits(v);
    const int E = (int)(b >> 23);
    WalkGrid g;
    g.qe = E > 1 ? E : 1;
    g.m = E == 0 ? (b & 0x7fffffu) : ((b & 0x7fffffu) | 0x800000u);
    return g;
}
__host__ __device__ inline float walk_value(uint64_t m, int qe) {  // m * 2^(qe - 150), m < 2^24
    return (float)m * zf_from_bits(qe >= 24 ? (uint32_t)(qe - 23) << 23 : 1u << (qe - 1));
}

// t (>= 0, finite) on the grid 2^(qe - 150): t/q = n + f; kind 0: f < 1/2
// (d = n), 1: f = 1/2 (tie), 2: f > 1/2 (d = n + 1), 3: exact (d = n).
struct WalkTerm {
    uint64_t n;
    int kind;
};
__host__ __device__ inline WalkTerm walk_term(float t, int qe) {
    WalkTerm w;
    const uint32_t b = zf_bits(t);
    const int E = (int)(b >> 23);
    const uint64_t M = E == 0 ? (b & 0x7fffffu) : ((b & 0x7fffffu) | 0x800000u);
    const int s = (E > 1 ? E : 1) - qe;
    if (s >= 0) {
        w.n = s >= 17 ? kWalkSat : (M << s);
        if (w.n > kWalkSat) w.n = kWalkSat;
        w.kind = 3;
        return w;
    }
    const int sh = -s;
    if (sh > 25) {  // t < q / 2
        w.n = 0;
        w.kind = M == 0 ? 3 : 0;
        return w;
    }
    w.n = M >> sh;
    const uint64_t rem = M & ((1ull << sh) - 1), half = 1ull << (sh - 1);
    w.kind = rem == 0 ? 3 : (rem < half ? 0 : (rem == half ? 1 : 2));
    return w;
}
__host__ __device__ inline uint64_t walk_sat(uint64_t a) { return a > kWalkSat ? kWalkSat : a; }
// min(c d, kWalkSat) without overflow or an integer division: a product the
// double estimate puts at or above kWalkSat saturates (anything above 2^25
// only ever signals that the grid is left, so the exact cut does not matter).
__host__ __device__ inline uint64_t walk_mul(uint64_t c, uint64_t d) {
    return (double)c * (double)d >= (double)kWalkSat ? kWalkSat : c * d;
}

// c copies of one term as a map of m's parity p: increment inc[p], parity out.
struct WalkMap {
    uint64_t inc0, inc1;
    uint32_t par0, par1;
};
__host__ __device__ inline WalkMap walk_map(const WalkTerm &w, uint32_t c) {
    WalkMap r;
    if (c == 0) {
        r.inc0 = r.inc1 = 0;
        r.par0 = 0;
        r.par1 = 1;
        return r;
    }
    if (w.kind == 1) {  // ties to an even result: the first copy by parity, then the even step
        const uint64_t de = w.n + (w.n & 1u);
        const uint64_t rest = walk_mul(c - 1, de);
        r.inc0 = walk_sat(w.n + (w.n & 1u) + rest);         // p = 0: n + (n & 1)
        r.inc1 = walk_sat(w.n + ((w.n + 1u) & 1u) + rest);  // p = 1: n + ((1 + n) & 1)
        r.par0 = r.par1 = 0;
        return r;
    }
    const uint64_t d = w.n + (w.kind == 2 ? 1u : 0u);
    const uint64_t inc = walk_mul(c, d);
    const uint32_t flip = (uint32_t)(inc & 1u);
    r.inc0 = r.inc1 = inc;
    r.par0 = flip;
    r.par1 = 1u ^ flip;
    return r;
}
// a, then b
__host__ __device__ inline WalkMap walk_compose(const WalkMap &a, const WalkMap &b) {
    WalkMap r;
    r.inc0 = walk_sat(a.inc0 + (a.par0 ? b.inc1 : b.inc0));
    r.par0 = a.par0 ? b.par1 : b.par0;
    r.inc1 = walk_sat(a.inc1 + (a.par1 ? b.inc1 : b.inc0));
    r.par1 = a.par1 ? b.par1 : b.par0;
    return r;
}

enum WalkMode { kWalkSum = 0, kWalkReach = 1, kWalkDrop = 2 };

// Applies c copies of t to v in order (kWalkSum / kWalkReach: v = fl(v + t);
// kWalkDrop: v = fl(v - t)), a binade at a time.  Returns the 0-based copy
// after which kWalkReach first has v >= thr, or kWalkDrop first has v <= 0;
// -1 when no copy stops.
__host__ __device__ inline int64_t walk_group(float &v, float t, uint64_t c, int mode, float thr) {
    uint64_t done = 0;
    while (done < c) {
        if (mode == kWalkDrop && !(v > 0.0f)) return (int64_t)done;  // v - t <= 0 for any t >= 0
        if (mode != kWalkDrop && v == 0.0f) {                        // fl(0 + t) = t
            v = t;
            if (mode == kWalkReach && v >= thr) return (int64_t)done;
            ++done;
            continue;
        }
        const WalkGrid g = walk_grid(v);
        const WalkTerm w = walk_term(t, g.qe);
        uint64_t d, cq;  // grid step of one copy, ceil(t/q)
        if (w.kind == 1) {
            if (g.m & 1u) {  // odd m: this copy's step depends on it; take it in f32
                v = mode == kWalkDrop ? v - t : v + t;
                if ((mode == kWalkReach && v >= thr) || (mode == kWalkDrop && v <= 0.0f)) return (int64_t)done;
                ++done;
                continue;
            }
            d = w.n + (w.n & 1u);  // even m: every copy takes the even step and m stays even
            cq = w.n + 1u;
        } else {
            d = w.n + (w.kind == 2 ? 1u : 0u);
            cq = w.kind == 3 ? d : w.n + 1u;
        }
        if (d == 0) return -1;  // no copy changes v any more
        const uint64_t left = c - done;
        if (mode != kWalkDrop) {
            const uint64_t jmax = ((1ull << 24) - 1 - g.m) / d;  // copies that keep m + j d < 2^24
            if (mode == kWalkReach) {  // first j >= 1 with (m + j d) q >= thr, if inside the binade
                const double q = (double)walk_value(1, g.qe);
                const double need = ((double)thr / q - (double)g.m) / (double)d;
                if (need <= (double)jmax + 1.0) {
                    uint64_t j = need <= 1.0 ? 1 : (uint64_t)need;
                    while ((double)(g.m + j * d) * q < (double)thr) ++j;
                    if (j <= jmax && j <= left) {
                        v = walk_value(g.m + j * d, g.qe);
                        return (int64_t)(done + j - 1);
                    }
                }
            }
            const uint64_t j = left < jmax ? left : jmax;
            v = walk_value(g.m + j * d, g.qe);
            done += j;
            if (done < c) {  // the copy that leaves the binade, in f32
                v = v + t;
                if (mode == kWalkReach && v >= thr) return (int64_t)done;
                ++done;
            }
        } else {
            // copy i is exact on this grid while (m - i d) - ceil(t/q) >= low
            // (low = 2^23 above the lowest grid; 1 on it, so the result stays > 0)
            const uint64_t low = g.qe >= 2 ? (1ull << 23) : 1u;
            uint64_t js = 0;
            if (g.m >= cq + low) js = (g.m - cq - low) / d + 1;
            const uint64_t j = left < js ? left : js;
            v = walk_value(g.m - j * d, g.qe);
            done += j;
            if (done < c) {  // the copy that may leave the binade, in f32
                v = v - t;
                if (v <= 0.0f) return (int64_t)done;
                ++done;
            }
        }
    }
    return -1;
}

// Whether the running value, m + P (sum) or m - P (drop) on the grid qe after
// the prefix P of a scan, may have left the plain-integer regime (or reached
// thr): the groups up to the first such one are applied as integers.
__host__ __device__ inline bool walk_event(uint32_t m, int qe, uint64_t P, int mode, float thr) {
    if (mode == kWalkDrop) {
        const uint64_t low = qe >= 2 ? (1ull << 23) : 1u;
        return P + low + 1 > (uint64_t)m;  // m - P < low + 1
    }
    if ((uint64_t)m + P >= (1ull << 24)) return true;
    return mode == kWalkReach && (double)((uint64_t)m + P) * (double)walk_value(1, qe) >= (double)thr;
}

}  // namespace zi
