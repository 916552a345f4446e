// zi_tail.hpp -- the reference tail of Sampler.sampleWithMargin
// (src/sampler.zig:211-275) on a row's sorted candidates, shared by the
// sampling kernels: margin, untempered top-p and min-p, temperature weights,
// XTC and the draw, with every sum in the reference's sequential f32 order.
#pragma once
#include "zi_launch.hpp"
#include "zi_rowpass.hpp"

namespace zi {

struct TailLds {
    alignas(16) float e[kCapA];  // untempered exponentials of the sorted candidates (read 4 at a time)
    alignas(16) float w[kCapA];  // temperature weights
};
// Whole-vocabulary rows (k = V): the reference's top-p total runs over all V
// terms in sorted order (src/sampler.zig:217-218), but only the row's first n
// candidates are at hand.  The stream bounds that total: the chunks' sums of
// exp(x - max) give T within a relative 1e-4 (hardware exp2 with f32 partial
// sums, well inside that), and a sequential f32 sum of V nonnegative terms is
// within gamma_{V-1} = (V-1)u / (1 - (V-1)u) of the exact sum (u = 2^-24).  So
// the reference's threshold fl(top_p * total) lies in [fl(top_p * lo),
// fl(top_p * hi)] and its keep in [kp_lo, kp_hi].  keep is settled when
// min-p cuts before kp_lo, or when kp_lo == kp_hi within the prefix; then the
// rest of the tail only reads the prefix.  Lane 0 only; returns false when
// the row needs the exact whole-order pass.
// The row's total T = sum exp(x - mx) from the chunks' (max, sum) records.
__device__ __forceinline__ double chunk_stats_total(const SampleParams &P, int row, float mx) {
    const int G = P.src.G;
    const double *gs = P.g_stat + (int64_t)row * G * 3;
    double Mr = -INFINITY;
    for (int g = 0; g < G; ++g) Mr = fmax(Mr, ld_agent(&gs[g * 3]));
    double Z = 0.0;
    for (int g = 0; g < G; ++g) {
        const double m = ld_agent(&gs[g * 3]);
        if (m != -INFINITY) Z += ld_agent(&gs[g * 3 + 1]) * exp(m - Mr);
    }
    return Z * exp(Mr - (double)mx);
}

// tot: the row's total when the caller has it (>= 0), else taken from the
// chunk records.  complete: every entry past the prefix fails min-p (the
// prefix holds all entries above a threshold below mx + ln(min_p)), so the
// min-p cut is at n at the latest.
__device__ __forceinline__ bool nucleus_keep(const SampleParams &P, int row, const float *e, int n, int live,
                                             int first_low, float mx, int &keep, double tot, bool complete) {
    int kp_lo = n + 1, kp_hi = n + 1;  // n + 1: past the prefix
    if (P.top_p < 1.0f) {
        if (!__builtin_isfinite(mx)) return false;
        const double T = tot >= 0.0 ? tot : chunk_stats_total(P, row, mx);
        if (!(T >= 0.5 && T < 1e30)) return false;  // the term of the maximum alone is 1
        const double nu = (double)(P.n_all - 1) * 0x1p-24;
        const double gam = nu / (1.0 - nu) + 1e-4;
        const double dlo = T * (1.0 - gam), dhi = T * (1.0 + gam);
        float lo = (float)dlo, hi = (float)dhi;
        if ((double)lo > dlo) lo = __uint_as_float(__float_as_uint(lo) - 1u);  // round down (lo > 0)
        if ((double)hi < dhi) hi = __uint_as_float(__float_as_uint(hi) + 1u);  // round up
        kp_lo = first_reach(e, live, P.top_p * lo, n + 1);
        kp_hi = first_reach(e, live, P.top_p * hi, n + 1);
    }
    // The reference's keep is min(keep_p, first_low) (first_low >= 1: the
    // maximum's term is 1): min-p cuts at first_low unless keep_p comes first,
    // and when keep_p == first_low the two agree.
    const bool cut = first_low < n || (complete && first_low == n);
    if (cut && first_low <= kp_lo) {  // min-p decides keep (:229-234)
        keep = first_low > 1 ? first_low : 1;
        return true;
    }
    if (kp_lo == kp_hi && kp_lo <= n) {  // top-p keep pinned, min-p does not cut before it
        keep = kp_lo;
        return true;
    }
    return false;
}

// The reference tail (src/sampler.zig:211-275) on the row's n sorted
// candidates, one wave with all 64 lanes active.  The lanes compute the
// exponentials; the sequential sums (top-p, temperature total, draw) run on
// lane 0 from LDS, in the reference's order.  NUC: the n candidates are the
// prefix of a whole-vocabulary row (nucleus_keep); an unsettled row only sets
// its flag, and the candidate outputs cover the kept entries.
template <bool NUC>
__device__ __forceinline__ void sample_tail(const SampleParams &P, int row, const uint64_t *okey, const float *oval,
                                            int n, TailLds &tl, float u0, float u1, double tot = -1.0,
                                            bool complete = false) {
    const int lane = threadIdx.x;
    float cv[4];
    uint32_t cid[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        int i = lane + 64 * c;
        cv[c] = (i < n) ? oval[i] : 0.0f;
        cid[c] = (i < n) ? ckey_id(okey[i]) : 0u;
    }
    const float mx = oval[0];  // :212-213
    const float margin = (n >= 2) ? mx - oval[1] : 10.0f;

    // untempered exp(v - mx) for top-p / min-p (:215-234) and the temperature
    // weights (:236-242, used for i < keep only)
    const float inv_t = 1.0f / P.temp;
    const bool use_e = (P.top_p < 1.0f) || (P.min_p > 0.0f);
    float e[4], w[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int i = lane + 64 * c;
        const bool in = i < n;
        e[c] = 0.0f;
        w[c] = 0.0f;
        if (64 * c < n) {  // wave-uniform: skip the exponentials of empty slices
            e[c] = (use_e && in) ? exp32(cv[c] - mx) : 0.0f;
            w[c] = in ? exp32((cv[c] - mx) * inv_t) : 0.0f;
            if (in) {
                tl.e[i] = e[c];
                tl.w[i] = w[c];
            }
        }
    }
    // Every prefix sum is >= e_0 = 1, whose half ulp is 2^-24: a term below
    // that cannot change the sum, and the terms are non-increasing, so the
    // sequential sum ends at the first such term (exactly).  NaN terms (from
    // an infinite maximum) stay live: the reference's sums are then NaN and
    // nothing is cut.
    int live = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c)
        if (64 * c < n) live += __popcll(ballot(lane + 64 * c < n && !(e[c] < 0x1p-24f)));
    // min-p (:228-234): the first i with e_i < min_p (applied below within keep)
    int first_low = n;
    if (P.min_p > 0.0f) {
#pragma unroll
        for (int c = 3; c >= 0; --c) {
            if (64 * c < n) {
                const uint64_t m = ballot(lane + 64 * c < n && e[c] < P.min_p);
                if (m) first_low = 64 * c + __ffsll((unsigned long long)m) - 1;
            }
        }
    }
    wave_sync();  // tl.e / tl.w complete before lane 0 reads them
    int keep0 = n;
    float total0 = 0.0f;
    int settled0 = 1;
    if (lane == 0) {
        int keep = n;
        if constexpr (NUC) {
            settled0 = nucleus_keep(P, row, tl.e, n, live, first_low, mx, keep, tot, complete) ? 1 : 0;
        } else {
            if (P.top_p < 1.0f) {  // :215-226
                const float thr = P.top_p * lane_sum(tl.e, 0, live, 0.0f);
                keep = first_reach(tl.e, live, thr, n);
            }
            if (first_low < keep) keep = first_low > 1 ? first_low : 1;
        }
        keep0 = keep;
        if (settled0) total0 = lane_sum(tl.w, 0, keep, 0.0f);  // :236-242
    }
    if constexpr (NUC) {
        const int settled = __builtin_amdgcn_readlane(settled0, 0);
        if (lane == 0) P.nuc_flag[row] = settled ? 0 : 1;
        if (!settled) return;
    }
    const int keep = __builtin_amdgcn_readlane(keep0, 0);
    float total = readlane_f(total0, 0);
#pragma unroll
    for (int c = 0; c < 4; ++c) w[c] = (lane + 64 * c < keep) ? w[c] : 0.0f;

    // XTC (:244-268)
    int start = 0;
    int draws = 0;
    float umain = u0;
    if (P.xtc_p > 0.0f && P.xtc_thr <= 0.5f && keep >= 2 && total > 0.0f) {
        draws = 1;
        umain = u1;
        if (u0 <= P.xtc_p) {
            const float inv_tot = 1.0f / total;
            int f = keep;
#pragma unroll
            for (int c = 3; c >= 0; --c) {
                const uint64_t m = ballot(lane + 64 * c < keep && !(w[c] * inv_tot >= P.xtc_thr));
                if (m) f = 64 * c + __ffsll((unsigned long long)m) - 1;
            }
            const int pos_last = f > 0 ? f - 1 : 0;
            const int min_keep = max(1, P.xtc_min_keep);
            if (keep - pos_last >= min_keep && pos_last > 0) {
                start = pos_last;
                float t0 = 0.0f;
                if (lane == 0) t0 = lane_sum(tl.w, start, keep, 0.0f);
                total = readlane_f(t0, 0);
            }
        }
    }
    draws += 1;

    // draw: r = u * total; r -= w_i until r <= 0, else c[keep-1] (:270-275)
    if (lane == 0) {
        const int pick = first_drop(tl.w, start, keep, umain * total);
        P.tok[row] = ckey_id(okey[pick]);
        P.margin[row] = margin;
        if (P.ndraws) P.ndraws[row] = draws;
        if (P.keep) P.keep[row] = keep;
    }
    if (P.cand_ids) {
        const int n_out = NUC ? min(keep, P.cand_ld) : n;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            int i = lane + 64 * c;
            if (i < n_out) {
                int64_t o = (int64_t)row * P.cand_ld + i;
                P.cand_ids[o] = cid[c];
                if (P.cand_vals) P.cand_vals[o] = cv[c];
                if (P.probs) P.probs[o] = (i >= start && i < keep) ? w[c] / total : 0.0f;
            }
        }
    }
}

}  // namespace zi
