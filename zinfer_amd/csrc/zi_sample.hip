// zi_sample.hip -- batched Sampler.sampleWithMargin (src/sampler.zig:190-276)
// for top_k in [1, 256].
//
// One launch covers the batch: grid = rows x G workgroups.  Stage A (every
// workgroup) streams its chunk of the row from HBM once with 16-byte loads,
// applies mask + penalties + edits, and publishes the chunk's exact top-k
// sorted by (value desc, id asc).  The last workgroup of each row (ticket
// counter) runs stage B: merges the G sorted lists into the row's top-k and
// runs the reference tail on one wave: untempered top-p and min-p,
// temperature weights, XTC and the draw, with every sum in the reference's
// sequential f32 order.
#include "zi_launch.hpp"
#include "zi_rowpass.hpp"

namespace zi {

template <bool P>
struct PenLds {
    PenTable pen;
};
template <>
struct PenLds<false> {};

template <typename T, int NV, bool HAS_PEN>
struct SampleStageA {
    PenLds<HAS_PEN> p;
    SelectLds<T, NV> sel;
};
struct TailLds {
    alignas(16) float e[kCapA];  // untempered exponentials of the sorted candidates (read 4 at a time)
    alignas(16) float w[kCapA];  // temperature weights
};
struct SampleStageB {
    MergeLds ml;
    uint64_t okey[kThreads];
    float oval[kThreads];
    TailLds tl;
};

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

// The reference tail (src/sampler.zig:211-275) on the row's n sorted
// candidates, one wave with all 64 lanes active.  The lanes compute the
// exponentials; the sequential sums (top-p, temperature total, draw) run on
// lane 0 from LDS, in the reference's order.
__device__ __forceinline__ void sample_tail(const SampleParams &P, int row, const uint64_t *okey, const float *oval,
                                            int n, TailLds &tl, float u0, float u1) {
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
    if (lane == 0) {
        int keep = n;
        if (P.top_p < 1.0f) {  // :215-226
            const float thr = P.top_p * lane_sum(tl.e, 0, live, 0.0f);
            keep = first_reach(tl.e, live, thr, n);
        }
        if (first_low < keep) keep = first_low > 1 ? first_low : 1;
        keep0 = keep;
        total0 = lane_sum(tl.w, 0, keep, 0.0f);  // :236-242
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
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            int i = lane + 64 * c;
            if (i < n) {
                int64_t o = (int64_t)row * P.cand_ld + i;
                P.cand_ids[o] = cid[c];
                if (P.cand_vals) P.cand_vals[o] = cv[c];
                if (P.probs) P.probs[o] = (i >= start && i < keep) ? w[c] / total : 0.0f;
            }
        }
    }
}

template <typename T, int NV, bool HAS_MASK, bool HAS_PEN>
__global__ __launch_bounds__(kThreads) void sample_kernel(SampleParams P) {
    __shared__ union {
        SampleStageA<T, NV, HAS_PEN> a;
        SampleStageB b;
    } sm;
    __shared__ uint32_t s_bins[256];
    __shared__ uint32_t s_tau[1];
    __shared__ int s_dig[2];
    __shared__ int s_n, s_flag;

    const RowSource &a = P.src;
    const int tid = threadIdx.x;
    const int G = a.G;
    const int row = blockIdx.x / G;
    const int g = blockIdx.x - row * G;
    const int c0 = g * a.CH;
    const int c1 = min(a.V, c0 + a.CH);
    const int k = P.k;

    PenTable *pen = nullptr;
    if constexpr (HAS_PEN) pen = &sm.a.p.pen;
    PenOwn own;
    ChunkRegs<T, NV> cr;
    chunk_stream<T, NV, HAS_MASK, HAS_PEN>(a, row, c0, c1, cr, pen, &own);
    // This row's two uniforms, requested now so that the tail never waits
    // for them: a vector load (lane-varying index), issued after the row's
    // loads, which a scalar load's early wait would otherwise hold back.
    int ur = 2 * row;
    asm volatile("" : "+v"(ur));
    const float u0 = P.uniforms[ur], u1 = P.uniforms[ur + 1];
    const int64_t rg = (int64_t)row * G + g;
    ChunkOut out{P.g_key + rg * kCapA, P.g_val + rg * kCapA, P.g_cnt + rg};
    chunk_select_publish<T, NV, HAS_PEN>(a, cr, c0, k, sm.a.sel, pen, &own, s_tau, &s_n, s_bins, s_dig, out);
    if (!row_ticket(P.tickets, row, G, &s_flag)) return;

    // ---------------- stage B: the last workgroup of this row ----------------
    const int n = row_merge(P.g_key, P.g_val, P.g_cnt, row, G, k, sm.b.ml, sm.b.okey, sm.b.oval);
    if (tid >= 64) return;  // the tail runs on wave 0 with all 64 lanes active
    if (n == 0) {           // no selectable logit (every entry NaN): outside the reference contract
        if (tid == 0) {
            P.tok[row] = 0u;
            P.margin[row] = 10.0f;
            if (P.ndraws) P.ndraws[row] = 0;
            if (P.keep) P.keep[row] = 0;
        }
        return;
    }
    sample_tail(P, row, sm.b.okey, sm.b.oval, n, sm.b.tl, u0, u1);
}

template <typename T, int NV, bool M, bool PN>
static hipError_t launch_sample_t(const SampleParams &P, int rows, hipStream_t st) {
    dim3 grid(rows * P.src.G), block(kThreads);
    hipLaunchKernelGGL((sample_kernel<T, NV, M, PN>), grid, block, 0, st, P);
    return hipGetLastError();
}

template <typename T, int NV>
static hipError_t launch_sample_nv(const SampleParams &P, int rows, hipStream_t st) {
    const bool m = P.src.mask != nullptr;
    const bool p = (P.src.hist != nullptr) || (P.src.edit_ids != nullptr);
    if (m && p) return launch_sample_t<T, NV, true, true>(P, rows, st);
    if (m) return launch_sample_t<T, NV, true, false>(P, rows, st);
    if (p) return launch_sample_t<T, NV, false, true>(P, rows, st);
    return launch_sample_t<T, NV, false, false>(P, rows, st);
}

hipError_t launch_sample(const SampleParams &P, int dtype, int nv, int rows, hipStream_t st) {
    if (dtype == 0) {
        switch (nv) {
            case 4: return launch_sample_nv<float, 4>(P, rows, st);
            case 8: return launch_sample_nv<float, 8>(P, rows, st);
            default: return launch_sample_nv<float, 16>(P, rows, st);
        }
    }
    switch (nv) {
        case 2: return launch_sample_nv<uint16_t, 2>(P, rows, st);
        case 4: return launch_sample_nv<uint16_t, 4>(P, rows, st);
        default: return launch_sample_nv<uint16_t, 8>(P, rows, st);
    }
}

}  // namespace zi
