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
struct SampleStageB {
    MergeLds ml;
    uint64_t okey[kThreads];
    float oval[kThreads];
};

// Sequential f32 sum of x_i over lanes/chunks for i in [0, end) (x must be 0
// outside the range so that leading entries are exact identities).
__device__ __forceinline__ float chain_sum(const float (&x)[4], int end) {
    float carry = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        if (64 * c < end) {
            int steps = min(64, end - 64 * c);
            float p = wave_serial_chain<false>(x[c], carry, steps);
            carry = readlane_f(p, steps - 1);
        }
    }
    return carry;
}

// The reference tail (src/sampler.zig:211-275) on the row's n sorted
// candidates, one wave with all 64 lanes active.
__device__ __forceinline__ void sample_tail(const SampleParams &P, int row, const uint64_t *okey, const float *oval,
                                            int n) {
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
    int keep = n;

    // top-p then min-p on untempered exp(v - mx) (:215-234).  The
    // temperature weights are computed alongside (used for i < keep only).
    const float inv_t = 1.0f / P.temp;
    float e[4], w[4];
    const bool use_e = (P.top_p < 1.0f) || (P.min_p > 0.0f);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const bool in = lane + 64 * c < n;
        e[c] = (use_e && in) ? exp32(cv[c] - mx) : 0.0f;
        w[c] = in ? exp32((cv[c] - mx) * inv_t) : 0.0f;
    }
    if (P.top_p < 1.0f) {
        // Every prefix sum is >= e_0 = 1, whose half ulp is 2^-24: a term below
        // that cannot change the sum, and the terms are non-increasing, so the
        // sequential sum ends at the first such term (exactly).
        // (NaN terms, from an infinite maximum, stay live: the reference's sums
        // are then NaN and nothing is cut.)
        const int live = __popcll(ballot(lane < n && !(e[0] < 0x1p-24f))) +
                         __popcll(ballot(lane + 64 < n && !(e[1] < 0x1p-24f))) +
                         __popcll(ballot(lane + 128 < n && !(e[2] < 0x1p-24f))) +
                         __popcll(ballot(lane + 192 < n && !(e[3] < 0x1p-24f)));
        float pc[4];
        float carry = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            pc[c] = carry;
            if (64 * c < live) {
                int steps = min(64, live - 64 * c);
                float p = wave_serial_chain<false>(e[c], carry, steps);
                pc[c] = (lane < steps) ? p : readlane_f(p, steps - 1);
                carry = readlane_f(p, steps - 1);
            }
        }
        const float thr = P.top_p * carry;  // carry == total
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            uint64_t m = ballot(lane + 64 * c < n && pc[c] >= thr);
            if (m) {
                keep = 64 * c + __ffsll((unsigned long long)m);
                break;
            }
        }
    }
    if (P.min_p > 0.0f) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            uint64_t m = ballot(lane + 64 * c < keep && e[c] < P.min_p);
            if (m) {
                int i = 64 * c + __ffsll((unsigned long long)m) - 1;
                keep = i > 1 ? i : 1;
                break;
            }
        }
    }

    // temperature on the survivors (:236-242)
#pragma unroll
    for (int c = 0; c < 4; ++c) w[c] = (lane + 64 * c < keep) ? w[c] : 0.0f;
    float total = chain_sum(w, keep);

    // XTC (:244-268)
    int start = 0;
    int draws = 0;
    const float u0 = P.uniforms[2 * row];
    const float u1 = P.uniforms[2 * row + 1];
    float umain = u0;
    if (P.xtc_p > 0.0f && P.xtc_thr <= 0.5f && keep >= 2 && total > 0.0f) {
        draws = 1;
        umain = u1;
        if (u0 <= P.xtc_p) {
            const float inv_tot = 1.0f / total;
            int f = keep;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                uint64_t m = ballot(lane + 64 * c < keep && !(w[c] * inv_tot >= P.xtc_thr));
                if (m) {
                    f = 64 * c + __ffsll((unsigned long long)m) - 1;
                    break;
                }
            }
            const int pos_last = f > 0 ? f - 1 : 0;
            const int min_keep = max(1, P.xtc_min_keep);
            if (keep - pos_last >= min_keep && pos_last > 0) {
                start = pos_last;
                float ws[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) ws[c] = (lane + 64 * c >= start) ? w[c] : 0.0f;
                total = chain_sum(ws, keep);
            }
        }
    }
    draws += 1;

    // draw: r = u * total; r -= w_i until r <= 0 (:270-275)
    uint32_t tok = ckey_id(okey[keep - 1]);  // fallback c[keep-1] (:275)
    {
        float carry = umain * total;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if (64 * c < keep) {
                int i = lane + 64 * c;
                int steps = min(64, keep - 64 * c);
                float x = (i >= start && i < keep) ? w[c] : 0.0f;
                float d = wave_serial_chain<true>(x, carry, steps);
                uint64_t m = ballot(i >= start && i < keep && d <= 0.0f);
                if (m) {
                    tok = ckey_id(okey[64 * c + __ffsll((unsigned long long)m) - 1]);
                    break;
                }
                carry = readlane_f(d, steps - 1);
            }
        }
    }

    if (lane == 0) {
        P.tok[row] = tok;
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
    sample_tail(P, row, sm.b.okey, sm.b.oval, n);
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
