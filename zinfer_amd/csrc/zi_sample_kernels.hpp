// zi_sample_kernels.hpp -- batched Sampler.sampleWithMargin (src/sampler.zig:190-276)
// for top_k in [1, 256], and the first pass of whole-vocabulary rows (top_k =
// 0 or >= V, src/sampler.zig:197-201).
//
// One launch covers the batch: grid = rows x G workgroups.  Stage A (every
// workgroup) streams its chunk of the row from HBM once with 16-byte loads,
// applies mask + penalties + edits, and publishes the chunk's exact top-k
// sorted by (value desc, id asc).  The last workgroup of each row (ticket
// counter) runs stage B: merges the G sorted lists into the row's top-k and
// runs the reference tail on one wave: untempered top-p and min-p,
// temperature weights, XTC and the draw, with every sum in the reference's
// sequential f32 order.
#pragma once
#include <type_traits>

#include "zi_launch.hpp"
#include "zi_rowpass.hpp"
#include "zi_prefix.hpp"
#include "zi_tail.hpp"

namespace zi {

constexpr int kRowLoopRows = kRowLoopRowsHost;  // batches this large run one workgroup per row
constexpr int kLatePenMinGroups = 64;  // grids from a quarter of the CUs take the late-penalty select
constexpr int kLatePenMaxK = 64;  // largest top_k measured faster with the late select (k = 100 is slower)

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
    TailLds tl;
};

// Stage B, run by the last workgroup of the row: merges the G sorted chunk
// lists and runs the reference tail on wave 0.
__device__ __forceinline__ void sample_stage_b(const SampleParams &P, int row, int G, int k, SampleStageB &b,
                                               float u0, float u1) {
    const int n = row_merge(P.g_key, P.g_val, P.g_cnt, row, G, k, b.ml, b.okey, b.oval);
    if (threadIdx.x >= 64) return;  // the tail runs on wave 0 with all 64 lanes active
    if (n == 0) {                   // no selectable logit (every entry NaN): outside the reference contract
        if (threadIdx.x == 0) {
            P.tok[row] = 0u;
            P.margin[row] = 10.0f;
            if (P.ndraws) P.ndraws[row] = 0;
            if (P.keep) P.keep[row] = 0;
        }
        return;
    }
    sample_tail<false>(P, row, b.okey, b.oval, n, b.tl, u0, u1);
}

// LATE (with HAS_PEN, for penalties that never raise a logit): the stream
// runs without the penalty inputs and only the chunk's candidates are
// penalized (chunk_select_late); with CAP, only they are softcapped as well.
template <typename T, int NV, bool HAS_MASK, bool HAS_PEN, bool CAP, bool LATE>
__global__ __launch_bounds__(kThreads) void sample_kernel(SampleParams P) {
    __shared__ union {
        SampleStageA<T, NV, HAS_PEN> a;
        SampleStageB b;
    } sm;
    __shared__ uint32_t s_bins[256];
    __shared__ uint32_t s_tau[1];
    __shared__ int s_dig[2];
    __shared__ int s_n, s_flag, s_bad;

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
    ChunkRegs<T, NV> cr;
    // The candidate threshold is computed from the first kSplit vectors while
    // the last ones are still arriving.  Sixteen vectors: 14 (config 2, 16.99
    // -> 16.79 us against 12).  A softcap keeps 12: its candidates are capped
    // against a bound on the rest, and on sparsely masked rows (config 3) the
    // tighter threshold from 14 vectors leaves the k-th capped candidate under
    // that bound, so chunks are streamed again (18.3 -> 38.5 us).
    constexpr int kSplit = (NV == 16 && !CAP) ? 14 : NV * 3 / 4;
    float tau = 0.0f;
    const int64_t rg = (int64_t)row * G + g;
    ChunkOut out{P.g_key + rg * kCapA, P.g_val + rg * kCapA, P.g_cnt + rg};
    if constexpr (LATE) {
        static_assert(HAS_PEN, "late penalties need the penalty table");
        // Penalty inputs first, as vector loads (lane-varying addresses), so
        // that waiting for them after the stream waits for nothing else.
        PenRegs pr;
        pen_prefetch(a, row, pr);
        int rv = row;
        asm volatile("" : "+v"(rv));
        const int hl_raw = row_pen_window_on(a) ? a.hist_len[rv] : 0;
        const int ne_raw = a.edit_ids ? a.edit_count[rv] : 0;
        if (tid == 0) s_bad = 0;
        auto mid = [&](float lmax) {
            pen_clear_hash(*pen);  // ordered before the inserts by the barriers below
            tau = select_prepare<T, NV>(lmax, k, sm.a.sel, s_tau, &s_n);
        };
        // with a softcap, the stream stays raw and only the candidates are capped
        chunk_stream<T, NV, HAS_MASK, false, false, NoHook, kSplit>(a, row, c0, c1, cr, nullptr, nullptr, NoHook(),
                                                                     mid);
        int ur = 2 * row;
        asm volatile("" : "+v"(ur));
        const float u0 = P.uniforms[ur], u1 = P.uniforms[ur + 1];
        chunk_select_late<T, NV, CAP, HAS_MASK>(a, row, cr, c0, c1, k, sm.a.sel, pen, &pr, hl_raw, ne_raw, s_tau,
                                                &s_n, &s_bad, s_bins, s_dig, out, tau);
        if (!row_ticket(P.tickets, row, G, &s_flag)) return;
        sample_stage_b(P, row, G, k, sm.b, u0, u1);
        return;
    }
    if constexpr (CAP && !HAS_PEN) {
        // a softcap without penalties: the stream stays raw and only the
        // candidates are capped (chunk_select_late without a hash)
        auto mid = [&](float lmax) { tau = select_prepare<T, NV>(lmax, k, sm.a.sel, s_tau, &s_n); };
        chunk_stream<T, NV, HAS_MASK, false, false, NoHook, kSplit>(a, row, c0, c1, cr, nullptr, nullptr, NoHook(),
                                                                     mid);
        int ur = 2 * row;
        asm volatile("" : "+v"(ur));
        const float u0 = P.uniforms[ur], u1 = P.uniforms[ur + 1];
        chunk_select_late<T, NV, true, HAS_MASK, false>(a, row, cr, c0, c1, k, sm.a.sel, nullptr, nullptr, 0, 0,
                                                        s_tau, &s_n, nullptr, s_bins, s_dig, out, tau);
        if (!row_ticket(P.tickets, row, G, &s_flag)) return;
        sample_stage_b(P, row, G, k, sm.b, u0, u1);
        return;
    }
    PenOwn own;
    auto mid = [&](float lmax) { tau = select_prepare<T, NV>(lmax, k, sm.a.sel, s_tau, &s_n); };
    chunk_stream<T, NV, HAS_MASK, HAS_PEN, CAP, NoHook, kSplit>(a, row, c0, c1, cr, pen, &own, NoHook(), mid);
    // This row's two uniforms, requested now so that the tail never waits
    // for them: a vector load (lane-varying index), issued after the row's
    // loads, which a scalar load's early wait would otherwise hold back.
    int ur = 2 * row;
    asm volatile("" : "+v"(ur));
    const float u0 = P.uniforms[ur], u1 = P.uniforms[ur + 1];
    chunk_select_publish<T, NV, HAS_PEN, true>(a, cr, c0, k, sm.a.sel, pen, &own, s_tau, &s_n, s_bins, s_dig, out,
                                               tau);
    if (!row_ticket(P.tickets, row, G, &s_flag)) return;
    sample_stage_b(P, row, G, k, sm.b, u0, u1);
}

// Per-thread running (ref, S) with S = sum exp(x - ref) over the thread's
// elements, updated per vector as its load lands; ref moves up only when an
// element exceeds it by 64, so S cannot overflow.  -inf, NaN (diverted or
// past the chunk) contribute 0.
struct SumHook {
    float *ref, *S;
    template <int VEC>
    __device__ void operator()(int, const float (&v)[VEC], float m4) const {
        if (m4 > *ref + 64.0f) {  // also the first finite value (ref = -inf)
            if (*ref != -INFINITY) *S = *S * __builtin_amdgcn_exp2f((*ref - m4) * kLog2e);
            *ref = m4;
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) *S = *S + __builtin_amdgcn_exp2f(fmaxf(v[e] - *ref, -200.0f) * kLog2e);
    }
};

// First pass of whole-vocabulary rows: sample_kernel's stream and selection
// with a k-entry prefix (k = kMaxTopK), plus each chunk's (max, sum exp(x -
// max)) for the bound on the reference's total.  Rows whose keep the prefix
// settles are finished here; the others get nuc_flag = 1 for exact_kernel.
template <typename T, int NV, bool HAS_MASK, bool HAS_PEN, bool CAP>
__global__ __launch_bounds__(kThreads) void nucleus_kernel(SampleParams P) {
    __shared__ union {
        SampleStageA<T, NV, HAS_PEN> a;
        SampleStageB b;
    } sm;
    __shared__ uint32_t s_bins[256];
    __shared__ uint32_t s_tau[1];
    __shared__ int s_dig[2];
    __shared__ int s_n, s_flag;
    __shared__ float s_wmax[kWaves];
    __shared__ double s_ws[kWaves];

    const RowSource &a = P.src;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
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
    float ref = -INFINITY, S = 0.0f;
    chunk_stream<T, NV, HAS_MASK, HAS_PEN, CAP, SumHook>(a, row, c0, c1, cr, pen, &own, SumHook{&ref, &S});
    int ur = 2 * row;
    asm volatile("" : "+v"(ur));
    const float u0 = P.uniforms[ur], u1 = P.uniforms[ur + 1];
    const int64_t rg = (int64_t)row * G + g;
    ChunkOut out{P.g_key + rg * kCapA, P.g_val + rg * kCapA, P.g_cnt + rg};
    chunk_select_publish<T, NV, HAS_PEN>(a, cr, c0, k, sm.a.sel, pen, &own, s_tau, &s_n, s_bins, s_dig, out);
    if constexpr (HAS_PEN) {  // the penalized entries this thread owns (hash settled by the barriers above)
#pragma unroll
        for (int u = 0; u < kOwnSlots; ++u) {
            if (own.id[u] != 0xFFFFFFFFu) {
                const float v = owned_value(a, *pen, own, u);
                if (v > ref) {
                    S = S * __builtin_amdgcn_exp2f((ref - v) * kLog2e) + 1.0f;
                    ref = v;
                } else if (v > -INFINITY) {
                    S = S + __builtin_amdgcn_exp2f(fmaxf(v - ref, -200.0f) * kLog2e);
                }
            }
        }
    }
    const float wm = wave_max_f(ref);
    if (lane == 0) s_wmax[wid] = wm;
    __syncthreads();
    float M = s_wmax[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_wmax[w]);
    double ds = (ref != -INFINITY && M != -INFINITY) ? (double)S * exp((double)ref - (double)M) : 0.0;
    ds = wave_sum_d(ds);
    if (lane == 0) s_ws[wid] = ds;
    __syncthreads();
    if (tid == 0) {
        double ts = 0.0;
        for (int w = 0; w < kWaves; ++w) ts += s_ws[w];
        st_agent(&P.g_stat[rg * 3], (double)M);
        st_agent(&P.g_stat[rg * 3 + 1], ts);
    }
    if (!row_ticket(P.tickets, row, G, &s_flag)) return;

    const int n = row_merge(P.g_key, P.g_val, P.g_cnt, row, G, k, sm.b.ml, sm.b.okey, sm.b.oval);
    if (tid >= 64) return;
    if (n == 0) {  // no selectable logit: let the exact pass apply the reference literally
        if (tid == 0) P.nuc_flag[row] = 1;
        return;
    }
    sample_tail<true>(P, row, sm.b.okey, sm.b.oval, n, sm.b.tl, u0, u1);
}

// Large batches: one workgroup per row loops over the row's G chunks and
// keeps the running top-k sorted in LDS, so there is no cross-workgroup
// handoff.  Each chunk is streamed and selected as in sample_kernel, with the
// candidate threshold raised to the running k-th value once k entries are
// held (elements below it cannot enter), its sorted list published to LDS,
// and merged with the running list by rank (entries of the two lists are
// distinct: each holds the count of greater entries of the other list by a
// binary search).  NUC: the prefix pass of whole-vocabulary rows, with the
// row total accumulated over the chunks in each thread.

template <typename T, int NV, bool HAS_MASK, bool HAS_PEN, bool NUC, bool CAP>
__global__ __launch_bounds__(kThreads) void row_kernel(SampleParams P) {
    __shared__ union {
        SampleStageA<T, NV, HAS_PEN> a;
        TailLds tl;
    } sm;
    __shared__ RowLoopLds rl;
    __shared__ uint32_t s_bins[256];
    __shared__ uint32_t s_tau[1];
    __shared__ int s_dig[2];
    __shared__ int s_n;
    __shared__ float s_wmax[kWaves];
    __shared__ double s_ws[kWaves];

    const RowSource &a = P.src;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int G = a.G;
    const int row = blockIdx.x;
    const int k = P.k;
    int ur = 2 * row;
    asm volatile("" : "+v"(ur));
    const float u0 = P.uniforms[ur], u1 = P.uniforms[ur + 1];

    PenTable *pen = nullptr;
    if constexpr (HAS_PEN) pen = &sm.a.p.pen;
    float ref = -INFINITY, S = 0.0f;  // NUC: running sum exp(x - ref) of this thread's elements
    int n_run = 0, cur = 0;           // running list length and buffer (uniform)
    // The row in steps of what the registers hold (the plan's chunking only
    // sets the layout of the row-total record below).
    constexpr int SUB = kThreads * NV * VecTraits<T>::VEC;
    // bf16 rows of up to 32 elements per thread per step: each step's loads
    // are requested during the previous step (NV registers stay live through
    // the select; larger steps would spill).
    constexpr bool PF = std::is_same<T, uint16_t>::value && NV <= 4;
    uint4 pf[NV];
    if constexpr (PF) chunk_request<T, NV>(a, row, 0, min(a.V, SUB), pf);
    for (int c0 = 0; c0 < a.V; c0 += SUB) {
        const int c1 = min(a.V, c0 + SUB);
        PenOwn own;
        ChunkRegs<T, NV> cr;
        chunk_stream<T, NV, HAS_MASK, HAS_PEN, CAP, NoHook, NV, NoMid, PF>(a, row, c0, c1, cr, pen, &own, NoHook(),
                                                                          NoMid(), pf, c1, min(a.V, c1 + SUB));
        float tau;
        if (n_run == k) {  // uniform: nothing below the running k-th value can enter
            if (tid == 0) s_n = 0;
            if (tid < kSortMax) sm.a.sel.rank[tid] = 0u;
            __syncthreads();
            tau = -INFINITY;
        } else {
            tau = select_prepare<T, NV>(cr.lmax, k, sm.a.sel, s_tau, &s_n);
        }
        if (n_run == k) tau = fmaxf(tau, okey_inv((uint32_t)(rl.key[cur][k - 1] >> 32)));
        chunk_select_publish<T, NV, HAS_PEN, true>(a, cr, c0, k, sm.a.sel, pen, &own, s_tau, &s_n, s_bins, s_dig,
                                                   ChunkOut{rl.bk, rl.bv, &rl.bn}, tau);
        if constexpr (NUC) {  // this chunk's elements, penalized ones from their owners
            constexpr int VEC = VecTraits<T>::VEC;
            float m = cr.lmax;
            if constexpr (HAS_PEN) {
#pragma unroll
                for (int u = 0; u < kOwnSlots; ++u)
                    if (own.id[u] != 0xFFFFFFFFu) m = fmaxf(m, owned_value(a, *pen, own, u));
            }
            if (m > ref) {
                S = (ref == -INFINITY) ? 0.0f : S * __builtin_amdgcn_exp2f((ref - m) * kLog2e);
                ref = m;
            }
            if (ref != -INFINITY) {
#pragma unroll
                for (int i = 0; i < NV * VEC; ++i)
                    S = S + __builtin_amdgcn_exp2f(fmaxf(cr.x[i] - ref, -200.0f) * kLog2e);
                if constexpr (HAS_PEN) {
#pragma unroll
                    for (int u = 0; u < kOwnSlots; ++u)
                        if (own.id[u] != 0xFFFFFFFFu)
                            S = S + __builtin_amdgcn_exp2f(fmaxf(owned_value(a, *pen, own, u) - ref, -200.0f) * kLog2e);
                }
            }
        }
        __syncthreads();  // the chunk's list is in rl.bk / rl.bv / rl.bn
        running_merge(rl, cur, n_run, k);
    }

    double tot = -1.0;
    if constexpr (NUC) {  // the row total from every thread's (ref, S)
        const float wm = wave_max_f(ref);
        if (lane == 0) s_wmax[wid] = wm;
        __syncthreads();
        float M = s_wmax[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_wmax[w]);
        double ds = (ref != -INFINITY && M != -INFINITY) ? (double)S * exp((double)ref - (double)M) : 0.0;
        ds = wave_sum_d(ds);
        if (lane == 0) s_ws[wid] = ds;
        __syncthreads();
        double Z = 0.0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) Z += s_ws[w];
        tot = (n_run > 0) ? Z * exp((double)M - (double)rl.val[cur][0]) : 0.0;
        // the row total as the plan's per-chunk (max, sum) records, which the
        // whole-order pass reads for its bounds: all of it in record 0
        if (tid < G) {
            double *gs = P.g_stat + ((int64_t)row * G + tid) * 3;
            gs[0] = tid == 0 ? (double)M : -INFINITY;
            gs[1] = tid == 0 ? Z : 0.0;
            gs[2] = 0.0;
        }
    }
    if (tid >= 64) return;  // the tail runs on wave 0 with all 64 lanes active
    if (n_run == 0) {
        if (tid == 0) {
            if constexpr (NUC) {
                P.nuc_flag[row] = 1;
            } else {
                P.tok[row] = 0u;
                P.margin[row] = 10.0f;
                if (P.ndraws) P.ndraws[row] = 0;
                if (P.keep) P.keep[row] = 0;
            }
        }
        return;
    }
    sample_tail<NUC>(P, row, rl.key[cur], rl.val[cur], n_run, sm.tl, u0, u1, tot);
}

}  // namespace zi
