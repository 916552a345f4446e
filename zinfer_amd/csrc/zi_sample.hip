// zi_sample.hip -- batched Sampler.sampleWithMargin (src/sampler.zig:190-276)
// for top_k in [1, 256].
//
// One launch covers the batch: grid = rows x G workgroups.  Stage A (every
// workgroup) streams its chunk of the row from HBM once with 16-byte loads,
// applies mask + penalties + edits in registers and publishes a superset of
// the chunk's top-k.  The last workgroup of each row (ticket counter) runs
// stage B: gathers the row's candidates, radix-selects the exact top-k by
// (value desc, id asc), sorts them and runs the reference tail on one wave:
// untempered top-p and min-p, temperature weights, XTC and the draw, with
// every sum in the reference's sequential f32 order.
#include "zi_launch.hpp"
#include "zi_rowpass.hpp"

namespace zi {

struct SmemSampleA {
    PenTable pen;
    uint64_t ckey[kCapA];
    float cval[kCapA];
};
struct SmemSampleB {
    uint64_t bkey[kMaxG * kCapA];
    float bval[kMaxG * kCapA];
    uint64_t tkey[kThreads];
    float tval[kThreads];
    uint64_t okey[kThreads];
    float oval[kThreads];
};
union SmemSample {
    SmemSampleA a;
    SmemSampleB b;
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

template <typename T, int NV>
__global__ __launch_bounds__(kThreads) void sample_kernel(SampleParams P) {
    __shared__ SmemSample sm;
    __shared__ uint32_t s_bins[256];
    __shared__ uint32_t s_tau[kWaves];
    __shared__ int s_dig[2];
    __shared__ int s_nc, s_flag, s_cnt;
    __shared__ int s_off[kMaxG + 1];

    const RowSource &a = P.src;
    const int tid = threadIdx.x;
    const int G = a.G;
    const int row = blockIdx.x / G;
    const int g = blockIdx.x - row * G;
    const int c0 = g * a.CH;
    const int c1 = min(a.V, c0 + a.CH);

    RowPen rp = row_pen(a, row);
    PenRegs pr;
    if (rp.any) pen_fetch(rp, pr);
    uint4 raw[NV];
    uint32_t mw[NV];
    chunk_load<T, NV>(a, row, c0, c1, raw, mw);
    if (rp.any) pen_build(sm.a.pen, rp, pr, c0, c1);
    ChunkRegs<T, NV> cr;
    float tmax = chunk_transform<T, NV>(a, sm.a.pen, rp, c0, c1, raw, mw, cr);

    const int k = P.k;
    int nc = chunk_candidates<T, NV>(cr, tmax, c0, c1, k, sm.a.ckey, sm.a.cval, kCapA, &s_nc, s_tau);
    if (nc > kCapA) nc = chunk_candidates_exact<T, NV>(cr, c0, c1, k, sm.a.ckey, sm.a.cval, &s_nc, s_bins, s_dig);
    if (!publish_and_ticket(sm.a.ckey, sm.a.cval, nc, P.g_key, P.g_val, P.g_cnt, P.tickets, row, g, G, &s_flag))
        return;

    // ---------------- stage B: the last workgroup of this row ----------------
    int N = gather_candidates(P.g_key, P.g_val, P.g_cnt, row, G, sm.b.bkey, sm.b.bval, s_off);
    const int n = min(k, N);
    if (n == 0) {  // no selectable logit (every entry NaN): outside the reference contract
        if (tid == 0) {
            P.tok[row] = 0u;
            P.margin[row] = 10.0f;
            if (P.ndraws) P.ndraws[row] = 0;
            if (P.keep) P.keep[row] = 0;
        }
        return;
    }
    select_sorted(sm.b.bkey, sm.b.bval, N, n, sm.b.okey, sm.b.oval, sm.b.tkey, sm.b.tval, s_bins, s_dig, &s_cnt);
    if (tid >= 64) return;  // the tail runs on wave 0 with all 64 lanes active

    const int lane = tid;
    float cv[4];
    uint32_t cid[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        int i = lane + 64 * c;
        cv[c] = (i < n) ? sm.b.oval[i] : 0.0f;
        cid[c] = (i < n) ? ckey_id(sm.b.okey[i]) : 0u;
    }
    const float mx = sm.b.oval[0];  // sampler.zig:212-213
    const float margin = (n >= 2) ? mx - sm.b.oval[1] : 10.0f;
    int keep = n;

    // top-p then min-p on untempered exp(v - mx) (sampler.zig:215-234)
    float e[4];
    const bool use_e = (P.top_p < 1.0f) || (P.min_p > 0.0f);
#pragma unroll
    for (int c = 0; c < 4; ++c) e[c] = (use_e && lane + 64 * c < n) ? exp32(cv[c] - mx) : 0.0f;
    if (P.top_p < 1.0f) {
        float pc[4];
        float carry = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            pc[c] = 0.0f;
            if (64 * c < n) {
                int steps = min(64, n - 64 * c);
                pc[c] = wave_serial_chain<false>(e[c], carry, steps);
                carry = readlane_f(pc[c], steps - 1);
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

    // temperature on the survivors (sampler.zig:236-242)
    const float inv_t = 1.0f / P.temp;
    float w[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) w[c] = (lane + 64 * c < keep) ? exp32((cv[c] - mx) * inv_t) : 0.0f;
    float total = chain_sum(w, keep);

    // XTC (sampler.zig:244-268)
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

    // draw: r = u * total; r -= w_i until r <= 0 (sampler.zig:270-275)
    uint32_t last_col = cid[0];
    const int lq = (keep - 1) >> 6;
    if (lq == 1) last_col = cid[1];
    if (lq == 2) last_col = cid[2];
    if (lq == 3) last_col = cid[3];
    uint32_t tok = __builtin_amdgcn_readlane(last_col, (keep - 1) & 63);  // fallback c[keep-1] (:275)
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
                    int l = __ffsll((unsigned long long)m) - 1;
                    tok = __builtin_amdgcn_readlane(cid[c], l);
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

template <typename T, int NV>
static hipError_t launch_sample_t(const SampleParams &P, int rows, hipStream_t st) {
    dim3 grid(rows * P.src.G), block(kThreads);
    hipLaunchKernelGGL((sample_kernel<T, NV>), grid, block, 0, st, P);
    return hipGetLastError();
}

hipError_t launch_sample(const SampleParams &P, int dtype, int nv, int rows, hipStream_t st) {
    if (dtype == 0) {
        switch (nv) {
            case 4: return launch_sample_t<float, 4>(P, rows, st);
            case 8: return launch_sample_t<float, 8>(P, rows, st);
            default: return launch_sample_t<float, 16>(P, rows, st);
        }
    }
    switch (nv) {
        case 2: return launch_sample_t<uint16_t, 2>(P, rows, st);
        case 4: return launch_sample_t<uint16_t, 4>(P, rows, st);
        default: return launch_sample_t<uint16_t, 8>(P, rows, st);
    }
}

}  // namespace zi
