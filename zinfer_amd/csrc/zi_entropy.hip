// zi_entropy.hip -- per-row statistics for speculative verification: Shannon
// entropy (nats) of the T = 1 full-vocabulary softmax, the top-k ids (value
// desc, id asc) with full-vocabulary probabilities, the lowest-index argmax
// and argmax == draft acceptance (the compare of src/gen.zig:559).
//
// The reference has no entropy: Gen.AdaptiveDraft (src/gen.zig:366-432) is
// driven by the logit margin.  Definition used here:
//   M = max x, Z = sum exp(x - M), A = sum exp(x - M) (x - M),
//   H = ln Z - A / Z,  p_i = exp(x_i - M) / Z.
// Each thread keeps (ref, S, U) with S = sum exp(x - ref), U = sum exp(x -
// ref)(x - ref) over its elements; ref is the thread's running maximum, so
// every term is at most 1 and no small term is added to a sum dominated by a
// far larger one (a dominant logit after small ones would otherwise round the
// later terms away).  Workgroup and row merges are in f64.
#include "zi_launch.hpp"
#include "zi_rowpass.hpp"

namespace zi {

template <typename T, int NV>
struct EntStageA {
    SelectLds<T, NV> sel;
};
struct EntStageB {
    MergeLds ml;
    uint64_t okey[kThreads];
    float oval[kThreads];
};

// Per-thread running (ref, S, U), updated per vector as its load lands.
struct EntHook {
    float *ref, *S, *U;
    template <int VEC>
    __device__ void operator()(int, const float (&v)[VEC], float m4) const {
        if (m4 > *ref) {  // also the first finite value (ref = -inf)
            if (*ref != -INFINITY) {
                float dl = *ref - m4;
                float sc = __builtin_amdgcn_exp2f(dl * kLog2e);
                *U = (*U + dl * *S) * sc;
                *S = *S * sc;
            }
            *ref = m4;
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            float d = fmaxf(v[e] - *ref, -200.0f);  // -inf and NaN contribute 0
            float ex = __builtin_amdgcn_exp2f(d * kLog2e);
            *S = *S + ex;
            *U = fmaf(ex, d, *U);
        }
    }
};

struct EntLds {
    float wmax[kWaves];
    double ws[kWaves], wu[kWaves];
    double M, Z;
};

// Workgroup merge of every thread's (ref, S, U) in f64 into sl.wmax / ws / wu
// (per wave); contains a barrier, and the per-wave sums are read after the
// caller's next barrier.
__device__ __forceinline__ void ent_stats_reduce(float ref, float S, float U, EntLds &sl) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    float wm = wave_max_f(ref);
    if (lane == 0) sl.wmax[wid] = wm;
    __syncthreads();
    float M = sl.wmax[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, sl.wmax[w]);
    double ds = 0.0, du = 0.0;
    if (ref != -INFINITY && M != -INFINITY) {
        double sh = (double)ref - (double)M;
        double sc = exp(sh);
        ds = (double)S * sc;
        du = ((double)U + sh * (double)S) * sc;
    }
    ds = wave_sum_d(ds);
    du = wave_sum_d(du);
    if (lane == 0) {
        sl.ws[wid] = ds;
        sl.wu[wid] = du;
    }
}

// Thread 0 stores the workgroup's (max, S, U) record for chunk rg (after a
// barrier that follows ent_stats_reduce).
__device__ __forceinline__ void ent_stats_publish(const EntropyParams &P, int64_t rg, const EntLds &sl) {
    if (threadIdx.x != 0) return;
    float M = sl.wmax[0];
    double ts = 0.0, tu = 0.0;
    for (int w = 0; w < kWaves; ++w) {
        M = fmaxf(M, sl.wmax[w]);
        ts += sl.ws[w];
        tu += sl.wu[w];
    }
    st_agent(&P.g_stat[rg * 3], (double)M);
    st_agent(&P.g_stat[rg * 3 + 1], ts);
    st_agent(&P.g_stat[rg * 3 + 2], tu);
}

__device__ __forceinline__ void entropy_stage_b(const EntropyParams &P, int row, int G, int k, EntStageB &b,
                                                EntLds &sl);

template <typename T, int NV>
__global__ __launch_bounds__(kThreads) void entropy_kernel(EntropyParams P) {
    __shared__ union {
        EntStageA<T, NV> a;
        EntStageB b;
    } sm;
    __shared__ uint32_t s_bins[256];
    __shared__ uint32_t s_tau[1];
    __shared__ int s_dig[2];
    __shared__ int s_n, s_flag;
    __shared__ EntLds sl;

    const RowSource &a = P.src;
    const int G = a.G;
    const int row = blockIdx.x / G;
    const int g = blockIdx.x - row * G;
    const int c0 = g * a.CH;
    const int c1 = min(a.V, c0 + a.CH);
    const int k = P.k;

    ChunkRegs<T, NV> cr;
    float ref = -INFINITY, S = 0.0f, U = 0.0f;
    chunk_stream<T, NV, false, false, false, EntHook>(a, row, c0, c1, cr, nullptr, nullptr,
                                                      EntHook{&ref, &S, &U});

    const int64_t rg = (int64_t)row * G + g;
    ent_stats_reduce(ref, S, U, sl);
    ChunkOut out{P.g_key + rg * kCapA, P.g_val + rg * kCapA, P.g_cnt + rg};
    chunk_select_publish<T, NV, false>(a, cr, c0, k, sm.a.sel, nullptr, nullptr, s_tau, &s_n, s_bins, s_dig, out);
    ent_stats_publish(P, rg, sl);
    if (!row_ticket(P.tickets, row, G, &s_flag)) return;
    entropy_stage_b(P, row, G, k, sm.b, sl);
}

// The last workgroup of the row: merges the G sorted lists, the G (max, S, U)
// records into the entropy, and writes the top-k with full-vocabulary
// probabilities, the argmax and the draft acceptance.
__device__ __forceinline__ void entropy_stage_b(const EntropyParams &P, int row, int G, int k, EntStageB &b,
                                                EntLds &sl) {
    const int tid = threadIdx.x;
    const int n = row_merge(P.g_key, P.g_val, P.g_cnt, row, G, k, b.ml, b.okey, b.oval);
    double &s_M = sl.M, &s_Z = sl.Z;
    if (tid == 0) {
        const double *gs = P.g_stat + (int64_t)row * G * 3;
        double Mr = -INFINITY;
        for (int gg = 0; gg < G; ++gg) Mr = fmax(Mr, ld_agent(&gs[gg * 3]));
        double Z = 0.0, A = 0.0;
        if (Mr != -INFINITY) {
            for (int gg = 0; gg < G; ++gg) {
                const double m = ld_agent(&gs[gg * 3]), sg = ld_agent(&gs[gg * 3 + 1]), ug = ld_agent(&gs[gg * 3 + 2]);
                if (m == -INFINITY) continue;
                double sh = m - Mr;
                double sc = exp(sh);
                Z += sg * sc;
                A += (ug + sh * sg) * sc;
            }
        }
        s_M = Mr;
        s_Z = Z;
        if (P.entropy) P.entropy[row] = (float)(log(Z) - A / Z);
        uint32_t am = n > 0 ? ckey_id(b.okey[0]) : 0u;
        if (P.argmax) P.argmax[row] = am;
        if (P.accept && P.draft) P.accept[row] = (uint8_t)(am == P.draft[row]);
    }
    __syncthreads();
    if (tid < n) {
        int64_t o = (int64_t)row * P.out_ld + tid;
        if (P.ids) P.ids[o] = ckey_id(b.okey[tid]);
        if (P.probs) P.probs[o] = (float)(exp((double)b.oval[tid] - s_M) / s_Z);
    }
}

// Batches whose chunked grid would take more than one round of workgroups
// (config 4: 64 rows x 8 chunks at one workgroup per CU): G segments per row,
// each walked by one workgroup in steps of what its registers hold.  The next
// step's loads are requested while this step is selected, the workgroup's
// top-k so far is kept sorted in LDS, and once it holds k entries its k-th
// value is the step's threshold (no threshold sort).  The segment's list and
// (max, S, U) record then take the chunked kernel's handoff and stage B.
template <typename T, int NV>
__global__ __launch_bounds__(kThreads) void entropy_walk_kernel(EntropyParams P) {
    __shared__ union {
        EntStageA<T, NV> a;
        EntStageB b;
    } sm;
    __shared__ RowLoopLds rl;
    __shared__ uint32_t s_bins[256];
    __shared__ uint32_t s_tau[1];
    __shared__ int s_dig[2];
    __shared__ int s_n, s_flag;
    __shared__ EntLds sl;

    constexpr int VEC = VecTraits<T>::VEC;
    constexpr int SUB = kThreads * NV * VEC;
    const RowSource &a = P.src;
    const int tid = threadIdx.x;
    const int G = a.G;
    const int row = blockIdx.x / G;
    const int g = blockIdx.x - row * G;
    const int s0 = g * a.CH;
    const int s1 = min(a.V, s0 + a.CH);
    const int k = P.k;

    float ref = -INFINITY, S = 0.0f, U = 0.0f;
    int n_run = 0, cur = 0;
    uint4 pf[NV];
    chunk_request<T, NV>(a, row, s0, min(s1, s0 + SUB), pf);
    for (int c0 = s0; c0 < s1; c0 += SUB) {
        const int c1 = min(s1, c0 + SUB);
        ChunkRegs<T, NV> cr;
        chunk_stream<T, NV, false, false, false, EntHook, NV, NoMid, true>(
            a, row, c0, c1, cr, nullptr, nullptr, EntHook{&ref, &S, &U}, NoMid(), pf, c1, min(s1, c1 + SUB));
        float tau;
        if (n_run == k) {  // uniform: nothing below the running k-th value can enter
            if (tid == 0) s_n = 0;
            if (tid < kSortMax) sm.a.sel.rank[tid] = 0u;
            __syncthreads();
            tau = okey_inv((uint32_t)(rl.key[cur][k - 1] >> 32));
        } else {
            tau = select_prepare<T, NV>(cr.lmax, k, sm.a.sel, s_tau, &s_n);
        }
        chunk_select_publish<T, NV, false, true>(a, cr, c0, k, sm.a.sel, nullptr, nullptr, s_tau, &s_n, s_bins,
                                                 s_dig, ChunkOut{rl.bk, rl.bv, &rl.bn}, tau);
        __syncthreads();  // the step's list is in rl.bk / rl.bv / rl.bn
        running_merge(rl, cur, n_run, k);
    }
    const int64_t rg = (int64_t)row * G + g;
    ent_stats_reduce(ref, S, U, sl);
    if (tid < k) {  // the segment's list, zero-padded to k like a chunk's
        st_agent(&P.g_key[rg * kCapA + tid], tid < n_run ? rl.key[cur][tid] : (uint64_t)0);
        if (tid < n_run) st_agent(&P.g_val[rg * kCapA + tid], rl.val[cur][tid]);
    }
    if (tid == 0) st_agent(P.g_cnt + rg, n_run);
    __syncthreads();  // per-wave sums of the record
    ent_stats_publish(P, rg, sl);
    if (!row_ticket(P.tickets, row, G, &s_flag)) return;
    entropy_stage_b(P, row, G, k, sm.b, sl);
}

hipError_t launch_entropy_walk(const EntropyParams &P, int dtype, int rows, hipStream_t st) {
    dim3 grid(rows * P.src.G), block(kThreads);
    if (dtype == 0) hipLaunchKernelGGL((entropy_walk_kernel<float, 8>), grid, block, 0, st, P);
    else hipLaunchKernelGGL((entropy_walk_kernel<uint16_t, 4>), grid, block, 0, st, P);
    return hipGetLastError();
}

template <typename T, int NV>
static hipError_t launch_entropy_t(const EntropyParams &P, int rows, hipStream_t st) {
    dim3 grid(rows * P.src.G), block(kThreads);
    hipLaunchKernelGGL((entropy_kernel<T, NV>), grid, block, 0, st, P);
    return hipGetLastError();
}

hipError_t launch_entropy(const EntropyParams &P, int dtype, int nv, int rows, hipStream_t st) {
    if (dtype == 0) {
        switch (nv) {
            case 4: return launch_entropy_t<float, 4>(P, rows, st);
            case 8: return launch_entropy_t<float, 8>(P, rows, st);
            default: return launch_entropy_t<float, 16>(P, rows, st);
        }
    }
    switch (nv) {
        case 2: return launch_entropy_t<uint16_t, 2>(P, rows, st);
        case 4: return launch_entropy_t<uint16_t, 4>(P, rows, st);
        default: return launch_entropy_t<uint16_t, 8>(P, rows, st);
    }
}

// ---------------------------------------------------------------- mask
// JsonValidator.applyMask (src/grammar.zig:446-479) for a packed mask: clear
// bit -> -inf, in place.  Vectors whose mask bits are all set are not touched.
template <typename T>
__global__ __launch_bounds__(kThreads) void mask_kernel(MaskParams P) {
    constexpr int VEC = VecTraits<T>::VEC;
    const int64_t nvr = (P.V + VEC - 1) / VEC;
    const int64_t total = nvr * P.rows;
    for (int64_t q = (int64_t)blockIdx.x * kThreads + threadIdx.x; q < total; q += (int64_t)gridDim.x * kThreads) {
        int row = (int)(q / nvr);
        int e0 = (int)(q - (int64_t)row * nvr) * VEC;
        uint32_t w = P.mask[(int64_t)row * P.mask_ld + (e0 >> 5)];
        uint32_t bits = (w >> (e0 & 31)) & ((1u << VEC) - 1u);
        int nvalid = min(VEC, P.V - e0);
        uint32_t need = (nvalid >= 32) ? 0xFFFFFFFFu : ((1u << nvalid) - 1u);
        if ((bits & need) == need) continue;
        T *p = reinterpret_cast<T *>(P.logits) + (int64_t)row * P.ld + e0;
        uint4 r = *reinterpret_cast<uint4 *>(p);
        uint32_t *rw = reinterpret_cast<uint32_t *>(&r);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            if (e < nvalid && !((bits >> e) & 1u)) {
                if (VEC == 4) {
                    rw[e] = 0xFF800000u;
                } else {
                    uint32_t sh = (e & 1) * 16;
                    rw[e >> 1] = (rw[e >> 1] & ~(0xFFFFu << sh)) | (0xFF80u << sh);
                }
            }
        }
        *reinterpret_cast<uint4 *>(p) = r;
    }
}

hipError_t launch_mask(const MaskParams &P, hipStream_t st) {
    const int VEC = P.dtype == 0 ? 4 : 8;
    int64_t total = (int64_t)((P.V + VEC - 1) / VEC) * P.rows;
    int64_t blocks = (total + kThreads - 1) / kThreads;
    if (blocks > 8192) blocks = 8192;
    if (blocks < 1) blocks = 1;
    if (P.dtype == 0)
        hipLaunchKernelGGL(mask_kernel<float>, dim3((unsigned)blocks), dim3(kThreads), 0, st, P);
    else
        hipLaunchKernelGGL(mask_kernel<uint16_t>, dim3((unsigned)blocks), dim3(kThreads), 0, st, P);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void window_compact_kernel(const uint32_t *hist, const int32_t *hist_len,
                                                               int hist_ld, int win, uint32_t *out,
                                                               int32_t *out_len) {
    const int row = blockIdx.x;
    int hl = hist_len[row];
    hl = hl < 0 ? 0 : (hl > hist_ld ? hist_ld : hl);
    const int nw = hl < win ? hl : win;
    const uint32_t *src = hist + (int64_t)row * hist_ld + (hl - nw);
    for (int i = threadIdx.x; i < nw; i += 256) out[(int64_t)row * kMaxWinHost + i] = src[i];
    if (threadIdx.x == 0) out_len[row] = nw;
}

hipError_t launch_window_compact(const uint32_t *hist, const int32_t *hist_len, int hist_ld, int win, int rows,
                                 uint32_t *out, int32_t *out_len, hipStream_t st) {
    if (win > kMaxWinHost) return hipErrorInvalidValue;
    hipLaunchKernelGGL(window_compact_kernel, dim3(rows), dim3(256), 0, st, hist, hist_len, hist_ld, win, out,
                       out_len);
    return hipGetLastError();
}

}  // namespace zi
