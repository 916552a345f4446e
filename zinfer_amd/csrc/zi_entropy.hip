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
// ref)(x - ref) over its elements; ref moves up only when an element exceeds
// it by 64 so the f32 sums cannot overflow.  Workgroup and row merges are in
// f64.
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
        if (m4 > *ref + 64.0f) {  // also the first finite value (ref = -inf)
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
    __shared__ float s_wmax[kWaves];
    __shared__ double s_ws[kWaves], s_wu[kWaves];
    __shared__ double s_M, s_Z;

    const RowSource &a = P.src;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
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

    // workgroup merge of (ref, S, U) in f64
    float wm = wave_max_f(ref);
    if (lane == 0) s_wmax[wid] = wm;
    __syncthreads();
    float M = s_wmax[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_wmax[w]);
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
        s_ws[wid] = ds;
        s_wu[wid] = du;
    }

    const int64_t rg = (int64_t)row * G + g;
    ChunkOut out{P.g_key + rg * kCapA, P.g_val + rg * kCapA, P.g_cnt + rg};
    chunk_select_publish<T, NV, false>(a, cr, c0, k, sm.a.sel, nullptr, nullptr, s_tau, &s_n, s_bins, s_dig, out);
    if (tid == 0) {
        double ts = 0.0, tu = 0.0;
        for (int w = 0; w < kWaves; ++w) {
            ts += s_ws[w];
            tu += s_wu[w];
        }
        st_agent(&P.g_stat[rg * 3], (double)M);
        st_agent(&P.g_stat[rg * 3 + 1], ts);
        st_agent(&P.g_stat[rg * 3 + 2], tu);
    }
    if (!row_ticket(P.tickets, row, G, &s_flag)) return;

    // ---------------- last workgroup of the row ----------------
    const int n = row_merge(P.g_key, P.g_val, P.g_cnt, row, G, k, sm.b.ml, sm.b.okey, sm.b.oval);
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
        uint32_t am = n > 0 ? ckey_id(sm.b.okey[0]) : 0u;
        if (P.argmax) P.argmax[row] = am;
        if (P.accept && P.draft) P.accept[row] = (uint8_t)(am == P.draft[row]);
    }
    __syncthreads();
    if (tid < n) {
        int64_t o = (int64_t)row * P.out_ld + tid;
        if (P.ids) P.ids[o] = ckey_id(sm.b.okey[tid]);
        if (P.probs) P.probs[o] = (float)(exp((double)sm.b.oval[tid] - s_M) / s_Z);
    }
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
