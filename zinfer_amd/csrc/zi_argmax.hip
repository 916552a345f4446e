// zi_argmax.hip -- batched argmaxWithMargin (src/sampler.zig:532-614), also
// the greedy branch of sampleWithMargin (temp <= 0, :191-193) when the row
// source carries a mask / penalty window / edits.
//
// The reference scans 16 lane classes (class = id mod 16, ids below
// 16*floor(V/16)), keeps each class's first maximum (strict >), reduces the
// classes in the order 0,8,1,9,...,7,15 with strict >, then scans the tail
// ids sequentially.  Its winner is the first class in that order holding the
// maximum, and its margin uses the class maxima and tail values only.  Here
// each chunk reduces per-class (max, lowest id) records -- the same thing as
// "first maximum" within a class -- plus the row's top-2 values; the last
// workgroup of the row replays the reference's 16-class + tail reduction.
#include "zi_launch.hpp"
#include "zi_rowpass.hpp"

namespace zi {

__device__ __forceinline__ void top2_merge(float &t1, float &t2, float o1, float o2) {
    t2 = fmaxf(fmaxf(t2, o2), fminf(t1, o1));
    t1 = fmaxf(t1, o1);
}

__device__ __forceinline__ void ref_step(float v, uint32_t id, float &best, float &second, uint32_t &best_idx) {
    if (v > best) {  // src/sampler.zig:581-587
        second = best;
        best = v;
        best_idx = id;
    } else if (v > second) {
        second = v;
    }
}

template <bool P>
struct ArgPenLds {
    PenTable pen;
};
template <>
struct ArgPenLds<false> {};

template <typename T, int NV, bool HAS_MASK, bool HAS_PEN, bool CAP>
__global__ __launch_bounds__(kThreads) void argmax_kernel(ArgmaxParams P) {
    __shared__ ArgPenLds<HAS_PEN> pl;
    __shared__ unsigned long long s_ck[16];
    __shared__ uint32_t s_raw[16];
    __shared__ float s_tail[16];
    __shared__ float s_t1[kWaves], s_t2[kWaves];
    __shared__ int s_flag;

    constexpr int VEC = VecTraits<T>::VEC;
    const RowSource &a = P.src;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int G = a.G;
    const int row = blockIdx.x / G;
    const int g = blockIdx.x - row * G;
    const int c0 = g * a.CH;
    const int c1 = min(a.V, c0 + a.CH);
    const int body_end = a.V & ~15;

    PenTable *pen = nullptr;
    if constexpr (HAS_PEN) pen = &pl.pen;
    PenOwn own;
    if (tid < 16) {
        s_ck[tid] = 0ull;
        s_raw[tid] = 0x7FC00000u;
        s_tail[tid] = __builtin_nanf("");
    }
    ChunkRegs<T, NV> cr;
    chunk_stream<T, NV, HAS_MASK, HAS_PEN, CAP>(a, row, c0, c1, cr, pen, &own);
    __syncthreads();  // s_* initialised

    // per-thread class records (thread t only meets classes (t*VEC + e) & 15)
    uint64_t ck[VEC];
    float t1 = -INFINITY, t2 = -INFINITY;
#pragma unroll
    for (int e = 0; e < VEC; ++e) ck[e] = 0ull;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        int e0 = c0 + (j * kThreads + tid) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            int id = e0 + e;
            float x = cr.x[j * VEC + e];
            if (x == x) {  // NaN: past the chunk, diverted, or a NaN input
                if (id < body_end) {
                    uint64_t k = ckey(x, (uint32_t)id);
                    ck[e] = k > ck[e] ? k : ck[e];
                } else {
                    s_tail[id - body_end] = x;
                }
                top2_merge(t1, t2, x, -INFINITY);
            }
        }
    }
    // penalized elements, each from its owner thread
    if constexpr (HAS_PEN) {
#pragma unroll
        for (int u = 0; u < kOwnSlots; ++u) {
            const uint32_t id = own.id[u];
            if (id != 0xFFFFFFFFu) {
                const float v = owned_value(a, *pen, own, u);
                if (v == v) {
                    if ((int)id < body_end) atomicMax(&s_ck[id & 15], (unsigned long long)ckey(v, id));
                    else s_tail[id - body_end] = v;
                    top2_merge(t1, t2, v, -INFINITY);
                }
            }
        }
    }
    // reduce records over lanes sharing the same classes, top-2 over the wave
#pragma unroll
    for (int m = 16 / VEC; m < 64; m <<= 1) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            uint64_t o = shfl_xor_u64(ck[e], m);
            ck[e] = o > ck[e] ? o : ck[e];
        }
        top2_merge(t1, t2, __shfl_xor(t1, m), __shfl_xor(t2, m));
    }
#pragma unroll
    for (int m = 1; m < 16 / VEC; m <<= 1) top2_merge(t1, t2, __shfl_xor(t1, m), __shfl_xor(t2, m));
    const int cls0 = (tid * VEC) & 15;
    if (lane < 16 / VEC) {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
            if (ck[e]) atomicMax(&s_ck[cls0 + e], (unsigned long long)ck[e]);
    }
    if (lane == 0) {
        s_t1[wid] = t1;
        s_t2[wid] = t2;
    }
    __syncthreads();
    // the owner of each class winner publishes its raw bits (keeps -0 vs +0)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        int e0 = c0 + (j * kThreads + tid) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            int id = e0 + e;
            float x = cr.x[j * VEC + e];
            if (id < body_end && x == x && ckey(x, (uint32_t)id) == s_ck[cls0 + e])
                s_raw[cls0 + e] = __float_as_uint(x);
        }
    }
    if constexpr (HAS_PEN) {
#pragma unroll
        for (int u = 0; u < kOwnSlots; ++u) {
            const uint32_t id = own.id[u];
            if (id != 0xFFFFFFFFu) {
                const float v = owned_value(a, *pen, own, u);
                if ((int)id < body_end && v == v && ckey(v, id) == s_ck[id & 15]) s_raw[id & 15] = __float_as_uint(v);
            }
        }
    }
    __syncthreads();
    const int64_t rg = (int64_t)row * G + g;
    if (tid < 16) {
        st_agent(&P.g_cls[rg * 16 + tid], (uint64_t)s_ck[tid]);
        st_agent(&P.g_raw[rg * 16 + tid], s_raw[tid]);
        if (body_end + tid < a.V && body_end + tid >= c0 && body_end + tid < c1)
            st_agent(&P.g_tail[(int64_t)row * 16 + tid], s_tail[tid]);
    }
    if (tid == 0) {
        float a1 = s_t1[0], a2 = s_t2[0];
        for (int w = 1; w < kWaves; ++w) top2_merge(a1, a2, s_t1[w], s_t2[w]);
        st_agent(&P.g_top2[rg * 2], a1);
        st_agent(&P.g_top2[rg * 2 + 1], a2);
    }
    if (!row_ticket(P.tickets, row, G, &s_flag)) return;
    if (tid != 0) return;

    // ---------------- the last workgroup of the row: lane 0 ----------------
    const int V = a.V;
    uint64_t cls[16];
    uint32_t craw[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        cls[c] = 0ull;
        craw[c] = 0x7FC00000u;
    }
    float a1 = -INFINITY, a2 = -INFINITY;
    for (int gg = 0; gg < G; ++gg) {
        const int64_t r2 = (int64_t)row * G + gg;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            uint64_t k = ld_agent(&P.g_cls[r2 * 16 + c]);
            uint32_t rw = ld_agent(&P.g_raw[r2 * 16 + c]);
            if (k > cls[c]) {
                cls[c] = k;
                craw[c] = rw;
            }
        }
        top2_merge(a1, a2, ld_agent(&P.g_top2[r2 * 2]), ld_agent(&P.g_top2[r2 * 2 + 1]));
    }
    const int nt = V - body_end;
    float *tl = s_tail;  // reused: this workgroup's own tail copy is no longer needed
    for (int i = 0; i < nt; ++i) tl[i] = ld_agent(&P.g_tail[(int64_t)row * 16 + i]);

    uint32_t tok = 0;
    float margin = 10.0f;
    if (V == 1) {  // :534
        tok = 0;
        margin = 10.0f;
    } else if (V < 16) {  // :535-551, all V values are in the tail buffer
        uint32_t best = 0, second = 1;
        if (tl[1] > tl[0]) {
            best = 1;
            second = 0;
        }
        for (int i = 2; i < V; ++i) {
            if (tl[i] > tl[best]) {
                second = best;
                best = (uint32_t)i;
            } else if (tl[i] > tl[second]) {
                second = (uint32_t)i;
            }
        }
        tok = best;
        margin = tl[best] - tl[second];
    } else {  // :553-609
        float best = -INFINITY, second = -INFINITY;
        uint32_t best_idx = 0;
        for (int j = 0; j < 8; ++j) {
            ref_step(__uint_as_float(craw[j]), ckey_id(cls[j]), best, second, best_idx);
            ref_step(__uint_as_float(craw[j + 8]), ckey_id(cls[j + 8]), best, second, best_idx);
        }
        for (int i = 0; i < nt; ++i) ref_step(tl[i], (uint32_t)(body_end + i), best, second, best_idx);
        tok = best_idx;
        margin = (second > -INFINITY) ? best - second : 10.0f;
    }
    if (P.tok) P.tok[row] = tok;
    if (P.margin) P.margin[row] = margin;
    if (P.ndraws) P.ndraws[row] = 0;
    if (P.tok_low) {
        uint64_t best = 0ull;
#pragma unroll
        for (int c = 0; c < 16; ++c) best = cls[c] > best ? cls[c] : best;
        for (int i = 0; i < nt; ++i) {
            float x = tl[i];
            if (x == x) {
                uint64_t k = ckey(x, (uint32_t)(body_end + i));
                best = k > best ? k : best;
            }
        }
        P.tok_low[row] = best ? ckey_id(best) : 0u;
    }
    if (P.margin_true) P.margin_true[row] = (V >= 2 && a2 > -INFINITY) ? a1 - a2 : 10.0f;
}

template <typename T, int NV, bool M, bool PN>
static hipError_t launch_argmax_t(const ArgmaxParams &P, int rows, hipStream_t st) {
    dim3 grid(rows * P.src.G), block(kThreads);
    if (P.src.cap > 0.0f) hipLaunchKernelGGL((argmax_kernel<T, NV, M, PN, true>), grid, block, 0, st, P);
    else hipLaunchKernelGGL((argmax_kernel<T, NV, M, PN, false>), grid, block, 0, st, P);
    return hipGetLastError();
}

template <typename T, int NV>
static hipError_t launch_argmax_nv(const ArgmaxParams &P, int rows, hipStream_t st) {
    const bool m = P.src.mask != nullptr;
    const bool p = (P.src.hist != nullptr) || (P.src.edit_ids != nullptr);
    if (m && p) return launch_argmax_t<T, NV, true, true>(P, rows, st);
    if (m) return launch_argmax_t<T, NV, true, false>(P, rows, st);
    if (p) return launch_argmax_t<T, NV, false, true>(P, rows, st);
    return launch_argmax_t<T, NV, false, false>(P, rows, st);
}

hipError_t launch_argmax(const ArgmaxParams &P, int dtype, int nv, int rows, hipStream_t st) {
    if (dtype == 0) {
        switch (nv) {
            case 4: return launch_argmax_nv<float, 4>(P, rows, st);
            case 8: return launch_argmax_nv<float, 8>(P, rows, st);
            default: return launch_argmax_nv<float, 16>(P, rows, st);
        }
    }
    switch (nv) {
        case 2: return launch_argmax_nv<uint16_t, 2>(P, rows, st);
        case 4: return launch_argmax_nv<uint16_t, 4>(P, rows, st);
        default: return launch_argmax_nv<uint16_t, 8>(P, rows, st);
    }
}

}  // namespace zi
