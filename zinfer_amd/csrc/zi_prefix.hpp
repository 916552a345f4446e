// zi_prefix.hpp -- the min-p prefix of whole-vocabulary rows (top_k = 0 or >=
// V with min_p > 0, src/sampler.zig:197-234) for batches of >= 256 rows, one
// workgroup per row, streamed without workgroup barriers.
//
// The reference sorts the whole row (std.mem.sort, sampler.zig:198-201), but
// its keep never passes the first entry with exp(x - mx) < min_p (:229-234),
// so only the entries above minp_floor(mx) (and the row's top two, for the
// margin) can matter; the rest of the tail reads them alone when the bounded
// total settles keep (nucleus_keep), and the row goes to the exact
// whole-order pass otherwise.
//
// Per row:
//  1. The penalty window and the edits are loaded once: a bitset of their ids
//     over the whole row and an id -> (count, delta) hash in LDS; the thread
//     that sets an id's bit owns it and loads its logit (mask and softcap
//     applied) while the row streams.
//  2. The row streams in steps of what the registers hold; each vector's
//     register takes the next step's load as soon as the vector is consumed.
//     Penalized ids leave the stream (NaN); the rest feed each thread's
//     (ref, sum exp(x - ref)) for the row total and each wave's running top
//     two lane maxima.
//  3. Each wave keeps its own threshold thr_w = min(minp_floor(m_w), m2_w)
//     from its running top two (both lower bounds of the row's maximum and
//     second entry, so thr_w never passes an entry the final floor keeps) and
//     appends its elements >= thr_w to its own region of an LDS buffer at a
//     wave-uniform count (no atomics).  No step waits at a barrier.
//  4. At the end: the row maximum (stream maxima and penalized values), the
//     row total, and the entries at or above the final floor tf (plus the
//     row's second entry when only the maximum reaches tf) are ranked into
//     the sorted prefix; the reference tail runs on it.
// A buffer overflow (flat rows: thousands of entries tie above the floor)
// sends the row to the exact pass, which is always correct.  The workgroup's
// LDS stays under 80 KiB so that two rows stream on each CU at once.
#pragma once
#include "zi_rowpass.hpp"
#include "zi_tail.hpp"

#include <cfloat>
#include <type_traits>

namespace zi {

// The whole-vocabulary prefix threshold for min_p > 0: an entry below it has
// exp(x - M) < min_p for every maximum >= M, with room for the f32 rounding of
// x - M and of the threshold itself (rounded down).  Monotone in M.
__device__ __forceinline__ float minp_floor(float M, double ln_minp) {
    const double d = (double)M + ln_minp - 0.01 - 1e-6 * fabs((double)M);
    float t = (float)d;
    if ((double)t > d) t = __uint_as_float(t > 0.0f ? __float_as_uint(t) - 1u : __float_as_uint(t) + 1u);
    return t;
}

constexpr int kPrefMarks = 2048;                // vectors with a hit, per row
constexpr int kPrefWave = kPrefMarks / kWaves;  // each wave's region of them
constexpr int kPrefCap = 1024;                  // entries at or above the floor, per row
constexpr int kPrefRank = kThreads;             // filtered entries ranked with one entry per thread

// Candidate keys: the ckey() order (value descending, id ascending) with the
// value's sign of zero kept in bit 0, below the id, so that the value is
// recovered exactly from the key alone.
__device__ __forceinline__ uint64_t pkey(float v, uint32_t id) {
    const uint32_t z = __float_as_uint(v) == 0x80000000u ? 1u : 0u;
    return ((uint64_t)okey(v) << 32) | (uint64_t)((~id << 1) | z);
}
__device__ __forceinline__ float pkey_val(uint64_t k) {
    return (k & 1u) ? -0.0f : okey_inv((uint32_t)(k >> 32));
}
__device__ __forceinline__ uint64_t pkey_ckey(uint64_t k) {
    const uint32_t id = ~((uint32_t)k >> 1) & 0x7FFFFFFFu;
    return (k & 0xFFFFFFFF00000000ull) | (uint64_t)(~id);
}

// Under 80 KiB, so that two workgroups share a CU.
struct PrefixLds {
    uint32_t bits[kMaxVocab / 32];  // ids of the penalty window and the edits
    uint32_t hkey[kHashMax];        // id + 1 -> window count, edit delta
    uint32_t hcnt[kHashMax];
    float hdelta[kHashMax];
    uint32_t mark[kPrefMarks];  // first ids of the vectors with a hit, kPrefWave per wave
    uint64_t fkey[kPrefCap];    // the entries at or above the floor (pkey)
    uint64_t okey[kCapA];       // the sorted prefix
    float oval[kCapA];
    TailLds tl;
    float pub[kWaves][2];  // each wave's running top two lane maxima, raised as it streams
    float wmax[kWaves];
    double ws[kWaves];
    uint64_t wbelow[kWaves];
    int wcn[kWaves];  // marks each wave appended
    int fn;
};
static_assert(sizeof(PrefixLds) <= 80 * 1024, "two prefix workgroups per CU");

__device__ __forceinline__ int prefix_hash_insert(PrefixLds &L, uint32_t id, int hs_log2) {
    uint32_t h = hash_slot(id, hs_log2);
    const uint32_t m = (1u << hs_log2) - 1;
    for (;;) {
        const uint32_t prev = atomicCAS(&L.hkey[h], 0u, id + 1);
        if (prev == 0u || prev == id + 1) return (int)h;
        h = (h + 1) & m;
    }
}

// Appends the keys of the lanes with p to `buf` at the count *n; one LDS
// atomic per wave.  Every lane of the wave calls it.
__device__ __forceinline__ void prefix_append(uint64_t *buf, int *n, bool p, uint64_t key) {
    const uint64_t b = ballot(p);
    if (!b) return;
    const int lead = __ffsll((unsigned long long)b) - 1;
    int base = 0;
    if (lane_id() == lead) base = atomicAdd(n, __popcll(b));
    base = __shfl(base, lead);
    const int pos = base + lanes_below(b);
    if (p && pos < kPrefCap) buf[pos] = key;
}

// A workgroup barrier that orders LDS only: it waits for this wave's LDS
// operations, not for its global loads in flight (which __syncthreads() does,
// through its workgroup-scope fence).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// A logit as loaded (the 16-bit pattern of a bfloat16 in the low half) and
// as a value.
template <typename T>
__device__ __forceinline__ uint32_t load_raw(const T *row, uint32_t id);
template <>
__device__ __forceinline__ uint32_t load_raw<float>(const float *row, uint32_t id) {
    return __float_as_uint(row[id]);
}
template <>
__device__ __forceinline__ uint32_t load_raw<uint16_t>(const uint16_t *row, uint32_t id) {
    return (uint32_t)row[id];
}
template <typename T>
__device__ __forceinline__ float raw_value(uint32_t r) {
    return std::is_same<T, float>::value ? __uint_as_float(r) : __uint_as_float(r << 16);
}

__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, __uint_as_float(lane_xor<1>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(lane_xor<2>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(lane_xor<4>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(lane_xor<8>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(lane_xor<16>(__float_as_uint(v))));
    v = fmaxf(v, __uint_as_float(lane_xor<32>(__float_as_uint(v))));
    return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const uint64_t o = shfl_xor_u64(v, m);
        v = o > v ? o : v;
    }
    return v;
}

// Vector [id0, id0 + VEC) of the row as values: softcap, mask bits mword
// (bit (id0 & 31) first); penalized ids and ids at or past lim_id as -inf
// (no maximum, no candidate, no weight).
template <typename T, bool HAS_MASK, bool HAS_PEN, bool CAP>
__device__ __forceinline__ void prefix_prep(const RowSource &a, const PrefixLds &L, uint4 raw, uint32_t mword,
                                            int id0, int lim_id, float (&v)[VecTraits<T>::VEC],
                                            const uint32_t *pword = nullptr) {
    constexpr int VEC = VecTraits<T>::VEC;
    unpack<T>(raw, v);
    if constexpr (CAP) softcap_vec<VEC>(a, id0, v);
    if (HAS_MASK) {
        const uint32_t mb = mword >> (id0 & 31);
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = ((mb >> e) & 1u) ? v[e] : -INFINITY;
    }
    const int lim = lim_id - id0;
    // (a word passed in is in bounds for any id0; ids past lim_id go to -inf below either way)
    if (HAS_PEN && (pword != nullptr || lim > 0)) {
        const uint32_t pb = ((pword ? *pword : L.bits[id0 >> 5]) >> (id0 & 31)) & ((1u << VEC) - 1u);
        if (pb) {
#pragma unroll
            for (int e = 0; e < VEC; ++e) v[e] = ((pb >> e) & 1u) ? -INFINITY : v[e];
        }
    }
    if (lim < VEC) {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
            if (e >= lim) v[e] = -INFINITY;
    }
}

template <typename T, int NV, bool HAS_MASK, bool HAS_PEN, bool CAP>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void prefix_kernel(SampleParams P) {
    __shared__ PrefixLds L;
    constexpr int VEC = VecTraits<T>::VEC;
    constexpr int SUB = kThreads * NV * VEC;  // elements per step
    const RowSource &a = P.src;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int row = blockIdx.x;
    const int V = a.V;
    const T *lrow = reinterpret_cast<const T *>(a.logits) + (int64_t)row * a.ld;
    const uint32_t *mrow = HAS_MASK ? a.mask + (int64_t)row * a.mask_ld : nullptr;
    int ur = 2 * row;
    asm volatile("" : "+v"(ur));
    const float u0 = P.uniforms[ur], u1 = P.uniforms[ur + 1];
    const double ln_minp = log((double)P.min_p);

    // The penalty inputs first (the whole history row, its length, the
    // edits), then the first step's loads: waiting for the former never waits
    // for the latter.
    // (Loads without branches: a load whose value merges at a branch is waited
    // for there.  A disabled input reads a valid word it then ignores.)
    PenRegs pr;
    int hl_raw = 0, ne_raw = 0;
    if constexpr (HAS_PEN) {
        pen_prefetch(a, row, pr);
        const int32_t *any = reinterpret_cast<const int32_t *>(P.uniforms);
        hl_raw = *(row_pen_window_on(a) ? a.hist_len + row : any);
        ne_raw = *(a.edit_ids ? a.edit_count + row : any);
        asm volatile("" ::: "memory");  // issued here, not sunk past the row's loads
    }
    uint4 raw[NV];
    uint32_t mw[NV];
    const int nvec_row = (V + VEC - 1) / VEC;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int q = min(j * kThreads + tid, nvec_row - 1);
        raw[j] = ld_stream(reinterpret_cast<const uint4 *>(lrow + q * VEC));
        if (HAS_MASK) mw[j] = mrow[(q * VEC) >> 5];
    }

    // 1. penalties: bitset and hash of the window and edits, owners' logits
    constexpr int kOwn = kOwnSlots;
    uint32_t oid[kOwn];
    uint32_t oraw[kOwn];  // the owners' logits and mask words as loaded, used at the end
    int oslot[kOwn];
#pragma unroll
    for (int u = 0; u < kOwn; ++u) {
        oid[u] = 0xFFFFFFFFu;
        oraw[u] = 0u;
        oslot[u] = 0;
    }
    uint32_t omw[HAS_MASK ? kOwn : 1];
#pragma unroll
    for (int u = 0; u < (HAS_MASK ? kOwn : 1); ++u) omw[u] = 0u;
    RowPen rp;
    rp.any = false;
    rp.hs_log2 = 6;
    if constexpr (HAS_PEN) {
        rp = row_pen_from(a, row, hl_raw, ne_raw);
        pen_window(rp, pr);
        for (int i = tid; i < (V + 31) / 32; i += kThreads) L.bits[i] = 0u;
        for (int i = tid; i < kHashMax; i += kThreads) {
            L.hkey[i] = 0u;
            L.hcnt[i] = 0u;
            L.hdelta[i] = 0.0f;
        }
        lds_barrier();  // cleared
#pragma unroll
        for (int u = 0; u < kOwn; ++u) {
            const uint32_t id = u < kWinPerThread ? pr.w[u] : pr.e;
            if (id < (uint32_t)V) {
                const uint32_t bit = 1u << (id & 31);
                if (!(atomicOr(&L.bits[id >> 5], bit) & bit)) oid[u] = id;
                const int h = prefix_hash_insert(L, id, rp.hs_log2);
                if (u < kWinPerThread) atomicAdd(&L.hcnt[h], 1u);
                else L.hdelta[h] = pr.d;
                if (oid[u] == id) oslot[u] = h;
            }
        }
#pragma unroll
        for (int u = 0; u < kOwn; ++u) {  // the owners' logits, needed only at the end
            const uint32_t id = oid[u] != 0xFFFFFFFFu ? oid[u] : 0u;
            oraw[u] = load_raw<T>(lrow, id);
            if (HAS_MASK) omw[u] = mrow[id >> 5];
        }
    }
    if (lane == 0) {
        L.pub[wid][0] = -INFINITY;
        L.pub[wid][1] = -INFINITY;
    }
    lds_barrier();  // bitset, hash and published pairs ready

    // 2-3. stream, totals, thresholds, marks
    // This thread's running sum exp(x - ref): ref starts finite and far below
    // any logit (exp of -inf - ref is then 0, not NaN) and lags the running
    // maximum by at most kRefLag, so each term is <= e^kRefLag and the sum
    // stays far from overflow; it is rescaled only when a vector passes it.
    constexpr float kRefLag = 20.0f;
    float ref = -1e30f, S = 0.0f;
    float m_run = -INFINITY, m2_run = -INFINITY;  // this wave's two largest lane maxima (distinct lanes)
    float thr = -FLT_MAX;  // marked vectors hold an entry >= thr, so never only -inf (or NaN)
    uint32_t *wmark = L.mark + wid * kPrefWave;  // this wave's marks
    int wcnt = 0;                                // wave-uniform
    // After each step: this wave's running top two, published, and the
    // threshold from every wave's latest published pair.  The largest value
    // over all pairs is a lower bound of the row's maximum and the second
    // largest one of its second entry (the values are those of distinct
    // entries), so thr = min(minp_floor(first), second) never passes an
    // entry the final floor keeps, nor the row's second entry.  A pair read
    // before its wave raises it is only lower.
    auto raise = [&](float lmax) {
        const float wm = wave_max_dpp(lmax);
        const uint64_t top = ballot(lmax == wm);
        const float w2 = __popcll(top) >= 2 ? wm : wave_max_dpp(lmax == wm ? -INFINITY : lmax);
        if (wm > m_run) {
            m2_run = fmaxf(m_run, w2);
            m_run = wm;
        } else {
            m2_run = fmaxf(m2_run, wm);
        }
        uint32_t *pub = reinterpret_cast<uint32_t *>(&L.pub[0][0]);  // read and written while other waves stream
        if (lane == 0) {
            __hip_atomic_store(pub + 2 * wid, __float_as_uint(m_run), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            __hip_atomic_store(pub + 2 * wid + 1, __float_as_uint(m2_run), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        float f = -INFINITY, sc = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float p0 = __uint_as_float(__hip_atomic_load(pub + 2 * w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
            const float p1 =
                __uint_as_float(__hip_atomic_load(pub + 2 * w + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
            const float x0 = w == wid ? m_run : p0;
            const float x1 = w == wid ? m2_run : p1;  // x1 <= x0
            sc = fmaxf(sc, fmaxf(fminf(f, x0), x1));
            f = fmaxf(f, x0);
        }
        if (f != -INFINITY) thr = fmaxf(thr, fmaxf(fminf(minp_floor(f, ln_minp), sc), -FLT_MAX));
    };
    {  // the first step's maxima set the first threshold
        const int c1 = min(V, SUB);
        float lmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            float v[VEC];
            prefix_prep<T, HAS_MASK, HAS_PEN, CAP>(a, L, raw[j], HAS_MASK ? mw[j] : 0u, (j * kThreads + tid) * VEC,
                                                   c1, v);
#pragma unroll
            for (int e = 0; e < VEC; ++e) lmax = fmaxf(lmax, v[e]);
        }
        raise(lmax);
        // the packed words are unpacked again below rather than kept as floats
#pragma unroll
        for (int j = 0; j < NV; ++j) asm volatile("" : "+v"(raw[j].x), "+v"(raw[j].y), "+v"(raw[j].z), "+v"(raw[j].w));
    }
    // One pass per step: each vector's register takes the next step's load
    // once it is consumed; the threshold a step uses is the one after the
    // previous step (lower, so it marks a superset).  A vector whose maximum
    // reaches the threshold is marked by its first id and read again at the
    // end.
    for (int c0 = 0; c0 < V; c0 += SUB) {
        const int c1 = min(V, c0 + SUB);
        const int n0 = c1, n1 = min(V, c1 + SUB);  // the next step
        const int nvec_next = (n1 - n0 + VEC - 1) / VEC;
        float lmax = -INFINITY;
        uint32_t pwv[NV];  // the step's penalty-bit words, read together
#pragma unroll
        for (int j = 0; j < NV; ++j)
            pwv[j] = HAS_PEN ? L.bits[min(c0 + (j * kThreads + tid) * VEC, V - 1) >> 5] : 0u;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int id0 = c0 + (j * kThreads + tid) * VEC;
            float v[VEC];
            prefix_prep<T, HAS_MASK, HAS_PEN, CAP>(a, L, raw[j], HAS_MASK ? mw[j] : 0u, id0, c1, v, &pwv[j]);
            if (n0 < n1) {  // uniform: the same vector of the next step
                const int nq = min(j * kThreads + tid, nvec_next - 1);
                raw[j] = ld_stream(reinterpret_cast<const uint4 *>(lrow + n0 + nq * VEC));
                if (HAS_MASK) mw[j] = mrow[(n0 + nq * VEC) >> 5];
            }
            float m = v[0];
#pragma unroll
            for (int e = 1; e < VEC; ++e) m = fmaxf(m, v[e]);
            lmax = fmaxf(lmax, m);
            const bool up = m > ref + kRefLag;
            if (ballot(up)) {  // a wave-uniform branch: taken about once per lane, so the rescale is not paid per vector
                if (up) {
                    S = S * __builtin_amdgcn_exp2f((ref - m) * kLog2e);
                    ref = m;
                }
                asm volatile("" : "+v"(S), "+v"(ref));  // keeps the branch (not flattened into selects)
            }
#pragma unroll
            for (int e = 0; e < VEC; ++e) S = S + __builtin_amdgcn_exp2f((v[e] - ref) * kLog2e);
            asm volatile("" : "+v"(S));  // summed here, not deferred with every vector's values live
            const bool hit = m >= thr;
            const uint64_t b = ballot(hit);
            if (!b) continue;
            const int pos = wcnt + lanes_below(b);
            if (hit && pos < kPrefWave) wmark[pos] = (uint32_t)id0;
            wcnt += __popcll(b);
        }
        if (c0 > 0) raise(lmax);  // the first step's maxima are in already
    }
    if (lane == 0) L.wcn[wid] = wcnt;

    // 4. the row maximum, total and floor
    float pv[kOwn];
    float omax = -INFINITY;
#pragma unroll
    for (int u = 0; u < kOwn; ++u) {
        pv[u] = -INFINITY;
        if (HAS_PEN && oid[u] != 0xFFFFFFFFu) {
            float v = raw_value<T>(oraw[u]);
            if constexpr (CAP) v = softcap_at(a, (int)oid[u], v);
            if (HAS_MASK && !((omw[HAS_MASK ? u : 0] >> (oid[u] & 31)) & 1u)) v = -INFINITY;
            pv[u] = pen_apply(v, L.hcnt[oslot[u]], L.hdelta[oslot[u]], a);
            omax = fmaxf(omax, pv[u]);
        }
    }
    if (omax > ref) {  // the penalized entries join this thread's total
        S = S * __builtin_amdgcn_exp2f((ref - omax) * kLog2e);
        ref = omax;
    }
#pragma unroll
    for (int u = 0; u < kOwn; ++u)
        if (pv[u] > -INFINITY) S = S + __builtin_amdgcn_exp2f((pv[u] - ref) * kLog2e);
    // the wave's largest entry: its stream maximum and its penalized values
    const float tmax = fmaxf(wave_max_dpp(omax), m_run);
    if (lane == 0) L.wmax[wid] = tmax;
    __syncthreads();  // maxima and mark counts
    float M = L.wmax[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, L.wmax[w]);
    double ds = M != -INFINITY ? (double)S * exp((double)ref - (double)M) : 0.0;
    ds = wave_sum_d(ds);
    if (lane == 0) L.ws[wid] = ds;
    if (tid == 0) L.fn = 0;
    bool overflow = false;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) overflow |= L.wcn[w] > kPrefWave;
    const bool empty = !(M > -INFINITY);  // every entry -inf or not selectable
    const float tf = minp_floor(M, ln_minp);
    __syncthreads();  // ws and fn
    double Z = 0.0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) Z += L.ws[w];
    if (tid < P.src.G) {  // the row total as per-chunk records (all in record 0) for the exact pass
        double *gs = P.g_stat + ((int64_t)row * P.src.G + tid) * 3;
        gs[0] = tid == 0 ? (double)M : -INFINITY;
        gs[1] = tid == 0 ? Z : 0.0;
        gs[2] = 0.0;
    }
    if (overflow || empty) {
        if (tid == 0) P.nuc_flag[row] = 1;
        return;
    }
    // The marked vectors, read again: their entries >= tf (with the penalized
    // ones, every entry >= tf: each threshold was <= tf), and each thread's
    // largest key below tf -- when only the maximum reaches tf, the largest
    // of those is the row's second entry (each threshold was also <= it).
    uint64_t below = 0;
    {
        int off[kWaves + 1];  // the marks as one list: wave w's at [off[w], off[w + 1])
        off[0] = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) off[w + 1] = off[w] + L.wcn[w];
        const int cn = off[kWaves];
        constexpr int R = kPrefMarks / kThreads;
        uint4 rr[R];
        uint32_t rmw[R];
        int rid[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {  // every load first
            const int t = tid + r * kThreads;
            rid[r] = -1;
            rmw[r] = 0u;
            rr[r] = make_uint4(0u, 0u, 0u, 0u);
            if (t < cn) {
                int w = 0;
#pragma unroll
                for (int k = 1; k < kWaves; ++k) w += t >= off[k] ? 1 : 0;
                rid[r] = (int)L.mark[w * kPrefWave + (t - off[w])];
                rr[r] = *reinterpret_cast<const uint4 *>(lrow + rid[r]);
                if (HAS_MASK) rmw[r] = mrow[rid[r] >> 5];
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (!ballot(rid[r] >= 0)) break;  // uniform: the marks fill the first slots
            float v[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) v[e] = -INFINITY;
            if (rid[r] >= 0) prefix_prep<T, HAS_MASK, HAS_PEN, CAP>(a, L, rr[r], rmw[r], rid[r], V, v);
            const uint32_t id0 = (uint32_t)max(rid[r], 0);
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const uint64_t k = pkey(v[e], id0 + (uint32_t)e);
                const bool p = v[e] >= tf && v[e] > -INFINITY;
                prefix_append(L.fkey, &L.fn, p, k);
                if (!p && v[e] > -INFINITY && k > below) below = k;
            }
        }
    }
#pragma unroll
    for (int u = 0; u < kOwn; ++u) {
        if (HAS_PEN && oid[u] != 0xFFFFFFFFu && pv[u] > -INFINITY) {
            const uint64_t k = pkey(pv[u], oid[u]);
            if (pv[u] >= tf) {
                const int pos = atomicAdd(&L.fn, 1);
                if (pos < kPrefCap) L.fkey[pos] = k;
            } else if (k > below) {
                below = k;
            }
        }
    }
    below = wave_max_u64(below);
    if (lane == 0) L.wbelow[wid] = below;
    __syncthreads();
    int fn = L.fn;
    const int m = fn;  // the entries >= tf
    if (fn > kPrefCap) {
        if (tid == 0) P.nuc_flag[row] = 1;
        return;
    }
    if (fn == 1) {  // uniform: the second entry joins
        uint64_t second = L.wbelow[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) second = L.wbelow[w] > second ? L.wbelow[w] : second;
        if (second) {
            if (tid == 0) L.fkey[1] = second;
            fn = 2;
            __syncthreads();
        }
    }
    // rank by counting: key i goes to okey[#greater] when that is < kCapA
    const int nl = min(fn, kCapA);  // the sorted list's length
    if (fn <= kPrefRank) {
        const uint64_t mine = tid < fn ? L.fkey[tid] : ~0ull;
        uint32_t c = 0;
        int q = 0;
        for (; q + 8 <= fn; q += 8) {
            uint64_t kk[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) kk[u] = L.fkey[q + u];
#pragma unroll
            for (int u = 0; u < 8; ++u) c += (uint32_t)(kk[u] > mine);
        }
        for (; q < fn; ++q) c += (uint32_t)(L.fkey[q] > mine);
        if (tid < fn && c < (uint32_t)kCapA) {
            L.okey[c] = pkey_ckey(mine);
            L.oval[c] = pkey_val(mine);
        }
    } else {  // up to kPrefCap / kThreads keys per thread, one sweep
        constexpr int R = kPrefCap / kThreads;
        uint64_t mine[R];
        uint32_t c[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            mine[r] = tid + r * kThreads < fn ? L.fkey[tid + r * kThreads] : ~0ull;
            c[r] = 0;
        }
        int q = 0;
        for (; q + 8 <= fn; q += 8) {
            uint64_t kk[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) kk[u] = L.fkey[q + u];
#pragma unroll
            for (int u = 0; u < 8; ++u)
#pragma unroll
                for (int r = 0; r < R; ++r) c[r] += (uint32_t)(kk[u] > mine[r]);
        }
        for (; q < fn; ++q) {
            const uint64_t kq = L.fkey[q];
#pragma unroll
            for (int r = 0; r < R; ++r) c[r] += (uint32_t)(kq > mine[r]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (tid + r * kThreads < fn && c[r] < (uint32_t)kCapA) {
                L.okey[c[r]] = pkey_ckey(mine[r]);
                L.oval[c[r]] = pkey_val(mine[r]);
            }
        }
    }
    __syncthreads();
    if (tid >= 64) return;  // the tail runs on wave 0 with all 64 lanes active
    // the prefix: every entry >= tf (at least the top two), capped at kCapA
    const int n = max(min(m, nl), min(2, nl));
    const bool complete = m < kCapA;  // nothing above tf was dropped by the cap
    if (n < 2 && P.n_all >= 2) {      // fewer than two entries in the row: whole-order pass
        if (tid == 0) P.nuc_flag[row] = 1;
        return;
    }
    const double tot = Z * exp((double)M - (double)L.oval[0]);
    sample_tail<true>(P, row, L.okey, L.oval, n, L.tl, u0, u1, tot, complete);
}

}  // namespace zi
