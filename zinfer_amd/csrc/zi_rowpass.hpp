// zi_rowpass.hpp -- the single streaming pass over a logit row chunk, fused
// with the grammar mask, the repetition/frequency/presence penalty and the
// sparse (DRY) edits, plus the cross-workgroup candidate machinery.
//
// Reference semantics fused here:
//   mask  : JsonValidator.applyMask, src/grammar.zig:446-479 (disallowed -> -inf),
//           applied before sampling (src/gen.zig:457-460).
//   pen   : Sampler.applyPenalty, src/sampler.zig:91-100 (each distinct id of the
//           window once: l > 0 ? l / rp : l * rp), then the frequency/presence
//           extension l -= fl(fl(count * freq) + presence).
//   edits : the DRY subtraction logits[tok] -= penalty, src/sampler.zig:184.
#pragma once
#include "zi_common.hpp"
#include "zi_launch.hpp"

namespace zi {

constexpr int kMaxCH = kMaxChunkElems;  // max chunk elements (256 threads x 64)
constexpr int kHashMax = 2048;          // LDS hash slots (window + edits <= 1152 ids)
constexpr int kMaxWin = kMaxWinHost;    // max penalty window
constexpr int kMaxEdits = kMaxEditsHost;
constexpr int kCapA = kCapAHost;        // candidates one chunk may publish
constexpr int kMaxG = kMaxGHost;        // max chunks per row (V <= 262144)
static_assert(kThreads == kThreadsHost, "workgroup size");

// RowSource is declared in zi_launch.hpp (host-visible).

struct PenTable {
    uint32_t bits[kMaxCH / 32];
    uint32_t key[kHashMax];
    uint32_t cnt[kHashMax];
    float delta[kHashMax];
};

__device__ __forceinline__ uint32_t hash_slot(uint32_t id, int hs_log2) {
    return (id * 2654435761u) >> (32 - hs_log2);
}

__device__ __forceinline__ int pen_insert(PenTable &t, uint32_t id, int hs_log2) {
    uint32_t h = hash_slot(id, hs_log2);
    const uint32_t m = (1u << hs_log2) - 1;
    for (;;) {
        uint32_t prev = atomicCAS(&t.key[h], 0u, id + 1);
        if (prev == 0u || prev == id + 1) return (int)h;
        h = (h + 1) & m;
    }
}

__device__ __forceinline__ int pen_find(const PenTable &t, uint32_t id, int hs_log2) {
    uint32_t h = hash_slot(id, hs_log2);
    const uint32_t m = (1u << hs_log2) - 1;
    while (t.key[h] != id + 1) h = (h + 1) & m;
    return (int)h;
}

// Per-row window bounds: the last min(hist_len, win) entries of hist.
struct RowPen {
    const uint32_t *win_ptr;
    int nw;
    const uint32_t *eid;
    const float *edl;
    int ne;
    int hs_log2;
    bool any;
};

__device__ __forceinline__ RowPen row_pen(const RowSource &a, int row) {
    RowPen r;
    r.nw = 0;
    r.win_ptr = nullptr;
    if (a.hist && (a.do_rep || a.do_fp) && a.win > 0) {
        int hl = a.hist_len[row];
        hl = hl < 0 ? 0 : (hl > a.hist_ld ? a.hist_ld : hl);
        r.nw = hl < a.win ? hl : a.win;
        r.win_ptr = a.hist + (int64_t)row * a.hist_ld + (hl - r.nw);
    }
    r.ne = 0;
    r.eid = nullptr;
    r.edl = nullptr;
    if (a.edit_ids) {
        int ne = a.edit_count[row];
        r.ne = ne < 0 ? 0 : (ne > a.edit_ld ? a.edit_ld : ne);
        r.ne = r.ne > kMaxEdits ? kMaxEdits : r.ne;
        r.eid = a.edit_ids + (int64_t)row * a.edit_ld;
        r.edl = a.edit_delta + (int64_t)row * a.edit_ld;
    }
    int n = r.nw + r.ne;
    int lg = 6;
    while ((1 << lg) < 2 * n && lg < 11) ++lg;
    r.hs_log2 = lg;
    r.any = n > 0;
    return r;
}

// Fetches this thread's share of the window and edits (issued before the
// logit loads so that waiting for them does not wait for the row).
struct PenRegs {
    uint32_t w[kMaxWin / kThreads];
    uint32_t e;
    float d;
};

__device__ __forceinline__ void pen_fetch(const RowPen &rp, PenRegs &pr) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int u = 0; u < kMaxWin / kThreads; ++u) {
        int i = tid + u * kThreads;
        pr.w[u] = (i < rp.nw) ? rp.win_ptr[i] : 0xFFFFFFFFu;
    }
    pr.e = (tid < rp.ne) ? rp.eid[tid] : 0xFFFFFFFFu;
    pr.d = (tid < rp.ne) ? rp.edl[tid] : 0.0f;
}

// Builds the chunk's bitset of penalized/edited ids and the id -> (count,
// delta) hash.  Contains barriers: call from all threads.
__device__ __forceinline__ void pen_build(PenTable &t, const RowPen &rp, const PenRegs &pr, int c0, int c1) {
    const int tid = threadIdx.x;
    const int hs = 1 << rp.hs_log2;
    for (int i = tid; i < kMaxCH / 32; i += kThreads) t.bits[i] = 0u;
    for (int i = tid; i < hs; i += kThreads) {
        t.key[i] = 0u;
        t.cnt[i] = 0u;
        t.delta[i] = 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kMaxWin / kThreads; ++u) {
        uint32_t id = pr.w[u];
        if (id >= (uint32_t)c0 && id < (uint32_t)c1) {
            int h = pen_insert(t, id, rp.hs_log2);
            atomicAdd(&t.cnt[h], 1u);
            atomicOr(&t.bits[(id - c0) >> 5], 1u << ((id - c0) & 31));
        }
    }
    if (pr.e >= (uint32_t)c0 && pr.e < (uint32_t)c1) {
        int h = pen_insert(t, pr.e, rp.hs_log2);
        t.delta[h] = pr.d;
        atomicOr(&t.bits[(pr.e - c0) >> 5], 1u << ((pr.e - c0) & 31));
    }
    __syncthreads();
}

__device__ __forceinline__ float pen_apply(float v, uint32_t cnt, float delta, const RowSource &a) {
    if (cnt) {
        if (a.do_rep) v = (v > 0.0f) ? v / a.rp : v * a.rp;
        if (a.do_fp) {
            float t = (float)cnt * a.freq;
            t = t + a.pres;
            v = v - t;
        }
    }
    return v - delta;  // exact identity when delta == 0
}

// One thread's chunk share: NV vectors of VEC elements, transformed to the
// penalized f32 values the reference samples from.
template <typename T, int NV>
struct ChunkRegs {
    static constexpr int VEC = VecTraits<T>::VEC;
    static constexpr int N = NV * VEC;
    float x[N];
};

template <typename T, int NV>
__device__ __forceinline__ void chunk_load(const RowSource &a, int row, int c0, int c1, uint4 (&raw)[NV],
                                           uint32_t (&mw)[NV]) {
    constexpr int VEC = VecTraits<T>::VEC;
    const int tid = threadIdx.x;
    const T *base = reinterpret_cast<const T *>(a.logits) + (int64_t)row * a.ld;
    const uint32_t *mrow = a.mask ? a.mask + (int64_t)row * a.mask_ld : nullptr;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        int e0 = c0 + (j * kThreads + tid) * VEC;
        if (e0 < c1) {
            raw[j] = *reinterpret_cast<const uint4 *>(base + e0);
            mw[j] = mrow ? mrow[e0 >> 5] : 0xFFFFFFFFu;
        } else {
            raw[j] = make_uint4(0u, 0u, 0u, 0u);
            mw[j] = 0u;
        }
    }
}

// Unpacks, applies mask / penalty / edits and returns the thread max over its
// valid elements (-inf if none; NaNs never win fmaxf).
template <typename T, int NV>
__device__ __forceinline__ float chunk_transform(const RowSource &a, const PenTable &t, const RowPen &rp, int c0,
                                                 int c1, const uint4 (&raw)[NV], const uint32_t (&mw)[NV],
                                                 ChunkRegs<T, NV> &cr) {
    constexpr int VEC = VecTraits<T>::VEC;
    const int tid = threadIdx.x;
    float tmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        int e0 = c0 + (j * kThreads + tid) * VEC;
        float v[VEC];
        unpack<T>(raw[j], v);
        uint32_t mbits = (mw[j] >> (e0 & 31)) & ((1u << VEC) - 1u);
        uint32_t pbits = 0u;
        if (rp.any && e0 < c1) pbits = (t.bits[(e0 - c0) >> 5] >> ((e0 - c0) & 31)) & ((1u << VEC) - 1u);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            float x = v[e];
            if (!((mbits >> e) & 1u)) x = -INFINITY;
            if ((pbits >> e) & 1u) {
                int h = pen_find(t, (uint32_t)(e0 + e), rp.hs_log2);
                x = pen_apply(x, t.cnt[h], t.delta[h], a);
            }
            bool valid = e0 + e < c1;
            cr.x[j * VEC + e] = x;
            if (valid) tmax = fmaxf(tmax, x);
        }
    }
    return tmax;
}

// Stage A: publish a superset of this chunk's top-k (value desc, id asc) to
// the LDS candidate list.  Threshold: each wave finds the ceil(k/4)-th largest
// of its lanes' maxima; the minimum over the 4 waves is <= the chunk's k-th
// largest element (each wave owns ceil(k/4) distinct elements at or above
// it), so every element of the chunk's top-k passes.  Returns the number of
// candidates found (which may exceed cap; then the list is incomplete).
template <typename T, int NV>
__device__ __forceinline__ int chunk_candidates(const ChunkRegs<T, NV> &cr, float tmax, int c0, int c1, int k,
                                                uint64_t *s_key, float *s_val, int cap, int *s_nc,
                                                uint32_t *s_tau) {
    constexpr int VEC = VecTraits<T>::VEC;
    const int tid = threadIdx.x;
    const int wid = tid >> 6;
    bool present = c0 + tid * VEC < c1;
    uint32_t mkey = present ? okey(tmax) : 0u;
    int r = (k + kWaves - 1) / kWaves;
    uint32_t tw = wave_kth_largest(mkey, r);
    if ((tid & 63) == 0) s_tau[wid] = tw;
    if (tid == 0) *s_nc = 0;
    __syncthreads();
    uint32_t tau = s_tau[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) tau = min(tau, s_tau[w]);
    float tau_f = (tau > kNegInfKey) ? okey_inv(tau) : -INFINITY;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        int e0 = c0 + (j * kThreads + tid) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            float x = cr.x[j * VEC + e];
            if (e0 + e < c1 && x >= tau_f) {
                int pos = atomicAdd(s_nc, 1);
                if (pos < cap) {
                    s_key[pos] = ckey(x, (uint32_t)(e0 + e));
                    s_val[pos] = x;
                }
            }
        }
    }
    __syncthreads();
    return *s_nc;
}

// Wave 0 helper: given 256 histogram bins, find digit d (scanning from 255
// down) with sum_{b>d} < rem <= sum_{b>=d}; writes d and sum_{b>d} to out[0..1].
__device__ __forceinline__ void find_digit(const uint32_t *bins, int rem, int *out) {
    const int lane = threadIdx.x & 63;
    uint32_t c[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) c[q] = bins[255 - 4 * lane - q];
    uint32_t s = c[0] + c[1] + c[2] + c[3];
    uint32_t incl = s;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        uint32_t o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
    }
    uint32_t before = incl - s;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if ((int)before < rem && rem <= (int)(before + c[q])) {
            out[0] = 255 - 4 * lane - q;
            out[1] = (int)before;
        }
        before += c[q];
    }
}

// Block radix select over unique 64-bit keys: returns T such that exactly
// `need` of the keys are >= T.  `src(prefix, shift, bins)` must add, for each
// key it owns whose bits above shift+8 equal prefix's, one to
// bins[(key >> shift) & 255].  Requires need >= 1 and at least `need` keys.
template <class Src>
__device__ __forceinline__ uint64_t block_select(Src src, int need, uint32_t *bins, int *s_dig) {
    const int tid = threadIdx.x;
    uint64_t prefix = 0;
    int rem = need;
    for (int shift = 56;; shift -= 8) {
        bins[tid] = 0u;
        __syncthreads();
        src(prefix, shift, bins);
        __syncthreads();
        if (tid < 64) find_digit(bins, rem, s_dig);
        __syncthreads();
        int d = s_dig[0];
        int greater = s_dig[1];
        int inbin = (int)bins[d];
        __syncthreads();
        prefix |= (uint64_t)d << shift;
        rem -= greater;
        if (inbin == rem || shift == 0) return prefix;
    }
}

struct LdsKeySrc {
    const uint64_t *keys;
    int n;
    __device__ void operator()(uint64_t prefix, int shift, uint32_t *bins) const {
        for (int i = threadIdx.x; i < n; i += kThreads) {
            uint64_t k = keys[i];
            bool match = (shift == 56) || ((k >> (shift + 8)) == (prefix >> (shift + 8)));
            if (match) atomicAdd(&bins[(k >> shift) & 255u], 1u);
        }
    }
};

template <typename T, int NV>
struct RegKeySrc {
    const ChunkRegs<T, NV> *cr;
    int c0, c1;
    __device__ void operator()(uint64_t prefix, int shift, uint32_t *bins) const {
        constexpr int VEC = VecTraits<T>::VEC;
        const int tid = threadIdx.x;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            int e0 = c0 + (j * kThreads + tid) * VEC;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                float x = cr->x[j * VEC + e];
                if (e0 + e < c1 && x == x) {
                    uint64_t k = ckey(x, (uint32_t)(e0 + e));
                    bool match = (shift == 56) || ((k >> (shift + 8)) == (prefix >> (shift + 8)));
                    if (match) atomicAdd(&bins[(k >> shift) & 255u], 1u);
                }
            }
        }
    }
};

// Overflow path of stage A: the chunk had more than `cap` candidates.  Select
// exactly min(k, valid) of them by radix select over the registers and
// rebuild the LDS list.  Rare (needs many equal or clustered values).
template <typename T, int NV>
__device__ __forceinline__ int chunk_candidates_exact(const ChunkRegs<T, NV> &cr, int c0, int c1, int k,
                                                      uint64_t *s_key, float *s_val, int *s_nc, uint32_t *bins,
                                                      int *s_dig) {
    constexpr int VEC = VecTraits<T>::VEC;
    const int tid = threadIdx.x;
    RegKeySrc<T, NV> src{&cr, c0, c1};
    uint64_t T0 = block_select(src, k, bins, s_dig);
    if (tid == 0) *s_nc = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        int e0 = c0 + (j * kThreads + tid) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            float x = cr.x[j * VEC + e];
            if (e0 + e < c1 && x == x) {
                uint64_t key = ckey(x, (uint32_t)(e0 + e));
                if (key >= T0) {
                    int pos = atomicAdd(s_nc, 1);
                    if (pos < kCapA) {
                        s_key[pos] = key;
                        s_val[pos] = x;
                    }
                }
            }
        }
    }
    __syncthreads();
    return min(*s_nc, kCapA);
}

// Publishes the chunk's candidates, then takes a ticket; returns true in the
// last workgroup of the row (which then owns the row's merge).  The last
// workgroup re-arms the ticket for the next launch.
__device__ __forceinline__ bool publish_and_ticket(const uint64_t *s_key, const float *s_val, int nc,
                                                   uint64_t *g_key, float *g_val, int32_t *g_cnt, int32_t *tickets,
                                                   int row, int g, int G, int *s_flag) {
    const int tid = threadIdx.x;
    uint64_t *dk = g_key + ((int64_t)row * G + g) * kCapA;
    float *dv = g_val + ((int64_t)row * G + g) * kCapA;
    for (int i = tid; i < nc; i += kThreads) {
        dk[i] = s_key[i];
        dv[i] = s_val[i];
    }
    if (tid == 0) g_cnt[row * G + g] = nc;
    __threadfence();
    __syncthreads();
    if (tid == 0) *s_flag = (atomicAdd(&tickets[row], 1) == G - 1);
    __syncthreads();
    bool last = *s_flag != 0;
    if (last) {
        __threadfence();
        if (tid == 0) tickets[row] = 0;
    }
    return last;
}

// Stage B gather: loads all published candidates of `row` into LDS and returns
// their number (<= G * kCapA).
__device__ __forceinline__ int gather_candidates(const uint64_t *g_key, const float *g_val, const int32_t *g_cnt,
                                                 int row, int G, uint64_t *b_key, float *b_val, int *s_off) {
    const int tid = threadIdx.x;
    if (tid == 0) {
        int o = 0;
        for (int g = 0; g < G; ++g) {
            s_off[g] = o;
            o += __hip_atomic_load(&g_cnt[row * G + g], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        s_off[G] = o;
    }
    __syncthreads();
    for (int g = 0; g < G; ++g) {
        int o = s_off[g], n = s_off[g + 1] - o;
        const uint64_t *sk = g_key + ((int64_t)row * G + g) * kCapA;
        const float *sv = g_val + ((int64_t)row * G + g) * kCapA;
        for (int i = tid; i < n; i += kThreads) {
            b_key[o + i] = sk[i];
            b_val[o + i] = sv[i];
        }
    }
    int N = s_off[G];
    __syncthreads();
    return N;
}

// Stage B: reduce N unique candidates to the top `need` sorted by key desc
// into o_key/o_val[0..need).  need <= 256 and need <= N.
__device__ __forceinline__ void select_sorted(const uint64_t *b_key, const float *b_val, int N, int need,
                                              uint64_t *o_key, float *o_val, uint64_t *t_key, float *t_val,
                                              uint32_t *bins, int *s_dig, int *s_cnt) {
    const int tid = threadIdx.x;
    const uint64_t *ck = b_key;
    const float *cv = b_val;
    if (N > need) {
        LdsKeySrc src{b_key, N};
        uint64_t T0 = block_select(src, need, bins, s_dig);
        if (tid == 0) *s_cnt = 0;
        __syncthreads();
        for (int i = tid; i < N; i += kThreads) {
            uint64_t k = b_key[i];
            if (k >= T0) {
                int pos = atomicAdd(s_cnt, 1);
                if (pos < kThreads) {
                    t_key[pos] = k;
                    t_val[pos] = b_val[i];
                }
            }
        }
        __syncthreads();
        ck = t_key;
        cv = t_val;
    }
    // rank sort: rank = number of keys greater (keys are unique)
    uint64_t mine = 0;
    float mv = 0.0f;
    int rank = 0;
    if (tid < need) {
        mine = ck[tid];
        mv = cv[tid];
        for (int j = 0; j < need; ++j) rank += (ck[j] > mine) ? 1 : 0;
    }
    __syncthreads();
    if (tid < need) {
        o_key[rank] = mine;
        o_val[rank] = mv;
    }
    __syncthreads();
}

}  // namespace zi
