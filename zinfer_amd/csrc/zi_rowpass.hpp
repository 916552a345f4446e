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
//
// Hot-loop design: every load is issued unconditionally (addresses clamped
// into the chunk) so the compiler waits per load and the transform overlaps
// the stream; lanes past the chunk end become NaN (never selected, ignored by
// fmaxf); penalized ids are rare, so they are pulled out of the stream into an
// LDS side list and penalized after it.
#pragma once
#include "zi_common.hpp"
#include "zi_launch.hpp"

namespace zi {

constexpr int kMaxCH = kMaxChunkElems;  // max chunk elements (256 threads x 64)
constexpr int kHashMax = 2048;          // LDS hash slots (window + edits <= 1152 ids)
constexpr int kMaxWin = kMaxWinHost;    // max penalty window
constexpr int kMaxEdits = kMaxEditsHost;
constexpr int kCapA = kCapAHost;        // published candidates per chunk (>= top-k)
constexpr int kMaxG = kMaxGHost;        // max chunks per row (V <= 262144)
constexpr int kWaveCap = 256;           // stage-A candidates one wave may hold
constexpr int kFlagMax = kMaxWin + kMaxEdits;
static_assert(kThreads == kThreadsHost, "workgroup size");

// ------------------------------------------------ cross-workgroup handoff
// Chunk results travel through device scratch with agent-scope relaxed
// atomics (sc1: coherent across the XCDs' L2s) and one vmcnt(0) wait before
// the row ticket, instead of whole-L2 writeback / invalidate fences.
template <class T>
__device__ __forceinline__ void st_agent(T *p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <class T>
__device__ __forceinline__ T ld_agent(const T *p) {
    return __hip_atomic_load(const_cast<T *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// Returns true in exactly one workgroup of the row (the last to finish);
// every thread's agent-scope stores are performed before the ticket moves.
// The last workgroup re-arms the ticket for the next launch.
__device__ __forceinline__ bool row_ticket(int32_t *tickets, int row, int G, int *s_flag) {
    wait_vmem();
    __syncthreads();
    if (threadIdx.x == 0) {
        int old = __hip_atomic_fetch_add(&tickets[row], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bool last = old == G - 1;
        if (last) st_agent(&tickets[row], 0);
        *s_flag = last;
    }
    __syncthreads();
    return *s_flag != 0;
}

// --------------------------------------------------------- penalty table
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
    const int nbw = (c1 - c0 + 31) >> 5;
    for (int i = tid; i < nbw; i += kThreads) t.bits[i] = 0u;
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

// ------------------------------------------------------------ the stream
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Logits are read exactly once: non-temporal loads keep them from displacing
// anything useful in the caches.
__device__ __forceinline__ uint4 ld_stream(const uint4 *p) {
    u32x4 t = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}

template <typename T, int NV>
struct ChunkRegs {
    static constexpr int VEC = VecTraits<T>::VEC;
    float x[NV * VEC];
    float m4[NV];  // per-vector maxima (NaN lanes ignored)
    float m1;      // lane max (first occurrence), its id, and the lane's
    uint32_t id1;  // second largest value (multiset), all kept as loads land
    float m2;
};

struct FlagList {  // penalized / edited elements diverted from the stream
    uint32_t id[kFlagMax];
    float x[kFlagMax];
    int n;
};

// Streams the chunk [c0, c1) of `row` into registers with the mask applied
// and penalized ids diverted into `fl` (their register copies become NaN).
// Returns the thread max (-inf if the thread holds no selectable value);
// hook(j, v, max) sees each transformed vector as soon as its load lands.
// HAS_PEN needs PenTable `t` and FlagList `fl` in LDS and contains barriers.
struct NoHook {
    template <int VEC>
    __device__ void operator()(int, const float (&)[VEC], float) const {}
};

template <typename T, int NV, bool HAS_MASK, bool HAS_PEN, class Hook = NoHook>
__device__ __forceinline__ float chunk_stream(const RowSource &a, int row, int c0, int c1, ChunkRegs<T, NV> &cr,
                                              PenTable *t, FlagList *fl, const RowPen &rp, Hook hook = Hook()) {
    constexpr int VEC = VecTraits<T>::VEC;
    const int tid = threadIdx.x;
    const int nvec = (c1 - c0 + VEC - 1) / VEC;
    const T *base = reinterpret_cast<const T *>(a.logits) + (int64_t)row * a.ld + c0;
    const uint32_t *mrow = HAS_MASK ? a.mask + (int64_t)row * a.mask_ld : nullptr;

    PenRegs pr;
    if (HAS_PEN) pen_fetch(rp, pr);  // issued first: waiting for these does not wait for the row
    uint4 raw[NV];
    uint32_t mw[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        int q = min(j * kThreads + tid, nvec - 1);
        raw[j] = ld_stream(reinterpret_cast<const uint4 *>(base + q * VEC));
        if (HAS_MASK) mw[j] = mrow[(c0 + q * VEC) >> 5];
    }
    uint32_t pw[NV];
    if (HAS_PEN) {
        if (tid == 0) fl->n = 0;
        pen_build(*t, rp, pr, c0, c1);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            int q = min(j * kThreads + tid, nvec - 1);
            pw[j] = t->bits[(q * VEC) >> 5];
        }
    }
    float tmax = -INFINITY;
    cr.m1 = -INFINITY;
    cr.m2 = -INFINITY;
    cr.id1 = 0xFFFFFFFFu;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int q = j * kThreads + tid;
        const int id0 = c0 + q * VEC;
        float v[VEC];
        unpack<T>(raw[j], v);
        if (HAS_MASK) {
            uint32_t mb = mw[j] >> (id0 & 31);
#pragma unroll
            for (int e = 0; e < VEC; ++e) v[e] = ((mb >> e) & 1u) ? v[e] : -INFINITY;
        }
        if (HAS_PEN) {
            uint32_t pb = (pw[j] >> ((q * VEC) & 31)) & ((1u << VEC) - 1u);
            if (pb && id0 < c1) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    if ((pb >> e) & 1u) {
                        int s = atomicAdd(&fl->n, 1);
                        fl->id[s] = (uint32_t)(id0 + e);
                        fl->x[s] = v[e];
                        v[e] = __builtin_nanf("");
                    }
                }
            }
        }
        const int lim = c1 - id0;
        if (lim < VEC) {
#pragma unroll
            for (int e = 0; e < VEC; ++e)
                if (e >= lim) v[e] = __builtin_nanf("");
        }
        float m = v[0];
#pragma unroll
        for (int e = 1; e < VEC; ++e) m = fmaxf(m, v[e]);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            cr.x[j * VEC + e] = v[e];
            const bool gt = v[e] > cr.m1;  // strict: the first (lowest id) maximum stays
            cr.m2 = gt ? cr.m1 : fmaxf(cr.m2, v[e]);
            cr.id1 = gt ? (uint32_t)(id0 + e) : cr.id1;
            cr.m1 = gt ? v[e] : cr.m1;
        }
        cr.m4[j] = m;
        tmax = fmaxf(tmax, m);
        hook.template operator()<VEC>(j, v, m);
    }
    return tmax;
}

// Penalized value of diverted entry i (call after a barrier that follows
// chunk_stream).
__device__ __forceinline__ float flag_value(const RowSource &a, const PenTable &t, const FlagList &fl,
                                            const RowPen &rp, int i, uint32_t &id) {
    id = fl.id[i];
    int h = pen_find(t, id, rp.hs_log2);
    return pen_apply(fl.x[i], t.cnt[h], t.delta[h], a);
}

// --------------------------------------------------------- stage A select
// Candidate threshold: each wave takes the ceil(k/4)-th largest of its lanes'
// maxima; the minimum over the 4 waves is <= the k-th largest value the
// stream kept (each wave owns ceil(k/4) distinct values at or above it), so
// every element of the chunk's top-k that the stream kept passes, and every
// diverted (penalized) element above it is added separately.  Returns tau
// (-inf when some wave has too few values).
__device__ __forceinline__ float chunk_tau(float tmax, int k, uint32_t *s_tau) {
    const int tid = threadIdx.x;
    uint32_t mkey = (tmax == tmax) ? okey(tmax) : 0u;
    int r = (k + kWaves - 1) / kWaves;
    uint32_t tw = wave_kth_largest(mkey, r);
    if ((tid & 63) == 0) s_tau[tid >> 6] = tw;
    __syncthreads();
    uint32_t tau = s_tau[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) tau = min(tau, s_tau[w]);
    return (tau > kNegInfKey) ? okey_inv(tau) : -INFINITY;
}

// Appends this thread's elements >= tau to its wave's LDS region (keys/vals,
// capacity wcap) by ballot compaction (no atomics); returns the wave's count,
// which may exceed wcap (entries past it are dropped).  A lane whose second
// largest value is below tau holds at most one candidate, its maximum, which
// the stream already located; only lanes with two or more candidates scan
// their vectors.
template <typename T, int NV>
__device__ __forceinline__ int chunk_extract(const ChunkRegs<T, NV> &cr, int c0, float tau, uint64_t *keys,
                                             float *vals, int wcap) {
    constexpr int VEC = VecTraits<T>::VEC;
    const int tid = threadIdx.x;
    const bool multi = cr.m2 >= tau;
    const bool one = !multi && cr.m1 >= tau;
    int cnt = 0;
    {
        const uint64_t m = ballot(one);
        const int pos = lanes_below(m);
        if (one && pos < wcap) {
            keys[pos] = ckey(cr.m1, cr.id1);
            vals[pos] = cr.m1;
        }
        cnt = __popcll(m);
    }
    if (ballot(multi)) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            if (ballot(multi && cr.m4[j] >= tau)) {
                const int id0 = c0 + (j * kThreads + tid) * VEC;
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    const float x = cr.x[j * VEC + e];
                    const bool p = multi && x >= tau;
                    const uint64_t m = ballot(p);
                    if (m) {
                        const int pos = cnt + lanes_below(m);
                        if (p && pos < wcap) {
                            keys[pos] = ckey(x, (uint32_t)(id0 + e));
                            vals[pos] = x;
                        }
                        cnt += __popcll(m);
                    }
                }
            }
        }
    }
    return cnt;
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
// bins[(key >> shift) & 255].  Requires 1 <= need <= number of keys.
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

__device__ __forceinline__ void hist_add(uint64_t k, uint64_t prefix, int shift, uint32_t *bins) {
    bool match = (shift == 56) || ((k >> (shift + 8)) == (prefix >> (shift + 8)));
    if (match) atomicAdd(&bins[(k >> shift) & 255u], 1u);
}

struct LdsKeySrc {
    const uint64_t *keys;
    int n;
    __device__ void operator()(uint64_t prefix, int shift, uint32_t *bins) const {
        for (int i = threadIdx.x; i < n; i += kThreads) hist_add(keys[i], prefix, shift, bins);
    }
};

template <typename T, int NV>
struct RegKeySrc {
    const ChunkRegs<T, NV> *cr;
    int c0;
    const uint64_t *extra;  // diverted (penalized) entries
    int n_extra;
    __device__ void operator()(uint64_t prefix, int shift, uint32_t *bins) const {
        constexpr int VEC = VecTraits<T>::VEC;
        const int tid = threadIdx.x;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            int e0 = c0 + (j * kThreads + tid) * VEC;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                float x = cr->x[j * VEC + e];
                if (x == x) hist_add(ckey(x, (uint32_t)(e0 + e)), prefix, shift, bins);
            }
        }
        for (int i = tid; i < n_extra; i += kThreads) hist_add(extra[i], prefix, shift, bins);
    }
};

// Writes the keys (unique) of keys/vals[0..n) ranked by key descending to
// okeys/ovals[rank] for rank < need.  One key per thread per round; the
// comparisons read 16 keys per LDS round trip.
__device__ __forceinline__ void rank_sort(const uint64_t *keys, const float *vals, int n, int need, uint64_t *okeys,
                                          float *ovals) {
    for (int i = threadIdx.x; i < n; i += kThreads) {
        const uint64_t mine = keys[i];
        int rank = 0;
        int j = 0;
        for (; j + 16 <= n; j += 16) {
            uint64_t b[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) b[u] = keys[j + u];
#pragma unroll
            for (int u = 0; u < 16; ++u) rank += (int)(b[u] > mine);
        }
        for (; j < n; ++j) rank += (int)(keys[j] > mine);
        if (rank < need) {
            okeys[rank] = mine;
            ovals[rank] = vals[i];
        }
    }
}

// ------------------------------------------------------ stage A, complete
// Scratch layout per (row, chunk): kCapA keys, kCapA values, one count.
struct ChunkOut {
    uint64_t *key;
    float *val;
    int32_t *cnt;
};

template <typename T, int NV>
struct SelectLds {
    uint64_t wkey[kWaves][kWaveCap];  // wave-private candidate regions
    float wval[kWaves][kWaveCap];
    uint64_t ckey[kWaves * kWaveCap];  // gathered candidates
    float cval[kWaves * kWaveCap];
    uint64_t skey[kCapA];  // sorted top-k
    float sval[kCapA];
};

// Stage A after chunk_stream: find the chunk's exact top-min(k, selectable)
// sorted by (value desc, id asc), publish it to `out` (agent-scope stores).
// LDS: `sl` (SelectLds), `t`/`fl` when HAS_PEN, small scalars.
template <typename T, int NV, bool HAS_PEN>
__device__ __forceinline__ void chunk_select_publish(const RowSource &a, const RowPen &rp, ChunkRegs<T, NV> &cr,
                                                     float tmax, int c0, int k, SelectLds<T, NV> &sl,
                                                     PenTable *t, FlagList *fl, uint32_t *s_tau, int *s_wcnt,
                                                     int *s_n, uint32_t *bins, int *s_dig, ChunkOut out) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const float tau = chunk_tau(tmax, k, s_tau);  // contains a barrier (fl->n final after it)
    int wc = chunk_extract<T, NV>(cr, c0, tau, sl.wkey[wid], sl.wval[wid], kWaveCap);
    if (lane == 0) s_wcnt[wid] = wc;
    int nf = 0;
    if (HAS_PEN) nf = fl->n;
    __syncthreads();
    int off[kWaves + 1];
    off[0] = 0;
    bool overflow = false;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        overflow |= s_wcnt[w] > kWaveCap;
        off[w + 1] = off[w] + min(s_wcnt[w], kWaveCap);
    }
    int n = off[kWaves];
    // gather the wave regions contiguously, then the diverted entries >= tau
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
        for (int i = tid; i < off[w + 1] - off[w]; i += kThreads) {
            sl.ckey[off[w] + i] = sl.wkey[w][i];
            sl.cval[off[w] + i] = sl.wval[w][i];
        }
    if (HAS_PEN) {
        if (tid == 0) *s_n = n;
        __syncthreads();
        for (int i = tid; i < nf; i += kThreads) {
            uint32_t id;
            float v = flag_value(a, *t, *fl, rp, i, id);
            if (v >= tau) {
                int pos = atomicAdd(s_n, 1);
                if (pos < kWaves * kWaveCap) {
                    sl.ckey[pos] = ckey(v, id);
                    sl.cval[pos] = v;
                } else {
                    overflow = true;
                }
            }
        }
        __syncthreads();
        n = *s_n;
        if (n > kWaves * kWaveCap) overflow = true;
    }
    __syncthreads();
    overflow = __syncthreads_or(overflow);
    if (overflow) {
        // More candidates than the buffers hold (clustered or tied values):
        // exact radix select over registers + diverted entries, then rebuild.
        uint64_t *extra = sl.skey;  // reuse: penalized keys (<= kFlagMax fits in ckey)
        int ne = 0;
        if (HAS_PEN) {
            for (int i = tid; i < nf; i += kThreads) {
                uint32_t id;
                float v = flag_value(a, *t, *fl, rp, i, id);
                sl.ckey[i] = ckey(v, id);
                sl.cval[i] = v;
            }
            ne = nf;
            __syncthreads();
        }
        (void)extra;
        RegKeySrc<T, NV> src{&cr, c0, sl.ckey, ne};
        uint64_t T0 = block_select(src, k, bins, s_dig);
        if (tid == 0) *s_n = 0;
        __syncthreads();
        constexpr int VEC = VecTraits<T>::VEC;
        // penalized entries first (they sit in ckey[0..ne)); collect into skey
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            int e0 = c0 + (j * kThreads + tid) * VEC;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                float x = cr.x[j * VEC + e];
                if (x == x) {
                    uint64_t key = ckey(x, (uint32_t)(e0 + e));
                    if (key >= T0) {
                        int pos = atomicAdd(s_n, 1);
                        if (pos < kCapA) {
                            sl.skey[pos] = key;
                            sl.sval[pos] = x;
                        }
                    }
                }
            }
        }
        for (int i = tid; i < ne; i += kThreads) {
            if (sl.ckey[i] >= T0) {
                int pos = atomicAdd(s_n, 1);
                if (pos < kCapA) {
                    sl.skey[pos] = sl.ckey[i];
                    sl.sval[pos] = sl.cval[i];
                }
            }
        }
        __syncthreads();
        n = min(*s_n, kCapA);
        __syncthreads();
        for (int i = tid; i < n; i += kThreads) {
            sl.ckey[i] = sl.skey[i];
            sl.cval[i] = sl.sval[i];
        }
        __syncthreads();
    }
    const int m = min(n, k);
    rank_sort(sl.ckey, sl.cval, n, m, sl.skey, sl.sval);
    __syncthreads();
    for (int i = tid; i < m; i += kThreads) {
        st_agent(&out.key[i], sl.skey[i]);
        st_agent(&out.val[i], sl.sval[i]);
    }
    if (tid == 0) st_agent(out.cnt, m);
}

// ------------------------------------------------------------- stage B
// Loads the G sorted chunk lists of a row (one round trip: every slot is
// requested before any is used) and merges them: the rank of an entry is its
// index in its own list plus, for every other list, the number of entries
// greater than it (binary search, all lists in parallel).  Writes the row's
// top-min(k, total) to okey/oval sorted; returns that count.
struct MergeLds {
    uint64_t key[kMaxG][kCapA];
    float val[kMaxG][kCapA];
    int cnt[kMaxG];
};

__device__ __forceinline__ int row_merge(const uint64_t *g_key, const float *g_val, const int32_t *g_cnt, int row,
                                         int G, int k, MergeLds &ml, uint64_t *okey, float *oval) {
    const int tid = threadIdx.x;
    const int slots = G * k;
    const int64_t rb = (int64_t)row * G;
    // one round trip: every slot of every list is requested before any is used
    int cn = 0;
    if (tid < G) cn = ld_agent(&g_cnt[rb + tid]);
    for (int s0 = 0; s0 < slots; s0 += 4 * kThreads) {
        uint64_t kk[4];
        float vv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            int s = s0 + u * kThreads + tid;
            if (s < slots) {
                int g = s / k, i = s - g * k;
                kk[u] = ld_agent(&g_key[(rb + g) * kCapA + i]);
                vv[u] = ld_agent(&g_val[(rb + g) * kCapA + i]);
            }
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            int s = s0 + u * kThreads + tid;
            if (s < slots) {
                int g = s / k, i = s - g * k;
                ml.key[g][i] = kk[u];
                ml.val[g][i] = vv[u];
            }
        }
    }
    if (tid < G) ml.cnt[tid] = cn;
    __syncthreads();
    int total = 0;
    for (int g = 0; g < G; ++g) total += ml.cnt[g];
    const int need = min(k, total);
    int half = 1;
    while (half * 2 <= k) half *= 2;  // largest power of two <= k
    // rank of entry (g, i) = i + sum over other lists of the entries greater
    // than it, by branch-free power-of-two searches advanced for every list in
    // lock-step (their LDS reads are independent and issue together)
    for (int s = tid; s < slots; s += kThreads) {
        const int g = s / k, i = s - g * k;
        const bool live = i < ml.cnt[g];
        const uint64_t mine = ml.key[g][min(i, kCapA - 1)];
        int pos[kMaxG], len[kMaxG];
#pragma unroll
        for (int h = 0; h < kMaxG; ++h) {
            pos[h] = 0;
            len[h] = (h < G && h != g) ? ml.cnt[h] : 0;
        }
        for (int st = half; st > 0; st >>= 1) {
            uint64_t kv[kMaxG];
#pragma unroll
            for (int h = 0; h < kMaxG; ++h) kv[h] = ml.key[h][max(min(pos[h] + st, len[h]) - 1, 0)];
#pragma unroll
            for (int h = 0; h < kMaxG; ++h) pos[h] += (pos[h] + st <= len[h] && kv[h] > mine) ? st : 0;
        }
        int rank = i;
#pragma unroll
        for (int h = 0; h < kMaxG; ++h) rank += pos[h];
        if (live && rank < need) {
            okey[rank] = mine;
            oval[rank] = ml.val[g][i];
        }
    }
    __syncthreads();
    return need;
}

}  // namespace zi
