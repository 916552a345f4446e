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
// fmaxf).  Penalized ids are rare: the stream only turns them into NaN, and
// each distinct penalized id of the chunk has an owner thread that reloads its
// logit while the stream is in flight and penalizes it after the stream.
#pragma once
#include "zi_common.hpp"
#include "zi_launch.hpp"

namespace zi {

constexpr int kMaxCH = kMaxChunkElems;  // max chunk elements (512 threads x 64)
constexpr int kHashMax = 2048;          // LDS hash slots (window + edits <= 1152 ids)
constexpr int kMaxWin = kMaxWinHost;    // max penalty window
constexpr int kMaxEdits = kMaxEditsHost;
constexpr int kCapA = kCapAHost;        // published candidates per chunk (>= top-k)
constexpr int kMaxG = kMaxGHost;        // max chunks per row (V <= 262144)
constexpr int kWaveCap = 256;           // stage-A candidates one wave may hold
constexpr int kWinPerThread = kMaxWin / kThreads;
constexpr int kOwnSlots = kWinPerThread + 1;  // window ids + one edit per thread
static_assert(kThreads == kThreadsHost, "workgroup size");
static_assert(kMaxWin + kMaxEdits <= kThreads * 4, "penalized entries fit the candidate buffer");

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
//
// Why the last workgroup sees every other workgroup's list:
//  1. Producers write their lists with agent-scope stores (sc1), which are
//     performed at the device's coherence point, not only in the XCD's L2.
//  2. wait_vmem() is s_waitcnt vmcnt(0): on gfx950 vmcnt counts stores as
//     well as loads, and a store leaves the count only once it is performed
//     at the scope its cache bits ask for.  After it, this thread's stores are
//     performed.
//  3. __syncthreads() (a workgroup fence, so the compiler moves no memory
//     operation across it, and s_barrier) puts every thread's step 2 before
//     thread 0's ticket increment, an agent-scope atomic performed at the
//     coherence point.
//  4. The increments of one row are totally ordered at that point: the
//     workgroup that reads G - 1 comes after the other G - 1 increments,
//     each of which came after its workgroup's stores.
//  5. The consumer reads the lists with agent-scope loads (sc1: they miss in
//     its own L2 rather than hit a stale line) issued after the ticket's
//     result, through *s_flag and a barrier, so none is issued early.
// The re-armed ticket (0) is read by the next launch only, after the kernel
// boundary.
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

// The final-logit softcap of logit `id` (src/model.zig:2492-2513): the vector
// body below cap_body, the scalar tail from there on.
__device__ __forceinline__ float softcap_at(const RowSource &a, int id, float v) {
    return id < a.cap_body ? softcap_f(v, a.cap, a.inv_cap) : softcap_tail_f(v, a.cap);
}
// The softcap of the vector [id0, id0 + VEC): the scalar tail (and its f64
// tanh) only in the one vector that reaches the row's last ids, behind a
// branch, so that the per-element code stays small enough to unroll (and the
// chunk's registers stay registers).
template <int VEC>
struct FVec {
    float x[VEC];
};
// Out of line (by value, so no array's address escapes the caller).
template <int VEC>
__device__ __attribute__((noinline)) FVec<VEC> softcap_vec_tail(FVec<VEC> v, int id0, int cap_body, float cap,
                                                                 float inv_cap) {
#pragma unroll
    for (int e = 0; e < VEC; ++e)
        v.x[e] = id0 + e < cap_body ? softcap_f(v.x[e], cap, inv_cap) : softcap_tail_f(v.x[e], cap);
    return v;
}
template <int VEC>
__device__ __forceinline__ void softcap_vec(const RowSource &a, int id0, float (&v)[VEC]) {
    if (id0 + VEC <= a.cap_body) {
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = softcap_f(v[e], a.cap, a.inv_cap);
    } else {
        FVec<VEC> t;
#pragma unroll
        for (int e = 0; e < VEC; ++e) t.x[e] = v[e];
        t = softcap_vec_tail<VEC>(t, id0, a.cap_body, a.cap, a.inv_cap);
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = t.x[e];
    }
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

template <class Table>  // PenTable or any table with the same key array
__device__ __forceinline__ int pen_insert(Table &t, uint32_t id, int hs_log2) {
    uint32_t h = hash_slot(id, hs_log2);
    const uint32_t m = (1u << hs_log2) - 1;
    for (;;) {
        const uint32_t prev = atomicCAS(&t.key[h], 0u, id + 1);
        if (prev == 0u || prev == id + 1) return (int)h;
        h = (h + 1) & m;
    }
}

// Per-row window bounds: the last min(hist_len, win) entries of hist.
struct RowPen {
    const uint32_t *win_ptr;  // hist[row] + hl - nw
    int hl;                   // history length (clamped to hist_ld)
    int nw;
    const uint32_t *eid;
    const float *edl;
    int ne;
    int hs_log2;
    bool any;
};

// hl_raw / ne_raw: hist_len[row] / edit_count[row] as loaded (callers that
// issue those loads early pass them in; row_pen loads them itself).
__device__ __forceinline__ bool row_pen_window_on(const RowSource &a) {
    return a.hist && (a.do_rep || a.do_fp) && a.win > 0;
}

__device__ __forceinline__ RowPen row_pen_from(const RowSource &a, int row, int hl_raw, int ne_raw) {
    RowPen r;
    r.nw = 0;
    r.hl = 0;
    r.win_ptr = nullptr;
    if (row_pen_window_on(a)) {
        int hl = hl_raw;
        hl = hl < 0 ? 0 : (hl > a.hist_ld ? a.hist_ld : hl);
        r.hl = hl;
        r.nw = hl < a.win ? hl : a.win;
        r.win_ptr = a.hist + (int64_t)row * a.hist_ld + (hl - r.nw);
    }
    r.ne = 0;
    r.eid = nullptr;
    r.edl = nullptr;
    if (a.edit_ids) {
        int ne = ne_raw;
        r.ne = ne < 0 ? 0 : (ne > a.edit_ld ? a.edit_ld : ne);
        r.ne = r.ne > kMaxEdits ? kMaxEdits : r.ne;
        r.eid = a.edit_ids + (int64_t)row * a.edit_ld;
        r.edl = a.edit_delta + (int64_t)row * a.edit_ld;
    }
    const int n = r.nw + r.ne;  // hash of >= 2n slots, 64 .. 2048 (no loop: keeps the load waits exact)
    r.hs_log2 = n > 0 ? min(11, max(6, 32 - __clz(2 * n - 1))) : 6;
    r.any = n > 0;
    return r;
}

__device__ __forceinline__ RowPen row_pen(const RowSource &a, int row) {
    return row_pen_from(a, row, row_pen_window_on(a) ? a.hist_len[row] : 0, a.edit_ids ? a.edit_count[row] : 0);
}

struct PenRegs {
    uint32_t w[kWinPerThread];
    uint32_t e;
    float d;
};

// Penalty inputs, issued before the row's loads so that waiting for them
// never waits for the row: the whole history row (hist_ld <= kMaxWin: lane
// slot i = tid + u*kThreads holds hist[row][i]; the host compacts longer rows
// to their windows first) and the first kMaxEdits edits, none of which needs
// hist_len / edit_count.
__device__ __forceinline__ void pen_prefetch(const RowSource &a, int row, PenRegs &pr) {
    const int tid = threadIdx.x;
    const bool on = a.hist && (a.do_rep || a.do_fp) && a.win > 0;
    const uint32_t *h = a.hist + (int64_t)row * a.hist_ld;
#pragma unroll
    for (int u = 0; u < kWinPerThread; ++u) {
        const int i = tid + u * kThreads;
        pr.w[u] = (on && i < a.hist_ld) ? h[i] : 0xFFFFFFFFu;
    }
    const bool ed = a.edit_ids && tid < min(a.edit_ld, kMaxEdits);
    pr.e = ed ? a.edit_ids[(int64_t)row * a.edit_ld + tid] : 0xFFFFFFFFu;
    pr.d = ed ? a.edit_delta[(int64_t)row * a.edit_ld + tid] : 0.0f;
}

// Restricts the prefetched inputs to the window [hl - nw, hl) and the edit count.
__device__ __forceinline__ void pen_window(const RowPen &rp, PenRegs &pr) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int u = 0; u < kWinPerThread; ++u) {
        const int i = tid + u * kThreads;
        pr.w[u] = (i >= rp.hl - rp.nw && i < rp.hl) ? pr.w[u] : 0xFFFFFFFFu;
    }
    if (tid >= rp.ne) {
        pr.e = 0xFFFFFFFFu;
        pr.d = 0.0f;
    }
}

// The penalized ids this thread owns (first inserter of each distinct id of
// the chunk), their hash slots and their logits with the mask applied.
struct PenOwn {
    uint32_t id[kOwnSlots];  // 0xFFFFFFFF: none
    int slot[kOwnSlots];
    float x[kOwnSlots];
};

template <typename T>
__device__ __forceinline__ float load_logit(const T *row, uint32_t id);
template <>
__device__ __forceinline__ float load_logit<float>(const float *row, uint32_t id) {
    return row[id];
}
template <>
__device__ __forceinline__ float load_logit<uint16_t>(const uint16_t *row, uint32_t id) {
    return __uint_as_float((uint32_t)row[id] << 16);
}

// Clears the chunk's bitset and the whole hash (no dependence on the row's
// window size, so it runs while the row streams; the caller's next barrier
// orders it before the inserts).
__device__ __forceinline__ void pen_clear(PenTable &t, int c0, int c1) {
    const int tid = threadIdx.x;
    const int nbw = (c1 - c0 + 31) >> 5;
    for (int i = tid; i < nbw; i += kThreads) t.bits[i] = 0u;
    for (int i = tid; i < kHashMax; i += kThreads) {
        t.key[i] = 0u;
        t.cnt[i] = 0u;
        t.delta[i] = 0.0f;
    }
}

// Marks the chunk's penalized/edited ids in the bitset; the thread whose
// atomicOr set an id's bit owns that id and issues the reload of its logit
// (row = logits row, mrow = mask row or null).  CAP: the reloaded logit gets
// the final-logit softcap.  No barrier.
template <typename T, bool CAP>
__device__ __forceinline__ void pen_mark(const RowSource &a, PenTable &t, const PenRegs &pr, int c0, int c1, PenOwn &own, const T *row,
                                         const uint32_t *mrow) {
#pragma unroll
    for (int u = 0; u < kOwnSlots; ++u) {
        const uint32_t id = u < kWinPerThread ? pr.w[u] : pr.e;
        own.id[u] = 0xFFFFFFFFu;
        own.slot[u] = 0;
        own.x[u] = 0.0f;
        if (id >= (uint32_t)c0 && id < (uint32_t)c1) {
            const uint32_t b = 1u << ((id - c0) & 31);
            if (!(atomicOr(&t.bits[(id - c0) >> 5], b) & b)) own.id[u] = id;
        }
    }
#pragma unroll
    for (int u = 0; u < kOwnSlots; ++u) {
        if (own.id[u] != 0xFFFFFFFFu) {
            float v = load_logit<T>(row, own.id[u]);
            if constexpr (CAP) v = softcap_at(a, (int)own.id[u], v);
            if (mrow && !((mrow[own.id[u] >> 5] >> (own.id[u] & 31)) & 1u)) v = -INFINITY;
            own.x[u] = v;
        }
    }
}

// Fills the id -> (count, delta) hash and the owners' slots.  No barrier:
// owners read their entries after the caller's next barrier.
__device__ __forceinline__ void pen_count(PenTable &t, const RowPen &rp, const PenRegs &pr, int c0, int c1,
                                          PenOwn &own) {
#pragma unroll
    for (int u = 0; u < kWinPerThread; ++u) {
        const uint32_t id = pr.w[u];
        if (id >= (uint32_t)c0 && id < (uint32_t)c1) {
            const int h = pen_insert(t, id, rp.hs_log2);
            atomicAdd(&t.cnt[h], 1u);
            if (own.id[u] == id) own.slot[u] = h;
        }
    }
    if (pr.e >= (uint32_t)c0 && pr.e < (uint32_t)c1) {
        const int h = pen_insert(t, pr.e, rp.hs_log2);
        t.delta[h] = pr.d;
        if (own.id[kWinPerThread] == pr.e) own.slot[kWinPerThread] = h;
    }
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
    float m4[NV];  // per-vector maxima (NaN lanes ignored; NaN if the vector holds no value)
    float lmax;    // lane maximum (-inf if the lane holds no value)
};

// Streams the chunk [c0, c1) of `row` into registers with the mask applied;
// penalized ids become NaN in registers (their owners in `own` carry them).
// The penalty inputs are prefetched ahead of the row and the bitset of
// penalized ids is built while the row's loads are in flight; the count/delta
// hash is filled after the stream.  Returns the thread max (-inf if the thread
// holds no selectable value); hook(j, v, max) sees each transformed vector as
// soon as its load lands.  HAS_PEN needs PenTable `t` in LDS and contains
// barriers.
struct NoHook {
    template <int VEC>
    __device__ void operator()(int, const float (&)[VEC], float) const {}
};

struct NoMid {
    __device__ void operator()(float) const {}
};

// CAP: every value gets the final-logit softcap (a.cap > 0) right after it is
// unpacked; instances without it carry no softcap code.
// SPLIT < NV: after vector SPLIT-1 is processed, mid(partial lane max) runs
// (the penalty hash is filled just before it) while the remaining vectors'
// loads are still in flight; workgroup barriers inside mid order LDS only and
// do not wait for them.
// PF: the chunk's logit vectors were requested by the caller into pf[]
// (chunk_request); as each one is unpacked, its register is refilled with the
// same vector of the next chunk [n0, n1) (none when n0 >= n1), so that chunk's
// loads are in flight while the caller selects from this one.
template <typename T, int NV>
__device__ __forceinline__ void chunk_request(const RowSource &a, int row, int c0, int c1, uint4 (&pf)[NV]) {
    constexpr int VEC = VecTraits<T>::VEC;
    const int nvec = (c1 - c0 + VEC - 1) / VEC;
    const T *base = reinterpret_cast<const T *>(a.logits) + (int64_t)row * a.ld + c0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int q = min(j * kThreads + (int)threadIdx.x, nvec - 1);
        pf[j] = ld_stream(reinterpret_cast<const uint4 *>(base + q * VEC));
    }
}

template <typename T, int NV, bool HAS_MASK, bool HAS_PEN, bool CAP = false, class Hook = NoHook, int SPLIT = NV,
          class Mid = NoMid, bool PF = false>
__device__ __forceinline__ float chunk_stream(const RowSource &a, int row, int c0, int c1, ChunkRegs<T, NV> &cr,
                                              PenTable *t, PenOwn *own, Hook hook = Hook(), Mid mid = Mid(),
                                              uint4 *pf = nullptr, int n0 = 0, int n1 = 0) {
    constexpr int VEC = VecTraits<T>::VEC;
    const int tid = threadIdx.x;
    const int nvec = (c1 - c0 + VEC - 1) / VEC;
    const T *base = reinterpret_cast<const T *>(a.logits) + (int64_t)row * a.ld + c0;
    const uint32_t *mrow = HAS_MASK ? a.mask + (int64_t)row * a.mask_ld : nullptr;
    const int nvec_next = (n1 - n0 + VEC - 1) / VEC;
    const T *base_next = reinterpret_cast<const T *>(a.logits) + (int64_t)row * a.ld + n0;

    PenRegs pr;
    if (HAS_PEN) pen_prefetch(a, row, pr);
    // the row's loads depend on nothing that waits for memory
    uint4 raw_own[NV];
    uint4 *raw = PF ? pf : raw_own;
    uint32_t mw[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        int q = min(j * kThreads + tid, nvec - 1);
        if (!PF) raw[j] = ld_stream(reinterpret_cast<const uint4 *>(base + q * VEC));
        if (HAS_MASK) mw[j] = mrow[(c0 + q * VEC) >> 5];
    }
    uint32_t pw[NV];
    RowPen rp;
    if (HAS_PEN) {
        pen_clear(*t, c0, c1);
        rp = row_pen(a, row);
        pen_window(rp, pr);
        __syncthreads();  // tables cleared
        pen_mark<T, CAP>(a, *t, pr, c0, c1, *own, reinterpret_cast<const T *>(a.logits) + (int64_t)row * a.ld, mrow);
        __syncthreads();  // bitset complete
#pragma unroll
        for (int j = 0; j < NV; ++j) pw[j] = t->bits[(min(j * kThreads + tid, nvec - 1) * VEC) >> 5];
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int q = j * kThreads + tid;
        const int id0 = c0 + q * VEC;
        float v[VEC];
        unpack<T>(raw[j], v);
        if constexpr (PF) {
            if (n0 < n1) {  // uniform
                const int nq = min(j * kThreads + tid, nvec_next - 1);
                raw[j] = ld_stream(reinterpret_cast<const uint4 *>(base_next + nq * VEC));
            }
        }
        if constexpr (CAP) softcap_vec<VEC>(a, id0, v);
        if (HAS_MASK) {
            uint32_t mb = mw[j] >> (id0 & 31);
#pragma unroll
            for (int e = 0; e < VEC; ++e) v[e] = ((mb >> e) & 1u) ? v[e] : -INFINITY;
        }
        if (HAS_PEN) {
            const uint32_t pb = (pw[j] >> ((q * VEC) & 31)) & ((1u << VEC) - 1u);
            if (pb) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) v[e] = ((pb >> e) & 1u) ? __builtin_nanf("") : v[e];
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
        for (int e = 0; e < VEC; ++e) cr.x[j * VEC + e] = v[e];
        cr.m4[j] = m;
        tmax = fmaxf(tmax, m);
        hook.template operator()<VEC>(j, v, m);
        if (SPLIT < NV && j == SPLIT - 1) {
            if (HAS_PEN) pen_count(*t, rp, pr, c0, c1, *own);  // ordered by the barriers in mid
            mid(tmax);
        }
    }
    if (HAS_PEN && SPLIT >= NV) pen_count(*t, rp, pr, c0, c1, *own);  // read by owners after the caller's next barrier
    cr.lmax = tmax;
    return tmax;
}

// Penalized value of owned entry u (call after a barrier that follows
// chunk_stream).
__device__ __forceinline__ float owned_value(const RowSource &a, const PenTable &t, const PenOwn &own, int u) {
    const int h = own.slot[u];
    return pen_apply(own.x[u], t.cnt[h], t.delta[h], a);
}

// --------------------------------------------------------- stage A select
// Candidate threshold tau <= the chunk's k-th largest value, from the lane
// maxima (distinct elements of the chunk).  k <= kTauWaveMaxK: each wave
// sorts its 64 lane maxima and contributes its r largest, r = max(ceil(k/W),
// 64/W); the union holds W*r >= k elements, so its k-th largest is a lower
// bound of the chunk's k-th largest.  Larger k: every lane maximum enters the
// union, and wave 0 bisects the top 20 key bits for the largest T with at
// least k union keys >= T (valid for any k).  Lanes without a value
// contribute okey(-inf) (a bound at -inf admits everything).  Penalized
// elements diverted from the stream are not in the union, which only lowers
// the bound.  Contains two barriers.
//
// The per-wave union has 64 entries, so as k nears 64 its k-th largest falls
// to about the smallest of 8 per-wave 8th maxima and admits many candidates.
// Config-2 rows (64 x 128256 f32, penalties), us per call, per-wave against
// bisection: k = 40 16.4 / 17.5, k = 56 17.1 / 18.3, k = 58 17.4 / ~18.3,
// k = 60 19.0 / 18.3, k = 64 48.4 / 18.4.
constexpr int kTauWaveMaxK = 58;
constexpr int kMaxR = 64;  // union entries per wave

__device__ __forceinline__ float chunk_tau(float m1, int k, uint32_t *uni, uint32_t *s_tau) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const uint32_t mkey = (m1 == m1) ? okey(m1) : 0u;
    if (k <= kTauWaveMaxK) {
        const int r = max((k + kWaves - 1) / kWaves, 64 / kWaves);
        const uint32_t key = wave_sort_desc_u32(mkey);
        if (lane < r) uni[wid * r + lane] = key;
    } else {
        uni[tid] = mkey;
    }
    __syncthreads();
    if (wid == 0) {
        uint32_t t;
        if (k <= kTauWaveMaxK) {
            const int U = kWaves * max((k + kWaves - 1) / kWaves, 64 / kWaves);
            const uint32_t u = wave_sort_desc_u32(lane < U ? uni[lane] : 0u);
            t = (uint32_t)__builtin_amdgcn_readlane((int)u, k - 1);
        } else {
            uint32_t u8[kWaves];
#pragma unroll
            for (int c = 0; c < kWaves; ++c) u8[c] = uni[lane + 64 * c];
            t = 0;
            for (int b = 31; b >= 12; --b) {
                const uint32_t cand = t | (1u << b);
                int c = 0;
#pragma unroll
                for (int i = 0; i < kWaves; ++i) c += __popcll(ballot(u8[i] >= cand));
                if (c >= k) t = cand;
            }
            // keys below okey(-inf) with the low bits cleared decode to NaN;
            // no key lies in (0, okey(-inf)), so the count is unchanged
            if (t != 0u && t < kNegInfKey) t = kNegInfKey;
        }
        if (lane == 0) *s_tau = t;
    }
    __syncthreads();
    const uint32_t t = *s_tau;
    return t ? okey_inv(t) : -INFINITY;
}

// Stages every pair of register vectors whose maximum is >= tau into its
// wave's LDS region (2*VEC values + the first id of each vector), by ballot
// compaction over the NV/2 slots; returns the wave's count, which may exceed
// `cap` (pairs past it are dropped).  A pair with no value has a NaN maximum
// and is never staged.
template <typename T, int NV>
__device__ __forceinline__ int chunk_stage(const ChunkRegs<T, NV> &cr, int c0, float tau, float *sx, uint32_t *sid,
                                           int cap) {
    constexpr int VEC = VecTraits<T>::VEC;
    static_assert(NV % 2 == 0, "vectors are staged in pairs");
    const int tid = threadIdx.x;
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < NV; j += 2) {
        const bool p = fmaxf(cr.m4[j], cr.m4[j + 1]) >= tau;
        const uint64_t b = ballot(p);
        if (b) {
            const int pos = cnt + lanes_below(b);
            if (p && pos < cap) {
                float4 *dst = reinterpret_cast<float4 *>(sx + pos * 2 * VEC);
#pragma unroll
                for (int q = 0; q < VEC / 2; ++q)
                    dst[q] = make_float4(cr.x[j * VEC + 4 * q], cr.x[j * VEC + 4 * q + 1], cr.x[j * VEC + 4 * q + 2],
                                         cr.x[j * VEC + 4 * q + 3]);
                sid[2 * pos] = (uint32_t)(c0 + (j * kThreads + tid) * VEC);
                sid[2 * pos + 1] = (uint32_t)(c0 + ((j + 1) * kThreads + tid) * VEC);
            }
            cnt += __popcll(b);
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
        if (tid < 256) bins[tid] = 0u;
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

// ------------------------------------------------------ stage A, complete
// Scratch layout per (row, chunk): kCapA keys, kCapA values, one count.
struct ChunkOut {
    uint64_t *key;
    float *val;
    int32_t *cnt;
};

constexpr int kSortMax = 256;  // candidates ranked without the radix-select path
constexpr int kCandCap = kThreads * 4;
constexpr int kStageCap = 32;  // staged vector pairs per wave
constexpr int kWaveCand = 64;  // candidates per wave region

template <typename T, int NV>
struct SelectLds {
    static constexpr int VEC = VecTraits<T>::VEC;
    uint32_t uni[kWaves * kMaxR];  // threshold union (all lane maxima for k > kTauWaveMaxK)
    float sx[kWaves][kStageCap * 2 * VEC];  // staged vector pairs
    uint32_t sid[kWaves][kStageCap * 2];
    uint64_t wkey[kWaves][kWaveCand];  // candidates, one region per wave
    float wval[kWaves][kWaveCand];
    uint32_t part[kWaves][kSortMax];  // per-region rank counts
    uint64_t ckey[kCandCap];          // overflow path: penalized keys
    float cval[kCandCap];
    uint64_t skey[kCapA];  // overflow path: the exact top-k, unsorted
    float sval[kCapA];
    uint32_t rank[kSortMax];
    int wcnt[kWaves];
    int wge[kWaves];  // late penalties: candidates still >= tau, per wave
};

// This wave's candidates: the elements >= tau of its staged vector pairs and
// (HAS_PEN) of the penalized entries its lanes own, appended to the wave's
// region by ballot compaction.  Returns the count, which may exceed
// kWaveCand (entries past it are dropped); no barrier.
template <typename T, int NV, bool HAS_PEN>
__device__ __forceinline__ int wave_candidates(const RowSource &a, const ChunkRegs<T, NV> &cr, int c0, float tau,
                                               SelectLds<T, NV> &sl, const PenTable *t, const PenOwn *own) {
    constexpr int VEC = VecTraits<T>::VEC;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int ns = chunk_stage<T, NV>(cr, c0, tau, sl.sx[wid], sl.sid[wid], kStageCap);
    if (ns > kStageCap) return kWaveCand + 1;
    wave_sync();  // staged by other lanes of this wave
    uint64_t *wk = sl.wkey[wid];
    float *wv = sl.wval[wid];
    int cnt = 0;  // wave-uniform: every lane runs every iteration
    const int lim = ns * 2 * VEC;
    for (int q0 = 0; q0 < lim; q0 += 64) {
        const int q = q0 + lane;
        const float x = q < lim ? sl.sx[wid][q] : __builtin_nanf("");
        const bool p = x >= tau;
        const uint64_t b = ballot(p);
        const int pos = cnt + lanes_below(b);
        if (p && pos < kWaveCand) {
            wk[pos] = ckey(x, sl.sid[wid][q / VEC] + (uint32_t)(q % VEC));
            wv[pos] = x;
        }
        cnt += __popcll(b);
    }
    if constexpr (HAS_PEN) {
#pragma unroll
        for (int u = 0; u < kOwnSlots; ++u) {
            const bool mine = own->id[u] != 0xFFFFFFFFu;
            const float v = mine ? owned_value(a, *t, *own, u) : 0.0f;
            const bool p = mine && v >= tau;
            const uint64_t b = ballot(p);
            const int pos = cnt + lanes_below(b);
            if (p && pos < kWaveCand) {
                wk[pos] = ckey(v, own->id[u]);
                wv[pos] = v;
            }
            cnt += __popcll(b);
        }
    }
    return cnt;
}

// Ranks the n <= kSortMax candidates held in the wave regions (region w has
// cnt[w] entries, concatenated in wave order) and publishes the first min(n,
// k) sorted.  Wave w counts, for every candidate, the entries of region w
// greater than it (broadcast reads); the counts meet after a barrier.  Slots
// [n, k) get key 0.  Contains a barrier.
template <typename T, int NV>
__device__ __forceinline__ void rank_regions(SelectLds<T, NV> &sl, const int (&off)[kWaves + 1], int k,
                                             ChunkOut out) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int n = off[kWaves];
    const int nb = off[wid + 1] - off[wid];
    const uint64_t *rk = sl.wkey[wid];
    for (int i0 = 0; i0 < n; i0 += 64) {
        const int i = i0 + lane;
        if (i < n) {
            int w = 0;
#pragma unroll
            for (int q = 1; q < kWaves; ++q) w += (i >= off[q]);
            int base = 0;
#pragma unroll
            for (int q = 1; q < kWaves; ++q) base = (w == q) ? off[q] : base;
            const uint64_t mine = sl.wkey[w][i - base];
            uint32_t c = 0;
            for (int j = 0; j < nb; ++j) c += (uint32_t)(rk[j] > mine);
            sl.part[wid][i] = c;
        }
    }
    __syncthreads();
    for (int i = tid; i < max(n, k); i += kThreads) {
        if (i < n) {
            uint32_t r = 0;
#pragma unroll
            for (int q = 0; q < kWaves; ++q) r += sl.part[q][i];
            if (r < (uint32_t)k) {
                int w = 0;
#pragma unroll
                for (int q = 1; q < kWaves; ++q) w += (i >= off[q]);
                int base = 0;
#pragma unroll
                for (int q = 1; q < kWaves; ++q) base = (w == q) ? off[q] : base;
                st_agent(&out.key[r], sl.wkey[w][i - base]);
                st_agent(&out.val[r], sl.wval[w][i - base]);
            }
        } else {
            st_agent(&out.key[i], (uint64_t)0);  // padding: below every real key
        }
    }
    if (tid == 0) st_agent(out.cnt, min(n, k));
}

// Ranks the n <= kSortMax unique keys by counting, split over the whole
// workgroup: thread (b, i) counts the keys of block b greater than key i
// (each wave reads the same block keys, so the reads are broadcasts), the
// counts meet in rank[i] (zero on entry), and key i goes to out[rank] when
// rank < k; slots [n, k) get key 0.  Contains a barrier.
__device__ __forceinline__ void rank_publish(const uint64_t *keys, const float *vals, int n, int k,
                                             uint32_t *rank, ChunkOut out) {
    const int tid = threadIdx.x;
    const int np = n <= 64 ? 64 : (n <= 128 ? 128 : 256);
    const int nb = kThreads / np, bs = np / nb;
    const int i = tid & (np - 1), b = tid / np;
    if (i < n) {
        const uint64_t mine = keys[i];
        const int j0 = b * bs, j1 = min(j0 + bs, n);
        uint32_t c = 0;
        for (int j = j0; j < j1; ++j) c += (uint32_t)(keys[j] > mine);
        if (c) atomicAdd(&rank[i], c);
    }
    __syncthreads();
    if (tid < n) {
        const uint32_t r = rank[tid];
        if (r < (uint32_t)k) {
            st_agent(&out.key[r], keys[tid]);
            st_agent(&out.val[r], vals[tid]);
        }
    } else if (tid < k) {
        st_agent(&out.key[tid], (uint64_t)0);  // padding: below every real key
    }
    if (tid == 0) st_agent(out.cnt, min(n, k));
}

// Ranks n <= kRankMax unique keys by counting (each key's rank is the number
// of keys greater than it; counting stops at k) and publishes the first
// min(n, k) sorted; slots [n, k) get key 0.  No barrier.
constexpr int kRankMax = 1024;
__device__ __forceinline__ void rank_count(const uint64_t *keys, const float *vals, int n, int k, ChunkOut out) {
    const int tid = threadIdx.x;
    for (int i = tid; i < n; i += kThreads) {
        const uint64_t mine = keys[i];
        uint32_t c = 0;
        int j = 0;
        for (; j + 8 <= n && c < (uint32_t)k; j += 8) {
#pragma unroll
            for (int q = 0; q < 8; ++q) c += (uint32_t)(keys[j + q] > mine);
        }
        for (; j < n && c < (uint32_t)k; ++j) c += (uint32_t)(keys[j] > mine);
        if (c < (uint32_t)k) {
            st_agent(&out.key[c], mine);
            st_agent(&out.val[c], vals[i]);
        }
    }
    for (int i = n + tid; i < k; i += kThreads) st_agent(&out.key[i], (uint64_t)0);  // padding
    if (tid == 0) st_agent(out.cnt, min(n, k));
}

// Stage A after chunk_stream: find the chunk's exact top-min(k, selectable)
// sorted by (value desc, id asc), publish it to `out` (agent-scope stores).
// LDS: `sl` (SelectLds), `t` when HAS_PEN (with the owners in `own`), small
// scalars.
// The threshold comes from chunk_tau here, or (PRE_TAU) from select_prepare
// run earlier, e.g. mid-stream on part of the chunk (a k-th largest of a
// subset is still a lower bound).
template <typename T, int NV>
__device__ __forceinline__ float select_prepare(float lmax, int k, SelectLds<T, NV> &sl, uint32_t *s_tau, int *s_n) {
    const int tid = threadIdx.x;
    if (tid == 0) *s_n = 0;
    if (tid < kSortMax) sl.rank[tid] = 0u;
    return chunk_tau(lmax, k, sl.uni, s_tau);  // barriers: *s_n and rank settled
}

template <typename T, int NV, bool HAS_PEN, bool PRE_TAU = false>
__device__ __forceinline__ void chunk_select_publish(const RowSource &a, ChunkRegs<T, NV> &cr, int c0, int k,
                                                     SelectLds<T, NV> &sl, const PenTable *t, const PenOwn *own,
                                                     uint32_t *s_tau, int *s_n, uint32_t *bins, int *s_dig,
                                                     ChunkOut out, float pre_tau = 0.0f) {
    constexpr int VEC = VecTraits<T>::VEC;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const float tau = PRE_TAU ? pre_tau : select_prepare<T, NV>(cr.lmax, k, sl, s_tau, s_n);
    const int wc = wave_candidates<T, NV, HAS_PEN>(a, cr, c0, tau, sl, t, own);
    if (lane == 0) sl.wcnt[wid] = wc;
    __syncthreads();
    int off[kWaves + 1];
    off[0] = 0;
    bool overflow = false;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        overflow |= sl.wcnt[w] > kWaveCand;
        off[w + 1] = off[w] + min(sl.wcnt[w], kWaveCand);
    }
    if (!overflow && off[kWaves] <= kSortMax) {  // uniform: read from LDS after the barrier
        rank_regions<T, NV>(sl, off, k, out);
        return;
    }
    // More candidates than the wave regions take: every entry >= tau (the
    // top-k are among them) is gathered and ranked by counting.
    if (tid == 0) *s_n = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if (cr.m4[j] >= tau) {  // NaN (empty vector) fails
            const int e0 = c0 + (j * kThreads + tid) * VEC;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                const float x = cr.x[j * VEC + e];
                if (x >= tau) {
                    const int q = atomicAdd(s_n, 1);
                    if (q < kCandCap) {
                        sl.ckey[q] = ckey(x, (uint32_t)(e0 + e));
                        sl.cval[q] = x;
                    }
                }
            }
        }
    }
    if constexpr (HAS_PEN) {
#pragma unroll
        for (int u = 0; u < kOwnSlots; ++u) {
            if (own->id[u] != 0xFFFFFFFFu) {
                const float v = owned_value(a, *t, *own, u);
                if (v >= tau) {
                    const int q = atomicAdd(s_n, 1);
                    if (q < kCandCap) {
                        sl.ckey[q] = ckey(v, own->id[u]);
                        sl.cval[q] = v;
                    }
                }
            }
        }
    }
    __syncthreads();
    const int nc = *s_n;
    if (nc <= kRankMax) {  // uniform
        rank_count(sl.ckey, sl.cval, nc, k, out);
        return;
    }
    // Still too many (ties, flat rows): exact radix select over registers +
    // penalized entries, then rank the top-k.
    __syncthreads();  // every thread has read *s_n before it is reset
    int ne = 0;
    if constexpr (HAS_PEN) {
        if (tid == 0) *s_n = 0;
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kOwnSlots; ++u) {
            if (own->id[u] != 0xFFFFFFFFu) {
                const float v = owned_value(a, *t, *own, u);
                const int q = atomicAdd(s_n, 1);  // < kMaxWin + kMaxEdits <= kCandCap
                sl.ckey[q] = ckey(v, own->id[u]);
                sl.cval[q] = v;
            }
        }
        __syncthreads();
        ne = *s_n;
    }
    RegKeySrc<T, NV> src{&cr, c0, sl.ckey, ne};
    const uint64_t T0 = block_select(src, k, bins, s_dig);
    if (tid == 0) *s_n = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e0 = c0 + (j * kThreads + tid) * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const float x = cr.x[j * VEC + e];
            if (x == x) {
                const uint64_t key = ckey(x, (uint32_t)(e0 + e));
                if (key >= T0) {
                    const int q = atomicAdd(s_n, 1);
                    if (q < kCapA) {
                        sl.skey[q] = key;
                        sl.sval[q] = x;
                    }
                }
            }
        }
    }
    for (int i = tid; i < ne; i += kThreads) {
        if (sl.ckey[i] >= T0) {
            const int q = atomicAdd(s_n, 1);
            if (q < kCapA) {
                sl.skey[q] = sl.ckey[i];
                sl.sval[q] = sl.cval[i];
            }
        }
    }
    __syncthreads();
    rank_publish(sl.skey, sl.sval, min(*s_n, kCapA), k, sl.rank, out);
}

// ------------------------------------------- stage A with late penalties
// For penalties that never raise a logit (repetition penalty >= 1, frequency
// and presence >= 0, edit deltas >= 0) the chunk is selected on its raw
// values and only the candidates are penalized, so nothing in the stream
// waits for the history, which arrives behind the row.
//
// Why it is exact: C = every raw value >= tau.  A value outside C is below
// tau before its penalty and so after it.  Penalize C in place; if at least k
// of C are still >= tau, the chunk's top-k lie in C and rank_regions ranks
// them by their penalized keys.  Otherwise (penalized candidates fell below
// tau) the penalties are applied to the registers and the plain select runs.

// Clears the id -> (count, delta) hash (the bitset is not used here).
__device__ __forceinline__ void pen_clear_hash(PenTable &t) {
    for (int i = threadIdx.x; i < kHashMax; i += kThreads) {
        t.key[i] = 0u;
        t.cnt[i] = 0u;
        t.delta[i] = 0.0f;
    }
}

// Fills the hash with the chunk's window ids (counts) and edits (deltas).
// Returns true when an edit of this chunk has a delta that is negative or
// NaN, which could raise a logit.  No barrier.
__device__ __forceinline__ bool pen_count_late(PenTable &t, const RowPen &rp, const PenRegs &pr, int c0, int c1) {
#pragma unroll
    for (int u = 0; u < kWinPerThread; ++u) {
        const uint32_t id = pr.w[u];
        if (id >= (uint32_t)c0 && id < (uint32_t)c1) atomicAdd(&t.cnt[pen_insert(t, id, rp.hs_log2)], 1u);
    }
    bool bad = false;
    if (pr.e >= (uint32_t)c0 && pr.e < (uint32_t)c1) {
        t.delta[pen_insert(t, pr.e, rp.hs_log2)] = pr.d;
        bad = !(pr.d >= 0.0f);
    }
    return bad;
}

// Slot of `id` in the hash, or -1.  The table holds at least twice as many
// slots as ids, so an empty slot ends every probe.
__device__ __forceinline__ int pen_find(const PenTable &t, uint32_t id, int hs_log2) {
    uint32_t h = hash_slot(id, hs_log2);
    const uint32_t m = (1u << hs_log2) - 1;
    for (;;) {
        const uint32_t kk = t.key[h];
        if (kk == id + 1) return (int)h;
        if (kk == 0u) return -1;
        h = (h + 1) & m;
    }
}

// Upper bound of the final-logit softcap of every value below tau (f32 body
// or scalar tail, src/model.zig:2492-2513): cap tanh(tau / cap) in f64 plus
// cap 2^-17, rounded up.  The exact function is monotone; the f32 forms stay
// within cap 2^-22 of it (the body) and a few ulps (the tail), and the body's
// argument rounding moves tanh by at most cap 9 2^-23 inside its +-9 clamp.
// Below tau = -9 cap (and for tau = -inf or NaN) the body's clamp maps -inf
// to -cap tanh(9), above cap tanh(tau / cap): no bound, *ok = false.
__device__ __forceinline__ float softcap_upper(const RowSource &a, float tau, bool *ok) {
    *ok = tau > -9.0f * a.cap;
    const double cp = (double)a.cap;
    const double e = cp * tanh((double)tau / cp) + cp * 0x1p-17;
    float u = (float)e;
    if ((double)u < e) u = nextafterf(u, INFINITY);
    return u;
}

// The chunk's selection after chunk_stream without penalties: `tau` from
// select_prepare (raw lane maxima), `pr` from pen_prefetch, hl_raw / ne_raw
// the row's hist_len / edit_count as loaded, `t` cleared by pen_clear_hash
// before a barrier that precedes this call, *s_bad zero.  Publishes the
// chunk's exact penalized top-k like chunk_select_publish.
// CAPC (a final-logit softcap): the stream ran without it, and only the
// candidates are capped (then penalized).  A value outside C is below tau,
// so its capped value is below tc = softcap_upper(tau) and its penalized one
// too; with at least k candidates >= tc the top-k lie in C.  Otherwise the
// chunk is streamed again with the softcap and selected as before.
// PENL = false (a softcap without penalties or edits): no hash; t, pr and
// s_bad are not used.
template <typename T, int NV, bool CAPC = false, bool HAS_MASK = false, bool PENL = true>
__device__ __forceinline__ void chunk_select_late(const RowSource &a, int row, ChunkRegs<T, NV> &cr, int c0, int c1,
                                                  int k, SelectLds<T, NV> &sl, PenTable *tp, PenRegs *pr, int hl_raw,
                                                  int ne_raw, uint32_t *s_tau, int *s_n, int *s_bad, uint32_t *bins,
                                                  int *s_dig, ChunkOut out, float tau) {
    static_assert(PENL || CAPC, "without penalties this select is for capped rows");
    constexpr int VEC = VecTraits<T>::VEC;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wc = wave_candidates<T, NV, false>(a, cr, c0, tau, sl, nullptr, nullptr);
    RowPen rp;
    rp.any = false;
    rp.hs_log2 = 6;
    if constexpr (PENL) {
        rp = row_pen_from(a, row, row_pen_window_on(a) ? hl_raw : 0, a.edit_ids ? ne_raw : 0);
        pen_window(rp, *pr);
        if (pen_count_late(*tp, rp, *pr, c0, c1)) *s_bad = 1;
    }
    if (lane == 0) sl.wcnt[wid] = wc;
    bool cap_ok = true;
    const float tc = CAPC ? softcap_upper(a, tau, &cap_ok) : tau;  // uniform
    __syncthreads();  // hash, wave counts and the bad-edit flag complete
    int off[kWaves + 1];
    off[0] = 0;
    bool overflow = (PENL && *s_bad != 0) || !cap_ok;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        overflow |= sl.wcnt[w] > kWaveCand;
        off[w + 1] = off[w] + min(sl.wcnt[w], kWaveCand);
    }
    if (!overflow && off[kWaves] <= kSortMax) {  // uniform
        const int nw = off[wid + 1] - off[wid];   // <= kWaveCand = 64: one entry per lane
        bool ge = false;
        if (lane < nw) {
            float x = sl.wval[wid][lane];
            const uint32_t id = ckey_id(sl.wkey[wid][lane]);
            bool upd = CAPC;
            if constexpr (CAPC) x = softcap_at(a, (int)id, x);
            if (PENL && rp.any) {
                const PenTable &t = *tp;
                const int h = pen_find(t, id, rp.hs_log2);
                if (h >= 0) {
                    x = pen_apply(x, t.cnt[h], t.delta[h], a);
                    upd = true;
                }
            }
            if (upd) {
                sl.wkey[wid][lane] = ckey(x, id);
                sl.wval[wid][lane] = x;
            }
            ge = x >= tc;
        }
        const uint64_t b = ballot(ge);
        if (lane == 0) sl.wge[wid] = __popcll(b);
        __syncthreads();  // penalized regions and counts complete
        int nge = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) nge += sl.wge[w];
        if (nge >= k) {  // uniform
            rank_regions<T, NV>(sl, off, k, out);
            return;
        }
    }
    // Fallback: penalize the registers (every element probes the hash) and
    // select from scratch.  select_prepare's barriers order its LDS writes
    // after every read above.
    if constexpr (CAPC) chunk_stream<T, NV, HAS_MASK, false, true>(a, row, c0, c1, cr, nullptr, nullptr);
    if (PENL && rp.any) {
        const PenTable &t = *tp;
        float tmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int e0 = c0 + (j * kThreads + tid) * VEC;
            float m = __builtin_nanf("");
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                float x = cr.x[j * VEC + e];
                if (x == x) {
                    const int h = pen_find(t, (uint32_t)(e0 + e), rp.hs_log2);
                    if (h >= 0) x = pen_apply(x, t.cnt[h], t.delta[h], a);
                    cr.x[j * VEC + e] = x;
                }
                m = fmaxf(m, x);
            }
            cr.m4[j] = m;
            tmax = fmaxf(tmax, m);
        }
        cr.lmax = tmax;
    }
    chunk_select_publish<T, NV, false>(a, cr, c0, k, sl, nullptr, nullptr, s_tau, s_n, bins, s_dig, out);
}

// ------------------------------------------- running list of a walking workgroup
// A workgroup that walks several chunks keeps its top-k so far sorted in LDS
// (double-buffered); each chunk publishes its own list to bk / bv / bn.
struct RowLoopLds {
    uint64_t key[2][kCapA];  // running list, double-buffered
    float val[2][kCapA];
    uint64_t bk[kCapA];      // this chunk's list
    float bv[kCapA];
    int32_t bn;
};

// Entries of the sorted-descending list L[0, n) greater than `mine`.
__device__ __forceinline__ int count_greater_n(const uint64_t *L, int n, uint64_t mine) {
    int lo = 0, hi = n;  // L[i] > mine for i < lo, L[i] <= mine for i >= hi
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (L[mid] > mine) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Merges the chunk's list (bk, bv, bn; after a barrier) into the running list
// by rank: each entry binary-searches the other list and writes itself to its
// rank in the other buffer.  Ends with a barrier.
__device__ __forceinline__ void running_merge(RowLoopLds &rl, int &cur, int &n_run, int k) {
    const int tid = threadIdx.x;
    const int nb = rl.bn;
    const int nxt = cur ^ 1;
    if (tid < n_run) {
        const uint64_t mine = rl.key[cur][tid];
        const int r = tid + count_greater_n(rl.bk, nb, mine);
        if (r < k) {
            rl.key[nxt][r] = mine;
            rl.val[nxt][r] = rl.val[cur][tid];
        }
    } else if (tid >= kCapA && tid - kCapA < nb) {
        const int i = tid - kCapA;
        const uint64_t mine = rl.bk[i];
        const int r = i + count_greater_n(rl.key[cur], n_run, mine);
        if (r < k) {
            rl.key[nxt][r] = mine;
            rl.val[nxt][r] = rl.bv[i];
        }
    }
    n_run = min(k, n_run + nb);
    cur = nxt;
    __syncthreads();  // the running list is complete; stage-A LDS may be reused
}

// ------------------------------------------------------------- stage B
// Loads the G sorted chunk lists of a row (one round trip: every slot is
// requested before any is used; every list holds k slots, padded with key 0)
// and merges them by rank: the rank of a live entry is the number of entries
// greater than it over all lists (its own list included), each count a
// branch-free binary search, the searches of one entry advanced in lock-step.
// Writes the row's top-min(k, total) to okey/oval sorted; returns that count.
struct MergeLds {
    uint64_t key[kMaxG][kCapA];
    float val[kMaxG][kCapA];
    int cnt[kMaxG];
};

// Entries of the sorted-descending, zero-padded list L[0, P) greater than
// `mine` (P a power of two; every read in bounds).
template <int MG>
__device__ __forceinline__ void count_greater(const MergeLds &ml, int P, uint64_t mine, int (&pos)[MG]) {
#pragma unroll
    for (int h = 0; h < MG; ++h) pos[h] = 0;
    for (int st = P >> 1; st > 0; st >>= 1) {
        uint64_t kv[MG];
#pragma unroll
        for (int h = 0; h < MG; ++h) kv[h] = ml.key[h][pos[h] + st - 1];
#pragma unroll
        for (int h = 0; h < MG; ++h) pos[h] += (kv[h] > mine) ? st : 0;
    }
    uint64_t kv[MG];
#pragma unroll
    for (int h = 0; h < MG; ++h) kv[h] = ml.key[h][pos[h]];
#pragma unroll
    for (int h = 0; h < MG; ++h) pos[h] += (kv[h] > mine) ? 1 : 0;
}

template <int MG>
__device__ __forceinline__ void merge_rank(const MergeLds &ml, int G, int P, int need, uint64_t *okey, float *oval) {
    const int lgP = __builtin_ctz(P);
    for (int s = threadIdx.x; s < G * P; s += kThreads) {
        const int g = s >> lgP, i = s & (P - 1);
        const uint64_t mine = ml.key[g][i];
        int pos[MG];
        count_greater<MG>(ml, P, mine, pos);
        int r = 0;
#pragma unroll
        for (int h = 0; h < MG; ++h) r += pos[h];
        if (mine != 0ull && r < need) {
            okey[r] = mine;
            oval[r] = ml.val[g][i];
        }
    }
}

__device__ __forceinline__ int row_merge(const uint64_t *g_key, const float *g_val, const int32_t *g_cnt, int row,
                                         int G, int k, MergeLds &ml, uint64_t *okey, float *oval) {
    const int tid = threadIdx.x;
    const int64_t rb = (int64_t)row * G;
    int P = 1;
    while (P < k) P <<= 1;  // k <= P <= kCapA
    const int MG = G <= 4 ? 4 : kMaxG;  // lists searched in lock-step (missing ones all zero)
    if (tid < k) {  // k <= kCapA <= kThreads
        uint64_t kk[kMaxG];
        float vv[kMaxG];
#pragma unroll
        for (int g = 0; g < kMaxG; ++g) {
            if (g < G) {
                kk[g] = ld_agent(&g_key[(rb + g) * kCapA + tid]);
                vv[g] = ld_agent(&g_val[(rb + g) * kCapA + tid]);
            }
        }
#pragma unroll
        for (int g = 0; g < kMaxG; ++g) {
            if (g < G) {
                ml.key[g][tid] = kk[g];
                ml.val[g][tid] = vv[g];
            }
        }
    }
    if (tid < G) ml.cnt[tid] = ld_agent(&g_cnt[rb + tid]);
    for (int s = tid; s < MG * P; s += kThreads) {  // padding slots and missing lists
        const int g = s / P, i = s - (s / P) * P;
        if (g >= G || i >= k) ml.key[g][i] = 0ull;
    }
    __syncthreads();
    int total = 0;
#pragma unroll
    for (int g = 0; g < kMaxG; ++g) total += g < G ? ml.cnt[g] : 0;
    const int need = min(k, total);
    if (MG == 4) merge_rank<4>(ml, G, P, need, okey, oval);
    else merge_rank<kMaxG>(ml, G, P, need, okey, oval);
    __syncthreads();
    return need;
}

}  // namespace zi
