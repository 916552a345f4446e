// zi_whole.hip -- whole-order sampling of bf16 rows without a sort:
// Sampler.sampleWithMargin (src/sampler.zig:190-276) with k = V (the
// std.mem.sort branch, :198-202) for the rows the prefix pass flagged, in
// O(V + distinct values) per row.
//
// A bf16 row holds at most 65536 distinct values, and only those within
// fl(x - mx) >= -16.75 (terms >= 2^-24; below it a term changes no sequential
// sum, every prefix being >= 1) or above the min-p floor can matter.  So the
// order the reference sorts is a list of groups (value, count) in descending
// value, and every sum of the tail is walked over the groups exactly
// (zi_walk.hpp).  Only the drawn entry's position needs its id: among the
// entries of its value, ascending id (the stable sort's tie rule).
//
// One 512-thread workgroup per flagged row:
//  1. penalty hash in LDS; each penalized id's first inserter loads its logit
//     and keeps its count and delta.
//  2-3. read the row: entries per 16-bit order key (two 16-bit counts per LDS
//     word, 128 KB), penalized ids' raw entries then taken out; a count that
//     overflowed (more than 65535 equal entries) shows as a short total.
//  4. each thread reads its 128 keys' counts: the row max and second value,
//     the floor, the penalized entries above it.
//  5. ranks of the present keys at or above the floor (descending, a suffix
//     count over threads, into arrays beside the counts); the group list: key
//     groups and penalized entries (one group each) merged by value.
//  6. wave 0 walks the groups: the top-p total and crossing, min-p, the
//     temperature total over keep, the draw.
//  7. the drawn entry's id: the (j+1)-th entry, in id order, of its value.
// A row with more distinct values above the floor than the group list holds,
// a non-finite maximum, or no selectable entry keeps its flag, and the
// sorting pass (zi_exact.hip) runs it.
#include "zi_launch.hpp"
#include "zi_rowpass.hpp"
#include "zi_walk.hpp"

namespace zi {

constexpr int kWholeKeys = 4096;                   // distinct bf16 values above the floor
constexpr int kWholePen = kMaxWin + kMaxEdits;      // penalized entries (distinct window and edit ids)
constexpr int kWholeGroups = kWholeKeys + kWholePen;
constexpr int kWholeBatch = 16;  // row vectors in flight per thread

// (group, running value) at the start of each step of a block walk
constexpr int kWalkCp = 64;
struct WalkCp {
    int g[kWalkCp];
    float v[kWalkCp];
    int n;
};

constexpr int kKeyWords = 65536 / 2;  // 16-bit order keys, two 16-bit counts per word

struct WholeLds {
    union {
        struct {  // step 1: the penalty hash
            uint32_t key[kHashMax];
            uint32_t cnt[kHashMax];
            float delta[kHashMax];
            uint32_t own[kHashMax];  // claimed by the id's first inserter
        } h;
        uint32_t kc[kKeyWords];  // steps 2-5: entries per key, two 16-bit counts per word
        struct {                 // steps 5-6
            float gval[kWholeGroups];
            uint32_t gcnt[kWholeGroups];
            union {
                uint32_t gpos[kWholeGroups];     // step 6: entries before each group
                uint32_t vbits[kMaxVocab / 32];  // step 7: penalized ids whose value is the drawn one
            } w;
        } g;
        uint32_t pbits[kMaxVocab / 32];  // step 7: penalized ids (over the group list, no longer read)
    } u;
    uint16_t bkey[kWholeKeys];  // step 5: key of each rank
    uint16_t bcnt[kWholeKeys];  // entries per key rank (at most 65535: step 4 checks)
    struct {  // block walks: the waves' total maps and first events, by chunk parity
        uint64_t inc0[2][kWaves], inc1[2][kWaves];
        uint32_t par[2][kWaves];
        int ev[2][kWaves];
        uint64_t ep;
        float et;
        uint32_t ec;
        int first;
    } wb;
    WalkCp cp;                   // the top-p total's checkpoints
    float pval[kWholePen];       // penalized entries: value, id (sorted in place by value desc, id asc)
    uint32_t pid[kWholePen];
    float wt1[kWaves], wt2[kWaves];
    uint32_t wsum[kWaves];
    uint32_t tcnt[kMaxVocab / (8 * kThreads)];  // entries of the drawn value per 4096-id tile
    int npen, nsel;
    int found;
    int k1, k2, c1;     // the highest present key, its count, the next present key
    uint32_t ncnt, nsum;  // entries counted, and the sum of the key counts (a 16-bit count overflowed if they differ)
    uint32_t tok;
    float f[4];
    int64_t i64[4];
};

// bf16 order key: the high half of okey (exact for bf16 values: their low
// halves are one constant per sign), and back.
__device__ __forceinline__ uint32_t key16(float v) { return okey(v) >> 16; }
__device__ __forceinline__ float key16_value(uint32_t k) {
    return (k & 0x8000u) ? __uint_as_float((k & 0x7FFFu) << 16) : __uint_as_float(((~k) & 0xFFFFu) << 16);
}

// The smallest float f with every x >= f having fl(x - mx) >= dlo (a value a
// little below mx + dlo, rounded down; a lower floor only keeps more).
__device__ __forceinline__ float whole_floor(float mx, float dlo) {
    const double d = (double)mx + (double)dlo - (fabs((double)mx) + fabs((double)dlo)) * 1e-6;
    float f = (float)d;
    if ((double)f > d) f = __uint_as_float(__float_as_uint(f) + (f > 0.0f ? -1 : 1));
    return f;
}

__device__ __forceinline__ void top2_merge(float &t1, float &t2, float x) {
    t2 = fmaxf(t2, fminf(t1, x));
    t1 = fmaxf(t1, x);
}

__device__ __forceinline__ uint64_t shfl_up_u64(uint64_t v, int o) {
    const uint32_t lo = __shfl_up((uint32_t)v, o), hi = __shfl_up((uint32_t)(v >> 32), o);
    return ((uint64_t)hi << 32) | lo;
}

// The whole workgroup walks groups [g, gk] from the running value v, the last
// group over its first ck entries: a chunk of 512 groups per step, one per
// thread, the maps scanned over the wave and then across the waves; only the
// group of the first event is walked on its own (by every thread alike).
// Every thread calls it and gets the same result: the entry index at which
// the walk stops (group *sg, copy *sc), or -1; v is the running value.
// With cp, thread 0 records (group, running value) at the start of every step
// (up to kWalkCp of them; the count in cp->n after the caller's next barrier).
template <class Term, class WB>
__device__ int64_t walk_block(const float *gval, const uint32_t *gcnt, const uint32_t *gpos, int gk, uint32_t ck,
                              Term term, int mode, float thr, float &v, int *sg, int64_t *sc, WB &W, int g = 0,
                              WalkCp *cp = nullptr) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    int buf = 0, ncp = 0;
    while (g <= gk) {
        if (cp && ncp < kWalkCp) {  // uniform
            if (tid == 0) {
                cp->g[ncp] = g;
                cp->v[ncp] = v;
                cp->n = ncp + 1;
            }
            ++ncp;
        }
        if ((mode != kWalkDrop && v == 0.0f) || (mode == kWalkDrop && !(v > 0.0f))) {  // no grid yet: one group
            const int64_t s = walk_group(v, term(gval[g]), g == gk ? ck : gcnt[g], mode, thr);
            if (s >= 0) {
                *sg = g;
                *sc = s;
                return (int64_t)gpos[g] + s;
            }
            ++g;
            continue;
        }
        const WalkGrid gr = walk_grid(v);
        const uint32_t p0 = gr.m & 1u;
        const int gl = g + tid;
        const uint32_t c = gl < gk ? gcnt[gl] : (gl == gk ? ck : 0u);
        const float t = c ? term(gval[gl]) : 0.0f;
        WalkMap mp = walk_map(walk_term(t, gr.qe), c);
        uint32_t par = mp.par0 | (mp.par1 << 1);
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {  // inclusive over the wave: earlier lanes' map, then this lane's
            WalkMap pm;
            pm.inc0 = shfl_up_u64(mp.inc0, o);
            pm.inc1 = shfl_up_u64(mp.inc1, o);
            const uint32_t pp = __shfl_up(par, o);
            pm.par0 = pp & 1u;
            pm.par1 = pp >> 1;
            if (lane >= o) {
                mp = walk_compose(pm, mp);
                par = mp.par0 | (mp.par1 << 1);
            }
        }
        WalkMap ex;  // the wave's lanes before this one
        ex.inc0 = shfl_up_u64(mp.inc0, 1);
        ex.inc1 = shfl_up_u64(mp.inc1, 1);
        const uint32_t pe = __shfl_up(par, 1);
        ex.par0 = pe & 1u;
        ex.par1 = pe >> 1;
        if (lane == 0) {
            ex.inc0 = ex.inc1 = 0;
            ex.par0 = 0;
            ex.par1 = 1;
        }
        if (lane == 63) {
            W.inc0[buf][wid] = mp.inc0;
            W.inc1[buf][wid] = mp.inc1;
            W.par[buf][wid] = par;
        }
        __syncthreads();
        WalkMap pre;  // the waves before this one
        pre.inc0 = pre.inc1 = 0;
        pre.par0 = 0;
        pre.par1 = 1;
        for (int w = 0; w < wid; ++w) {
            WalkMap o;
            o.inc0 = W.inc0[buf][w];
            o.inc1 = W.inc1[buf][w];
            o.par0 = W.par[buf][w] & 1u;
            o.par1 = W.par[buf][w] >> 1;
            pre = walk_compose(pre, o);
        }
        const WalkMap in = walk_compose(pre, mp);
        const bool ev = c > 0 && walk_event(gr.m, gr.qe, p0 ? in.inc1 : in.inc0, mode, thr);
        const uint64_t b = ballot(ev);
        if (lane == 0) W.ev[buf][wid] = b ? __ffsll((unsigned long long)b) - 1 : 64;
        __syncthreads();
        int E = -1;
        for (int w = 0; w < kWaves && E < 0; ++w)
            if (W.ev[buf][w] < 64) E = w * 64 + W.ev[buf][w];
        if (E < 0) {  // no event in the chunk: all of it as integers
            WalkMap tot = pre;
            for (int w = wid; w < kWaves; ++w) {
                WalkMap o;
                o.inc0 = W.inc0[buf][w];
                o.inc1 = W.inc1[buf][w];
                o.par0 = W.par[buf][w] & 1u;
                o.par1 = W.par[buf][w] >> 1;
                tot = walk_compose(tot, o);
            }
            const uint64_t Pt = p0 ? tot.inc1 : tot.inc0;
            v = walk_value(mode == kWalkDrop ? gr.m - Pt : gr.m + Pt, gr.qe);
            g += kThreads;
            buf ^= 1;
            continue;
        }
        if (tid == E) {
            const WalkMap bx = walk_compose(pre, ex);
            W.ep = p0 ? bx.inc1 : bx.inc0;
            W.et = t;
            W.ec = c;
        }
        __syncthreads();
        const uint64_t Pp = W.ep;
        const float te = W.et;
        const uint32_t ce = W.ec;
        __syncthreads();  // read by every thread before the next event rewrites them
        v = walk_value(mode == kWalkDrop ? gr.m - Pp : gr.m + Pp, gr.qe);
        const int64_t s = walk_group(v, te, ce, mode, thr);
        const int ge = g + E;
        if (s >= 0) {
            *sg = ge;
            *sc = s;
            return (int64_t)gpos[ge] + s;
        }
        g = ge + 1;
        buf ^= 1;
    }
    return -1;
}

template <bool HAS_MASK, bool HAS_PEN>
__global__ __launch_bounds__(kThreads) void whole_kernel(ExactParams P) {
    __shared__ WholeLds L;
    const RowSource &a = P.src;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int row = blockIdx.x;
    if (P.flags[row] == 0) return;  // settled by the prefix pass (uniform)
    const int V = a.V;
    constexpr int VEC = 8;
    const int nvec = (V + VEC - 1) / VEC;
    const uint16_t *lrow = reinterpret_cast<const uint16_t *>(a.logits) + (int64_t)row * a.ld;
    const uint32_t *mrow = HAS_MASK ? a.mask + (int64_t)row * a.mask_ld : nullptr;

    // 1. penalties: the window ids (counts) and the edits (deltas) in a hash;
    //    the first inserter of each id owns it, loads its logit and keeps its
    //    count and delta in registers (the hash's memory then holds the key
    //    counts)
    uint32_t oid[kOwnSlots];
    uint32_t oraw[kOwnSlots];
    uint32_t ocnt[kOwnSlots];
    float odel[kOwnSlots];
#pragma unroll
    for (int s = 0; s < kOwnSlots; ++s) {
        oid[s] = 0xFFFFFFFFu;
        oraw[s] = 0u;
        ocnt[s] = 0u;
        odel[s] = 0.0f;
    }
    if constexpr (HAS_PEN) {
        PenRegs pr;
        pen_prefetch(a, row, pr);
        const RowPen rp = row_pen(a, row);
        pen_window(rp, pr);
        for (int i = tid; i < kHashMax; i += kThreads) {
            L.u.h.key[i] = 0u;
            L.u.h.cnt[i] = 0u;
            L.u.h.delta[i] = 0.0f;
            L.u.h.own[i] = 0u;
        }
        __syncthreads();
        int oslot[kOwnSlots];
#pragma unroll
        for (int s = 0; s < kOwnSlots; ++s) {
            oslot[s] = -1;
            const uint32_t id = s < kWinPerThread ? pr.w[s] : pr.e;
            if (id < (uint32_t)V) {
                const int h = pen_insert(L.u.h, id, rp.hs_log2);
                if (s < kWinPerThread) atomicAdd(&L.u.h.cnt[h], 1u);
                else L.u.h.delta[h] = pr.d;
                if (atomicOr(&L.u.h.own[h], 1u) == 0u) {
                    oid[s] = id;
                    oslot[s] = h;
                }
            }
        }
#pragma unroll
        for (int s = 0; s < kOwnSlots; ++s)
            if (oid[s] != 0xFFFFFFFFu) oraw[s] = (uint32_t)lrow[oid[s]];
        __syncthreads();  // counts and deltas complete
#pragma unroll
        for (int s = 0; s < kOwnSlots; ++s) {
            if (oslot[s] >= 0) {
                ocnt[s] = L.u.h.cnt[oslot[s]];
                odel[s] = L.u.h.delta[oslot[s]];
            }
        }
        __syncthreads();  // every read of the hash is done
    }

    // 2. the key counts, cleared
    for (int i = tid; i < kKeyWords; i += kThreads) L.u.kc[i] = 0u;
    if (tid == 0) {
        L.npen = 0;
        L.nsel = 0;
        L.found = 0;
        L.k1 = -1;
        L.k2 = -1;
        L.c1 = 0;
        L.ncnt = 0u;
        L.nsum = 0u;
    }
    __syncthreads();

    // 3. read the row: entries per 16-bit order key, every non-NaN entry
    //    (penalized ones too: their raw entries leave the counts below)
    uint32_t ncount = 0;
    for (int q0 = tid; q0 < nvec; q0 += kThreads * kWholeBatch) {
        uint4 rawb[kWholeBatch];
        uint32_t mwb[kWholeBatch];
#pragma unroll
        for (int j = 0; j < kWholeBatch; ++j) {  // every load first
            const int q = q0 + j * kThreads;
            rawb[j] = make_uint4(0u, 0u, 0u, 0u);
            mwb[j] = 0u;
            if (q < nvec) {
                rawb[j] = *reinterpret_cast<const uint4 *>(lrow + q * VEC);
                if (HAS_MASK) mwb[j] = mrow[(q * VEC) >> 5];
            }
        }
#pragma unroll
        for (int j = 0; j < kWholeBatch; ++j) {
            const int q = q0 + j * kThreads;
            if (q >= nvec) continue;  // (not break: the loop stays unrolled, rawb in registers)
            float v[VEC];
            unpack<uint16_t>(rawb[j], v);
            const int id0 = q * VEC;
            const uint32_t mb = HAS_MASK ? mwb[j] >> (id0 & 31) : 0xFFu;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                if (id0 + e >= V) continue;
                float x = v[e];
                if (HAS_MASK && !((mb >> e) & 1u)) x = -INFINITY;
                if (x != x) continue;  // NaN: no place in the order (outside the reference's contract)
                const uint32_t k = key16(x);
                atomicAdd(&L.u.kc[k >> 1], (k & 1u) ? 0x10000u : 1u);  // no return: nothing waits on it
                ++ncount;
            }
        }
    }
    // the penalized entries: their raw entries out, their penalized values kept
    float pvs[kOwnSlots];
#pragma unroll
    for (int s = 0; s < kOwnSlots; ++s) {
        pvs[s] = __builtin_nanf("");
        if (HAS_PEN && oid[s] != 0xFFFFFFFFu) {
            float x = __uint_as_float(oraw[s] << 16);
            if (HAS_MASK && !((mrow[oid[s] >> 5] >> (oid[s] & 31)) & 1u)) x = -INFINITY;
            if (x == x) {
                const uint32_t k = key16(x);
                atomicSub(&L.u.kc[k >> 1], (k & 1u) ? 0x10000u : 1u);
                --ncount;
            }
            pvs[s] = pen_apply(x, ocnt[s], odel[s], a);
        }
    }
    __syncthreads();  // counts final

    // 4. this thread's 128 keys [128 tid, 128 tid + 128) (slot q = key - 128
    //    tid): the two highest present, and the sum of the counts
    constexpr int kKeyPer = 65536 / kThreads;  // 128
    const uint4 *kc4 = reinterpret_cast<const uint4 *>(L.u.kc + tid * (kKeyPer / 2));
    auto count_at = [](const uint4 &t, int q) -> uint32_t {  // slot q of a 16-byte group of 8 slots
        const uint32_t w = (q >> 1) == 0 ? t.x : (q >> 1) == 1 ? t.y : (q >> 1) == 2 ? t.z : t.w;
        return (q & 1) ? (w >> 16) : (w & 0xFFFFu);
    };
    uint32_t nsum = 0;
    int st1 = -1, st2 = -1;
    uint32_t ct1 = 0;
#pragma unroll
    for (int q8 = 0; q8 < kKeyPer / 8; ++q8) {  // keys ascend with the slot
        const uint4 t = kc4[q8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t c = count_at(t, q);
            nsum += c;
            if (c) {
                st2 = st1;
                st1 = 8 * q8 + q;
                ct1 = c;
            }
        }
    }
    const int kt1 = st1 < 0 ? -1 : kKeyPer * tid + st1, kt2 = st2 < 0 ? -1 : kKeyPer * tid + st2;
    atomicAdd(&L.ncnt, ncount);
    atomicAdd(&L.nsum, nsum);
    atomicMax(&L.k1, kt1);
    __syncthreads();
    const int K1 = L.k1;
    if (K1 >= 0 && kt1 == K1) L.c1 = (int)ct1;  // one thread holds each key
    atomicMax(&L.k2, kt1 == K1 ? kt2 : kt1);
    __syncthreads();
    if (L.ncnt != L.nsum) return;  // a 16-bit count overflowed: the sorting pass (uniform)
    float mx = -INFINITY, second = -INFINITY;  // the unpenalized entries' top two
    if (K1 >= 0) {
        mx = key16_value((uint32_t)K1);
        if (L.c1 >= 2) second = mx;
        else if (L.k2 >= 0) second = key16_value((uint32_t)L.k2);
    }
    {  // and the penalized values
        float t1 = -INFINITY, t2 = -INFINITY;
#pragma unroll
        for (int s = 0; s < kOwnSlots; ++s)
            if (pvs[s] == pvs[s]) top2_merge(t1, t2, pvs[s]);
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const float o1 = __shfl_xor(t1, o), o2 = __shfl_xor(t2, o);
            t2 = fmaxf(fmaxf(t2, o2), fminf(t1, o1));
            t1 = fmaxf(t1, o1);
        }
        if (lane == 0) {
            L.wt1[wid] = t1;
            L.wt2[wid] = t2;
        }
        __syncthreads();
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float o1 = L.wt1[w], o2 = L.wt2[w];
            second = fmaxf(fmaxf(second, o2), fminf(mx, o1));
            mx = fmaxf(mx, o1);
        }
    }
    if (!__builtin_isfinite(mx)) return;  // the sorting pass handles it (uniform)
    // the floor: entries below it cannot reach keep nor change a sum
    float fv = -INFINITY;
    if (P.top_p < 1.0f) fv = whole_floor(mx, -16.75f);
    else if (P.min_p > 0.0f) fv = whole_floor(mx, fminf(logf(P.min_p) - 0.01f, 0.0f));
    uint32_t kmin = fv == -INFINITY ? 0u : key16(fv);
    if (fv != -INFINITY && key16_value(kmin) < fv) ++kmin;  // first key whose value is >= fv
#pragma unroll
    for (int s = 0; s < kOwnSlots; ++s) {  // penalized entries at or above the floor
        if (pvs[s] == pvs[s] && pvs[s] >= fv) {
            const int i = atomicAdd(&L.npen, 1);
            L.pval[i] = pvs[s];
            L.pid[i] = oid[s];
        }
    }
    // 5. the present keys at or above the floor, ranked in descending order
    uint32_t mine = 0;
#pragma unroll
    for (int q8 = 0; q8 < kKeyPer / 8; ++q8) {
        const uint4 t = kc4[q8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
            mine += (count_at(t, q) && (uint32_t)(kKeyPer * tid + 8 * q8 + q) >= kmin) ? 1u : 0u;
    }
    uint32_t incl = mine;  // inclusive over higher-or-equal lanes within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_down(incl, o);
        if (lane + o < 64) incl += y;
    }
    if (lane == 0) L.wsum[wid] = incl;
    __syncthreads();  // wave sums; penalized entries collected
    uint32_t rk = incl - mine;  // present keys in higher lanes of this wave, then in higher waves
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
        if (w > wid) rk += L.wsum[w];
    uint32_t D = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) D += L.wsum[w];
    if (D > (uint32_t)kWholeKeys) return;  // too many distinct values: the sorting pass (uniform)
#pragma unroll
    for (int q8 = kKeyPer / 8 - 1; q8 >= 0; --q8) {  // this thread's keys, highest first
        const uint4 t = kc4[q8];
#pragma unroll
        for (int q = 7; q >= 0; --q) {
            const uint32_t c = count_at(t, q);
            const uint32_t k = (uint32_t)(kKeyPer * tid + 8 * q8 + q);
            if (c && k >= kmin) {
                L.bkey[rk] = (uint16_t)k;
                L.bcnt[rk] = (uint16_t)c;
                ++rk;
            }
        }
    }
    const int npen = L.npen;
    {  // penalized entries sorted in place by (value desc, id asc): ranks, then moves
        float pv[kWholePen / kThreads + 1];
        uint32_t pi[kWholePen / kThreads + 1];
        int pr[kWholePen / kThreads + 1];
#pragma unroll
        for (int u = 0; u < kWholePen / kThreads + 1; ++u) {
            const int i = tid + u * kThreads;
            pr[u] = -1;
            pv[u] = 0.0f;
            pi[u] = 0u;
            if (i < npen) {
                pv[u] = L.pval[i];
                pi[u] = L.pid[i];
                int r = 0;
                for (int j = 0; j < npen; ++j) {
                    const float vj = L.pval[j];
                    r += (vj > pv[u] || (vj == pv[u] && L.pid[j] < pi[u])) ? 1 : 0;
                }
                pr[u] = r;
            }
        }
        __syncthreads();  // every rank computed; key ranks stored; every count read
#pragma unroll
        for (int u = 0; u < kWholePen / kThreads + 1; ++u) {
            if (pr[u] >= 0) {
                L.pval[pr[u]] = pv[u];
                L.pid[pr[u]] = pi[u];
            }
        }
    }
    __syncthreads();  // penalized order complete

    // the group list: key groups and penalized entries merged by value (a key
    // group before the penalized entries of its value)
    for (int r = tid; r < (int)D; r += kThreads) {
        const float vr = key16_value(L.bkey[r]);
        int lo = 0, hi = npen;  // penalized entries with value > vr
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (L.pval[mid] > vr) lo = mid + 1;
            else hi = mid;
        }
        L.u.g.gval[r + lo] = vr;
        L.u.g.gcnt[r + lo] = L.bcnt[r];
    }
    for (int p = tid; p < npen; p += kThreads) {
        const float vp = L.pval[p];
        int lo = 0, hi = (int)D;  // key groups with value >= vp
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (key16_value(L.bkey[mid]) >= vp) lo = mid + 1;
            else hi = mid;
        }
        L.u.g.gval[p + lo] = vp;
        L.u.g.gcnt[p + lo] = 1u;
    }
    __syncthreads();
    const int G = (int)D + npen;

    // 6. the tail's sums, every thread walking alike; first the entries
    //    before each group
    {
        constexpr int kPer = (kWholeGroups + kThreads - 1) / kThreads;
        const int g0 = tid * kPer;
        uint32_t loc = 0;
        for (int k = 0; k < kPer; ++k)
            if (g0 + k < G) loc += L.u.g.gcnt[g0 + k];
        uint32_t incl = loc;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t y = __shfl_up(incl, o);
            if (lane >= o) incl += y;
        }
        if (lane == 63) L.wsum[wid] = incl;
        __syncthreads();
        uint32_t run = incl - loc;
        for (int w = 0; w < wid; ++w) run += L.wsum[w];
        for (int k = 0; k < kPer; ++k)
            if (g0 + k < G) {
                L.u.g.w.gpos[g0 + k] = run;
                run += L.u.g.gcnt[g0 + k];
            }
        __syncthreads();
    }
    const float *gval = L.u.g.gval;
    const uint32_t *gcnt = L.u.g.gcnt;
    const uint32_t *gpos = L.u.g.w.gpos;
    const uint64_t in_list = (uint64_t)gpos[G - 1] + gcnt[G - 1];  // entries in the group list
    // the group holding entry e - 1 and how many of its entries come before e
    auto cut = [&](uint64_t e, int &gk, uint32_t &ck) {
        int lo = 0, hi = G - 1;  // last group with gpos <= e - 1
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if ((uint64_t)gpos[mid] <= e - 1) lo = mid;
            else hi = mid - 1;
        }
        gk = lo;
        ck = (uint32_t)(e - gpos[lo]);
    };
    auto eterm = [&](float x) { return zexpf_nb(x - mx); };
    int sg = 0;
    int64_t sc = 0;
    uint64_t keep = (uint64_t)P.n;  // the reference's candidate count (V)
    if (P.top_p < 1.0f) {          // :215-227
        float total = 0.0f;
        if (tid == 0) L.cp.n = 0;
        __syncthreads();
        walk_block(gval, gcnt, gpos, G - 1, gcnt[G - 1], eterm, kWalkSum, 0.0f, total, &sg, &sc, L.wb, 0, &L.cp);
        __syncthreads();  // the checkpoints
        const float thr = P.top_p * total;
        // The crossing adds the same terms in the same order as the total, and
        // the running value never decreases: it lies past the last checkpoint
        // still below thr, from which the walk resumes with that value.
        int c = 0;
        for (int j = 1; j < L.cp.n; ++j)
            if (L.cp.v[j] < thr) c = j;
        float acc = L.cp.n > 0 ? L.cp.v[c] : 0.0f;
        const int gs = L.cp.n > 0 ? L.cp.g[c] : 0;
        const int64_t pos =
            walk_block(gval, gcnt, gpos, G - 1, gcnt[G - 1], eterm, kWalkReach, thr, acc, &sg, &sc, L.wb, gs);
        keep = pos >= 0 ? (uint64_t)pos + 1 : keep;
    }
    if (P.min_p > 0.0f) {  // :228-234: the first term below min_p within keep
        if (tid == 0) L.wb.first = G;
        __syncthreads();
        for (int g = tid; g < G; g += kThreads)
            if (gcnt[g] > 0 && (uint64_t)gpos[g] < keep && eterm(gval[g]) < P.min_p) atomicMin(&L.wb.first, g);
        __syncthreads();
        const int fg = L.wb.first;
        const uint64_t first = fg < G ? (uint64_t)gpos[fg] : in_list;  // past the list every term is below min_p
        if (first < keep) keep = first > 1 ? first : 1;
    }
    if (keep > in_list) keep = in_list;  // more only with NaN logits, outside the reference's contract
    // :236-242 temperature weights and their total over keep, then the draw (:270-275)
    int gk;
    uint32_t ck;
    cut(keep, gk, ck);
    const float inv_t = 1.0f / P.temp;
    auto wterm = [&](float x) { return zexpf_nb((x - mx) * inv_t); };
    float total = 0.0f;
    int gs = 0;
    if (inv_t == 1.0f && P.top_p < 1.0f) {
        // (x - mx) * 1 is x - mx exactly: the weights are the top-p terms, and
        // their total over keep continues the top-p total from its last
        // checkpoint at or before the group holding entry keep - 1
        int c = -1;
        for (int j = 0; j < L.cp.n; ++j)
            if (L.cp.g[j] <= gk) c = j;
        if (c >= 0) {
            total = L.cp.v[c];
            gs = L.cp.g[c];
        }
    }
    walk_block(gval, gcnt, gpos, gk, ck, wterm, kWalkSum, 0.0f, total, &sg, &sc, L.wb, gs);
    const float u0 = P.uniforms[2 * row];
    float r = u0 * total;
    if (walk_block(gval, gcnt, gpos, gk, ck, wterm, kWalkDrop, 0.0f, r, &sg, &sc, L.wb) < 0) {
        sg = gk;  // none reaches r <= 0: the last kept entry
        sc = (int64_t)ck - 1;
    }
    // the entry's index among all entries of its value (equal groups are adjacent)
    const float vt = gval[sg];
    int64_t idx = sc;
    for (int g = sg - 1; g >= 0 && gval[g] == vt; --g) idx += gcnt[g];
    __syncthreads();  // every thread is done with the group list and gpos (their space: pbits, vbits)

    // 7. the drawn entry's id: the (idx+1)-th entry of value vt in id order.
    //    One read of the row counts each 4096-id tile's entries of value vt
    //    (kWholeBatch vectors in flight per thread); the tile that holds the
    //    entry is read again and ranked.
    const int ntile = (nvec + kThreads - 1) / kThreads;
    auto vhit = [&](const uint4 &raw, uint32_t mword, int q) -> uint32_t {  // entries of value vt in vector q
        float v[VEC];
        unpack<uint16_t>(raw, v);
        const int id0 = q * VEC;
        const uint32_t mb = HAS_MASK ? mword >> (id0 & 31) : 0xFFu;
        const uint32_t pb = HAS_PEN ? (L.u.pbits[id0 >> 5] >> (id0 & 31)) : 0u;
        uint32_t hit = 0u;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            if (id0 + e >= V) continue;
            float x = v[e];
            if (HAS_MASK && !((mb >> e) & 1u)) x = -INFINITY;
            if (!((pb >> e) & 1u) && x == vt) hit |= 1u << e;
        }
        if (HAS_PEN) hit |= (L.u.g.w.vbits[id0 >> 5] >> (id0 & 31)) & 0xFFu;  // penalized ones of value vt
        return hit;
    };
    for (int i = tid; i < ntile; i += kThreads) L.tcnt[i] = 0u;
    if (HAS_PEN) {  // penalized ids, and those whose penalized value is vt
        for (int i = tid; i < (V + 31) / 32; i += kThreads) {
            L.u.g.w.vbits[i] = 0u;
            L.u.pbits[i] = 0u;
        }
        __syncthreads();
        for (int p = tid; p < npen; p += kThreads)
            if (L.pval[p] == vt) atomicOr(&L.u.g.w.vbits[L.pid[p] >> 5], 1u << (L.pid[p] & 31));
#pragma unroll
        for (int s = 0; s < kOwnSlots; ++s)
            if (oid[s] != 0xFFFFFFFFu) atomicOr(&L.u.pbits[oid[s] >> 5], 1u << (oid[s] & 31));
    }
    __syncthreads();
    for (int t0 = 0; t0 < ntile; t0 += kWholeBatch) {
        uint4 raw[kWholeBatch];
        uint32_t mw[kWholeBatch];
#pragma unroll
        for (int j = 0; j < kWholeBatch; ++j) {  // every load first
            const int q = (t0 + j) * kThreads + tid;
            raw[j] = make_uint4(0u, 0u, 0u, 0u);
            mw[j] = 0u;
            if (q < nvec) {
                raw[j] = *reinterpret_cast<const uint4 *>(lrow + q * VEC);
                if (HAS_MASK) mw[j] = mrow[(q * VEC) >> 5];
            }
        }
#pragma unroll
        for (int j = 0; j < kWholeBatch; ++j) {
            const int q = (t0 + j) * kThreads + tid;
            uint32_t c = q < nvec ? (uint32_t)__popc(vhit(raw[j], mw[j], q)) : 0u;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) c += __shfl_xor(c, o);
            if (lane == 0 && c) atomicAdd(&L.tcnt[t0 + j], c);
        }
    }
    __syncthreads();
    int tj = -1;
    int64_t seen = 0;  // entries of value vt in the tiles before tj
    for (int j = 0; j < ntile; ++j) {
        if (seen + (int64_t)L.tcnt[j] > idx) {
            tj = j;
            break;
        }
        seen += L.tcnt[j];
    }
    if (tj >= 0) {  // uniform
        const int q = tj * kThreads + tid;
        uint32_t hit = 0u;
        if (q < nvec) hit = vhit(*reinterpret_cast<const uint4 *>(lrow + q * VEC), HAS_MASK ? mrow[(q * VEC) >> 5] : 0u, q);
        const uint32_t c = (uint32_t)__popc(hit);
        uint32_t cin = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t y = __shfl_up(cin, o);
            if (lane >= o) cin += y;
        }
        if (lane == 63) L.wsum[wid] = cin;
        __syncthreads();
        uint32_t before = cin - c;
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
            if (w < wid) before += L.wsum[w];
        const int64_t lo = seen + before;
        if (c && idx >= lo && idx < lo + c) {  // this thread holds it
            uint32_t h = hit;
            for (int64_t k = lo; k < idx; ++k) h &= h - 1u;
            L.tok = (uint32_t)(q * VEC + __ffs(h) - 1);
            L.found = 1;
        }
    }
    __syncthreads();
    if (tid == 0) {
        P.tok[row] = L.found ? L.tok : 0u;
        P.margin[row] = (P.n >= 2) ? mx - second : 10.0f;
        if (P.ndraws) P.ndraws[row] = 1;
        if (P.keep) P.keep[row] = (int32_t)keep;
        if (L.found) P.flags[row] = 0;  // settled here: the sorting pass skips it
    }
}

template <bool M, bool PN>
static hipError_t launch_whole_t(const ExactParams &P, int rows, hipStream_t st) {
    hipLaunchKernelGGL((whole_kernel<M, PN>), dim3(rows), dim3(kThreads), 0, st, P);
    return hipGetLastError();
}

hipError_t launch_whole(const ExactParams &P, int rows, hipStream_t st) {
    const bool m = P.src.mask != nullptr;
    const bool p = (P.src.hist != nullptr) || (P.src.edit_ids != nullptr);
    if (m && p) return launch_whole_t<true, true>(P, rows, st);
    if (m) return launch_whole_t<true, false>(P, rows, st);
    if (p) return launch_whole_t<false, true>(P, rows, st);
    return launch_whole_t<false, false>(P, rows, st);
}

}  // namespace zi
