// zi_exact.hip -- exact whole-order sampling: Sampler.sampleWithMargin
// (src/sampler.zig:190-276) for rows whose candidate list is longer than the
// 256-entry machinery holds: top_k = 0 / top_k >= V rows whose keep the
// prefix pass could not settle (the k = V std.mem.sort branch, :198-202), and
// 256 < top_k < V (the insertion branch, :203-209; both give the order
// (value desc, id asc), so the candidates are the first n of that order).
//
// One 512-thread workgroup per row:
//  A. penalty table for the whole row in LDS.
//  B. sort keys ~okey(x) of every entry in id order (one read of the row),
//     with the row max and second value (c[0].v, c[1].v).
//  C. stable LSD radix sort of (key, id) over 4 digits of 8 bits, in global
//     scratch, of the entries at or above a value threshold (id order in, so
//     equal values stay in ascending id order, the stable sort's tie rule).
//     Each tile of 4096 entries is ranked with wave-level digit matching,
//     staged in LDS by digit and written out in runs.  The threshold keeps a
//     superset of what can reach keep: with min_p > 0, keep never passes the
//     first term below min_p (stage 1); with top_p < 1, a term below 2^-24
//     never changes the sequential total (every prefix is >= the first term,
//     1), so neither it nor any later term is inside keep (stage 2).
//  D. keep: stage 1 settles it from the min-p prefix when top_p >= 1 or when
//     the bounded total places the top-p crossing; otherwise stage 2 runs the
//     reference's sequential f32 sums in its order on one lane, over
//     exponentials that all lanes compute tile by tile into LDS.
//  E. temperature, XTC and the draw over the kept prefix, likewise.
#include "zi_launch.hpp"
#include "zi_rowpass.hpp"

namespace zi {

constexpr int kRounds = 8;                  // sort: entries per thread per tile
constexpr int kTile = kThreads * kRounds;   // 4096
constexpr int kSeqTile = 4096;              // sequential phase: terms per LDS tile
constexpr uint32_t kNoKey = 0xFFFFFFFFu;    // ~okey(x) of no float (okey never 0)

struct ExactPenLds {
    uint32_t bits[kMaxVocab / 32];
    uint32_t key[kHashMax];
    uint32_t cnt[kHashMax];
    float delta[kHashMax];
};
struct ExactSortLds {
    uint32_t wcnt[2][kWaves][256];  // per-wave digit counts, two tiles in flight
    uint32_t tpre[256];             // tile: first staged slot of each digit
    uint32_t tbase[256];            // tile: first global slot of each digit
    uint32_t skey[kTile];
    uint32_t sid[kTile];
};
struct ExactSeqLds {
    alignas(16) float t[kSeqTile];
};
union ExactLds {
    ExactPenLds pen;
    ExactSortLds sort;
    ExactSeqLds seq;
};

// Lanes of this wave holding a valid entry with this lane's 8-bit digit (0
// for an invalid lane).
__device__ __forceinline__ uint64_t wave_match8(bool valid, uint32_t d) {
    uint64_t m = ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t bb = ballot(valid && bit);
        m &= bit ? bb : ~bb;
    }
    return valid ? m : 0ull;
}

// Whole-row penalty lookup: the bitset marks penalized / edited ids, the hash
// holds their window counts and edit deltas (the same table as the chunk
// pass, over all V ids).
__device__ __forceinline__ float exact_penalize(const ExactPenLds &t, const RowSource &a, int hs_log2, uint32_t id,
                                                float x) {
    if (!((t.bits[id >> 5] >> (id & 31)) & 1u)) return x;
    const uint32_t m = (1u << hs_log2) - 1;
    uint32_t h = hash_slot(id, hs_log2);
    while (t.key[h] != id + 1) h = (h + 1) & m;  // present: every marked id was inserted
    return pen_apply(x, t.cnt[h], t.delta[h], a);
}

// The VEC logits of vector q of the row after mask and penalties; ids >= V
// become NaN.
template <typename T, bool HAS_MASK, bool HAS_PEN, bool CAP>
__device__ __forceinline__ void exact_vector(const RowSource &a, int row, const ExactPenLds &t, int hs_log2, int q,
                                             float (&v)[VecTraits<T>::VEC]) {
    constexpr int VEC = VecTraits<T>::VEC;
    const T *base = reinterpret_cast<const T *>(a.logits) + (int64_t)row * a.ld;
    const int id0 = q * VEC;
    unpack<T>(*reinterpret_cast<const uint4 *>(base + id0), v);
    if constexpr (CAP) softcap_vec<VEC>(a, id0, v);
    if (HAS_MASK) {
        const uint32_t mb = a.mask[(int64_t)row * a.mask_ld + (id0 >> 5)] >> (id0 & 31);
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = ((mb >> e) & 1u) ? v[e] : -INFINITY;
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
        if (id0 + e >= a.V) v[e] = __builtin_nanf("");
        else if (HAS_PEN) v[e] = exact_penalize(t, a, hs_log2, (uint32_t)(id0 + e), v[e]);
    }
}

__device__ __forceinline__ void top2_merge_f(float &t1, float &t2, float o1, float o2) {
    t2 = fmaxf(fmaxf(t2, o2), fminf(t1, o1));
    t1 = fmaxf(t1, o1);
}

// Runs tiles of terms [i0, i1) through LDS: every thread computes term(i)
// for its share of the tile, then thread 0 runs cons(tile, count, base),
// which returns true to stop.  Uniform control flow; two barriers per tile.
template <class Term, class Cons>
__device__ __forceinline__ void seq_tiles(int i0, int i1, float *buf, int *s_stop, Term term, Cons cons) {
    for (int b = i0; b < i1; b += kSeqTile) {
        const int cnt = min(kSeqTile, i1 - b);
        for (int j = threadIdx.x; j < cnt; j += kThreads) buf[j] = term(b + j);
        __syncthreads();
        if (threadIdx.x == 0) *s_stop = cons(buf, cnt, b) ? 1 : 0;
        __syncthreads();
        const int stop = *s_stop;
        __syncthreads();  // *s_stop read by all before thread 0 may write it again
        if (stop) break;
    }
}

// Lane-serial scans over one LDS tile (16-byte aligned, c terms), carrying
// their running value across tiles; each returns the index within the tile
// where it stops, or -1.  Sixteen terms are loaded per step so that the LDS
// round trips overlap the dependent f32 chain; the running values are
// monotone, so a block is tested by its last value.
//   reach: acc = fl(acc + s_j), stop at the first acc >= thr
//   drop:  r = fl(r - s_j), stop at the first r <= 0
//   below: stop at the first s_j < lim (no running value)
__device__ __forceinline__ int tile_reach(const float *s, int c, float thr, float &acc) {
    int j = 0;
    for (; j + 16 <= c; j += 16) {
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 f = *reinterpret_cast<const float4 *>(s + j + 4 * q);
            v[4 * q] = f.x;
            v[4 * q + 1] = f.y;
            v[4 * q + 2] = f.z;
            v[4 * q + 3] = f.w;
        }
        float p[16];
        p[0] = acc + v[0];
#pragma unroll
        for (int q = 1; q < 16; ++q) p[q] = p[q - 1] + v[q];
        if (p[15] >= thr) {
#pragma unroll
            for (int q = 0; q < 16; ++q)
                if (p[q] >= thr) return j + q;
        }
        acc = p[15];
    }
    for (; j < c; ++j) {
        acc = acc + s[j];
        if (acc >= thr) return j;
    }
    return -1;
}

__device__ __forceinline__ int tile_drop(const float *s, int c, float &r) {
    int j = 0;
    for (; j + 16 <= c; j += 16) {
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 f = *reinterpret_cast<const float4 *>(s + j + 4 * q);
            v[4 * q] = f.x;
            v[4 * q + 1] = f.y;
            v[4 * q + 2] = f.z;
            v[4 * q + 3] = f.w;
        }
        float p[16];
        p[0] = r - v[0];
#pragma unroll
        for (int q = 1; q < 16; ++q) p[q] = p[q - 1] - v[q];
        if (p[15] <= 0.0f) {
#pragma unroll
            for (int q = 0; q < 16; ++q)
                if (p[q] <= 0.0f) return j + q;
        }
        r = p[15];
    }
    for (; j < c; ++j) {
        r = r - s[j];
        if (r <= 0.0f) return j;
    }
    return -1;
}

template <class Pred>
__device__ __forceinline__ int tile_first(const float *s, int c, Pred pred) {
    int j = 0;
    for (; j + 16 <= c; j += 16) {
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 f = *reinterpret_cast<const float4 *>(s + j + 4 * q);
            v[4 * q] = f.x;
            v[4 * q + 1] = f.y;
            v[4 * q + 2] = f.z;
            v[4 * q + 3] = f.w;
        }
        bool any = false;
#pragma unroll
        for (int q = 0; q < 16; ++q) any |= pred(v[q]);
        if (any) {
#pragma unroll
            for (int q = 0; q < 16; ++q)
                if (pred(v[q])) return j + q;
        }
    }
    for (; j < c; ++j)
        if (pred(s[j])) return j;
    return -1;
}

// Sort buffers of one row: K holds every entry's key in id order (written
// once); the sort alternates between the pairs (ka, ia) and (kb, ib).
struct SortBufs {
    uint32_t *K, *ka, *ia, *kb, *ib;
};

// Stable LSD radix sort (4 digits of 8 bits) of the entries of K with key <=
// thr, ids ascending within equal keys.  Returns the entry count m; sorted
// keys / ids in *sk / *si.  Uses sm.sort; barriers throughout.
__device__ int exact_sort(const SortBufs &B, int V, uint32_t thr, ExactSortLds &ss, uint32_t (*hist)[256], int *s_m,
                          int *s_tcnt, const uint32_t **sk, const uint32_t **si) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    for (int i = tid; i < 4 * 256; i += kThreads) (&hist[0][0])[i] = 0u;
    if (tid == 0) *s_m = 0;
    __syncthreads();
    int mine = 0;
    for (int i = tid; i < V; i += kThreads) {
        const uint32_t key = B.K[i];
        if (key <= thr) {
            ++mine;
#pragma unroll
            for (int dg = 0; dg < 4; ++dg) atomicAdd(&hist[dg][(key >> (8 * dg)) & 255u], 1u);
        }
    }
    if (mine) atomicAdd(s_m, mine);
    __syncthreads();
    const int m = *s_m;

    const uint32_t *ck = B.K, *ci = nullptr;  // input keys / ids (pass 0: ids implicit)
    uint32_t *ok = B.ka, *oi = B.ia;          // output keys / ids
    for (int pass = 0; pass < 4; ++pass) {
        const int sh = 8 * pass;
        const int len = pass == 0 ? V : m;
        // a digit shared by every entry leaves the order as it is
        if (pass > 0 && __syncthreads_or(tid < 256 && hist[pass][tid] == (uint32_t)m)) continue;
        // wave 0 keeps the running global start of digits 4*lane .. 4*lane+3
        uint32_t gb[4];
        if (wid == 0) {
            uint32_t h[4], s = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                h[c] = hist[pass][4 * lane + c];
                s += h[c];
            }
            uint32_t incl = s;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t y = __shfl_up(incl, o);
                if (lane >= o) incl += y;
            }
            uint32_t ex = incl - s;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                gb[c] = ex;
                ex += h[c];
            }
        }
        for (int i = tid; i < 2 * kWaves * 256; i += kThreads) (&ss.wcnt[0][0][0])[i] = 0u;
        __syncthreads();
        int buf = 0;
        for (int t0 = 0; t0 < len; t0 += kTile) {
            uint32_t kk[kRounds], ii[kRounds], rk[kRounds];
            // rank within the wave, round by round (positions in order)
#pragma unroll
            for (int r = 0; r < kRounds; ++r) {
                const int pos = t0 + wid * (64 * kRounds) + r * 64 + lane;
                bool valid = pos < len;
                const uint32_t key = valid ? ck[pos] : kNoKey;
                const uint32_t id = pass == 0 ? (uint32_t)pos : (valid ? ci[pos] : 0u);
                if (pass == 0) valid = valid && key <= thr;
                kk[r] = key;
                ii[r] = id;
                rk[r] = 0xFFFFFFFFu;
                if (ballot(valid) == 0ull) continue;  // wave-uniform: nothing to rank
                const uint32_t d = (key >> sh) & 255u;
                const uint64_t peers = wave_match8(valid, d);
                const uint32_t below = (uint32_t)lanes_below(peers);
                const uint32_t before = valid ? ss.wcnt[buf][wid][d] : 0u;
                wave_sync();
                if (valid && below == 0) ss.wcnt[buf][wid][d] = before + (uint32_t)__popcll(peers);
                wave_sync();
                if (valid) rk[r] = before + below;
            }
            __syncthreads();
            if (wid == 0) {  // wave prefixes, tile digit starts, global starts
                uint32_t tot[4], s = 0;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int d = 4 * lane + c;
                    uint32_t acc = 0;
#pragma unroll
                    for (int w = 0; w < kWaves; ++w) {
                        const uint32_t x = ss.wcnt[buf][w][d];
                        ss.wcnt[buf][w][d] = acc;
                        acc += x;
                    }
                    tot[c] = acc;
                    s += acc;
                }
                uint32_t incl = s;
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const uint32_t y = __shfl_up(incl, o);
                    if (lane >= o) incl += y;
                }
                uint32_t ex = incl - s;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    ss.tpre[4 * lane + c] = ex;
                    ss.tbase[4 * lane + c] = gb[c];
                    gb[c] += tot[c];
                    ex += tot[c];
                }
                if (lane == 63) *s_tcnt = (int)incl;
            } else {  // the other buffer is idle: clear it for the next tile
                for (int i = tid - 64; i < kWaves * 256; i += kThreads - 64) (&ss.wcnt[buf ^ 1][0][0])[i] = 0u;
            }
            __syncthreads();
#pragma unroll
            for (int r = 0; r < kRounds; ++r) {
                if (rk[r] != 0xFFFFFFFFu) {
                    const uint32_t d = (kk[r] >> sh) & 255u;
                    const uint32_t lp = ss.tpre[d] + ss.wcnt[buf][wid][d] + rk[r];
                    ss.skey[lp] = kk[r];
                    ss.sid[lp] = ii[r];
                }
            }
            __syncthreads();
            const int tcnt = *s_tcnt;
            for (int j = tid; j < tcnt; j += kThreads) {  // consecutive slots of a digit: one run
                const uint32_t key = ss.skey[j];
                const uint32_t d = (key >> sh) & 255u;
                const uint32_t dst = ss.tbase[d] + (uint32_t)j - ss.tpre[d];
                ok[dst] = key;
                oi[dst] = ss.sid[j];
            }
            buf ^= 1;
        }
        __syncthreads();  // this pass's stores are visible to the next pass's loads
        ck = ok;
        ci = oi;
        if (ok == B.ka) {
            ok = B.kb;
            oi = B.ib;
        } else {
            ok = B.ka;
            oi = B.ia;
        }
    }
    *sk = ck;
    *si = ci;
    return m;
}

// Largest sort key admitted for entries x with fl(x - mx) >= dlo: the key of
// a value a little below mx + dlo (a superset is harmless; the tail tests
// each term itself).
__device__ __forceinline__ uint32_t key_floor(float mx, float dlo) {
    const double v = (double)mx + (double)dlo - (fabs((double)mx) + fabs((double)dlo)) * 1e-6;
    float f = (float)v;
    if ((double)f > v) f = __uint_as_float(__float_as_uint(f) + (f > 0.0f ? -1 : 1));  // round toward -inf
    return ~okey(f);
}

template <typename T, bool HAS_MASK, bool HAS_PEN, bool CAP>
__global__ __launch_bounds__(kThreads) void exact_kernel(ExactParams P) {
    __shared__ ExactLds sm;
    __shared__ uint32_t s_hist[4][256];  // counts of each digit over the entries being sorted
    __shared__ float s_t1[kWaves], s_t2[kWaves];
    __shared__ int s_m, s_stop, s_tcnt;
    __shared__ int s_i[4];
    __shared__ float s_f[2];

    constexpr int VEC = VecTraits<T>::VEC;
    const RowSource &a = P.src;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int row = blockIdx.x;
    if (P.flags && P.flags[row] == 0) return;  // settled by the prefix pass (uniform)
    const int V = a.V;
    const int nvec = (V + VEC - 1) / VEC;

    // ---- A: penalty table, row max and second value
    RowPen rp = row_pen(a, row);
    if (HAS_PEN) {
        for (int i = tid; i < (V + 31) / 32; i += kThreads) sm.pen.bits[i] = 0u;
        for (int i = tid; i < kHashMax; i += kThreads) {
            sm.pen.key[i] = 0u;
            sm.pen.cnt[i] = 0u;
            sm.pen.delta[i] = 0.0f;
        }
        __syncthreads();
        for (int i = tid; i < rp.nw; i += kThreads) {
            const uint32_t id = rp.win_ptr[i];
            if (id < (uint32_t)V) {
                atomicOr(&sm.pen.bits[id >> 5], 1u << (id & 31));
                atomicAdd(&sm.pen.cnt[pen_insert(sm.pen, id, rp.hs_log2)], 1u);
            }
        }
        for (int i = tid; i < rp.ne; i += kThreads) {
            const uint32_t id = rp.eid[i];
            if (id < (uint32_t)V) {
                atomicOr(&sm.pen.bits[id >> 5], 1u << (id & 31));
                sm.pen.delta[pen_insert(sm.pen, id, rp.hs_log2)] = rp.edl[i];
            }
        }
        __syncthreads();
    }
    SortBufs B;
    {
        const int64_t o = (int64_t)row * P.ldk;
        B.K = P.keys + o;
        B.ka = P.key0 + o;
        B.ia = P.id0 + o;
        B.kb = P.key1 + o;
        B.ib = P.id1 + o;
    }
    // ---- B: keys ~okey(x) in id order (kNoKey for NaN), max and second value
    float t1 = -INFINITY, t2 = -INFINITY;
    for (int q = tid; q < nvec; q += kThreads) {
        float v[VEC];
        exact_vector<T, HAS_MASK, HAS_PEN, CAP>(a, row, sm.pen, rp.hs_log2, q, v);
        uint32_t kk[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            const bool ok = v[e] == v[e];
            kk[e] = ok ? ~okey(v[e]) : kNoKey;
            if (ok) top2_merge_f(t1, t2, v[e], -INFINITY);
        }
#pragma unroll
        for (int e = 0; e < VEC; e += 4)  // slots past V (up to the row's key stride) hold kNoKey
            *reinterpret_cast<uint4 *>(B.K + q * VEC + e) = make_uint4(kk[e], kk[e + 1], kk[e + 2], kk[e + 3]);
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) top2_merge_f(t1, t2, __shfl_xor(t1, m), __shfl_xor(t2, m));
    if (lane == 0) {
        s_t1[wid] = t1;
        s_t2[wid] = t2;
    }
    __syncthreads();
    float mx = s_t1[0], second = s_t2[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) top2_merge_f(mx, second, s_t1[w], s_t2[w]);
    const bool fin = __builtin_isfinite(mx);
    const int n = P.n;
    const float u0 = P.uniforms[2 * row], u1 = P.uniforms[2 * row + 1];
    float *tb = sm.seq.t;
    const float inv_t = 1.0f / P.temp;
    const uint32_t *sk = nullptr, *si = nullptr;  // sorted keys / ids
    auto value = [&](int i) { return okey_inv(~sk[i]); };
    auto eterm = [&](int i) { return exp32(value(i) - mx); };
    auto wterm = [&](int i) { return exp32((value(i) - mx) * inv_t); };

    // ---- C/D: sort a prefix of the order, then settle keep (:215-234).
    // Stage 1 (min_p > 0): keep never passes the first term below min_p, so
    // only entries with fl(x - mx) >= ln(min_p) are sorted; keep is settled
    // there when top_p >= 1, or when the bounded total (prefix pass, k = V)
    // places the top-p crossing.  Stage 2: every entry whose term can change
    // the sequential sums is sorted and the reference's sums run exactly.
    const bool bounds = P.g_stat != nullptr && P.n_all == V;
    const float dlo_minp = fminf(logf(P.min_p) - 0.01f, 0.0f);
    int m = 0, mp = 0, keep = 0;
    for (int stage = (fin && P.min_p > 0.0f && (P.top_p >= 1.0f || bounds)) ? 1 : 2; stage <= 2; ++stage) {
        uint32_t thr = kNoKey - 1;  // every non-NaN entry
        if (stage == 1) thr = key_floor(mx, dlo_minp);
        else if (fin && P.top_p < 1.0f) thr = key_floor(mx, -16.75f);  // below ln(2^-24) = -16.636
        else if (fin && P.min_p > 0.0f) thr = key_floor(mx, dlo_minp);
        m = exact_sort(B, V, thr, sm.sort, s_hist, &s_m, &s_tcnt, &sk, &si);
        if (m == 0) break;
        mp = min(m, n);
        if (stage == 1) {
            // first term below min_p inside the sorted prefix (else the first
            // entry past it, whose term is below min_p by construction)
            const float lim = P.min_p;
            int first = -1;
            seq_tiles(0, mp, tb, &s_stop, eterm, [&](const float *s, int c, int b) {
                const int j = tile_first(s, c, [lim](float x) { return x < lim; });
                if (j >= 0) first = b + j;
                return j >= 0;
            });
            int kp_lo = m + 1, kp_hi = m + 1;  // 1 + first crossing index; m + 1: past the prefix
            float thr_lo = 0.0f, thr_hi = 0.0f;
            bool ok_bounds = true;
            if (P.top_p < 1.0f && tid == 0) {
                const int G = a.G;
                const double *gs = P.g_stat + (int64_t)row * G * 3;
                double Mr = -INFINITY;
                for (int g = 0; g < G; ++g) Mr = fmax(Mr, gs[g * 3]);
                double Z = 0.0;
                for (int g = 0; g < G; ++g)
                    if (gs[g * 3] != -INFINITY) Z += gs[g * 3 + 1] * exp(gs[g * 3] - Mr);
                const double tot = Z * exp(Mr - (double)mx);
                const double nu = (double)(V - 1) * 0x1p-24;
                const double gam = nu / (1.0 - nu) + 1e-4;
                const double dl = tot * (1.0 - gam), dh = tot * (1.0 + gam);
                ok_bounds = tot >= 0.5 && tot < 1e30;
                float lo = (float)dl, hi = (float)dh;
                if ((double)lo > dl) lo = __uint_as_float(__float_as_uint(lo) - 1u);
                if ((double)hi < dh) hi = __uint_as_float(__float_as_uint(hi) + 1u);
                thr_lo = P.top_p * lo;
                thr_hi = P.top_p * hi;
            }
            if (P.top_p < 1.0f) {
                float acc = 0.0f;
                int f_lo = -1, f_hi = -1;
                seq_tiles(0, mp, tb, &s_stop, eterm, [&](const float *s, int c, int b) {
                    for (int j = 0; j < c; ++j) {  // one chain, two thresholds
                        acc = acc + s[j];
                        if (f_lo < 0 && acc >= thr_lo) f_lo = b + j;
                        if (acc >= thr_hi) {
                            f_hi = b + j;
                            return true;
                        }
                    }
                    return false;
                });
                if (f_lo >= 0) kp_lo = f_lo + 1;
                if (f_hi >= 0) kp_hi = f_hi + 1;
            }
            int res = -1;  // settled keep, or -1
            if (tid == 0) {
                const int fl = first >= 0 ? first : m;  // <= m
                if (P.top_p >= 1.0f) res = fl < n ? max(fl, 1) : n;
                else if (ok_bounds && fl <= kp_lo) res = max(fl, 1);  // keep = min(keep_p, fl)
                else if (ok_bounds && kp_lo == kp_hi && kp_lo <= m) res = kp_lo;
                s_i[0] = res;
            }
            __syncthreads();
            res = s_i[0];
            __syncthreads();
            if (res > 0) {
                keep = min(res, mp);
                break;
            }
            continue;
        }
        // stage 2: top-p on untempered terms, exact (:215-227)
        int keep_p = n;
        if (P.top_p < 1.0f) {
            float total = 0.0f;
            seq_tiles(0, mp, tb, &s_stop, eterm, [&](const float *s, int c, int) {
                total = lane_sum(s, 0, c, total);
                return false;
            });
            float thr_p = 0.0f;
            if (tid == 0) thr_p = P.top_p * total;
            float acc = 0.0f;
            int found = -1;
            seq_tiles(0, mp, tb, &s_stop, eterm, [&](const float *s, int c, int b) {
                const int j = tile_reach(s, c, thr_p, acc);
                if (j >= 0) found = b + j;
                return j >= 0;
            });
            if (tid == 0) s_i[0] = found >= 0 ? found + 1 : n;
            __syncthreads();
            keep_p = s_i[0];
            __syncthreads();
        }
        // min-p (:228-234): first i < keep_p with e_i < min_p
        keep = keep_p;
        if (P.min_p > 0.0f) {
            int first = -1;
            const float lim = P.min_p;
            seq_tiles(0, min(keep_p, mp), tb, &s_stop, eterm, [&](const float *s, int c, int b) {
                const int j = tile_first(s, c, [lim](float x) { return x < lim; });
                if (j >= 0) first = b + j;
                return j >= 0;
            });
            if (tid == 0) s_i[0] = first >= 0 ? max(first, 1) : (keep_p > mp ? max(mp, 1) : keep_p);
            __syncthreads();
            keep = s_i[0];
            __syncthreads();
        }
        keep = min(keep, mp);  // entries past mp exist only out of contract (NaN logits)
    }
    if (m == 0) {  // no selectable logit (every entry NaN): outside the reference contract
        if (tid == 0) {
            P.tok[row] = 0u;
            P.margin[row] = 10.0f;
            if (P.ndraws) P.ndraws[row] = 0;
            if (P.keep) P.keep[row] = 0;
        }
        return;
    }

    // ---- E: temperature weights and their sequential total (:236-242)
    float total = 0.0f;
    seq_tiles(0, keep, tb, &s_stop, wterm, [&](const float *s, int c, int) {
        total = lane_sum(s, 0, c, total);
        return false;
    });
    if (tid == 0) s_f[0] = total;
    __syncthreads();
    total = s_f[0];
    __syncthreads();

    // XTC (:244-268)
    int start = 0, draws = 0;
    float umain = u0;
    if (P.xtc_p > 0.0f && P.xtc_thr <= 0.5f && keep >= 2 && total > 0.0f) {
        draws = 1;
        umain = u1;
        if (u0 <= P.xtc_p) {
            const float inv_tot = 1.0f / total;
            int f = -1;
            const float thr = P.xtc_thr;
            seq_tiles(0, keep, tb, &s_stop, wterm, [&](const float *s, int c, int b) {
                const int j = tile_first(s, c, [inv_tot, thr](float x) { return !(x * inv_tot >= thr); });
                if (j >= 0) f = b + j;
                return j >= 0;
            });
            if (tid == 0) s_i[0] = f >= 0 ? f : keep;
            __syncthreads();
            const int ff = s_i[0];
            __syncthreads();
            const int pos_last = ff > 0 ? ff - 1 : 0;
            if (keep - pos_last >= max(1, P.xtc_min_keep) && pos_last > 0) {
                start = pos_last;
                float t = 0.0f;
                seq_tiles(start, keep, tb, &s_stop, wterm, [&](const float *s, int c, int) {
                    t = lane_sum(s, 0, c, t);
                    return false;
                });
                if (tid == 0) s_f[0] = t;
                __syncthreads();
                total = s_f[0];
                __syncthreads();
            }
        }
    }
    draws += 1;

    // draw (:270-275)
    float r = umain * total;
    int pick = -1;
    seq_tiles(start, keep, tb, &s_stop, wterm, [&](const float *s, int c, int b) {
        const int j = tile_drop(s, c, r);
        if (j >= 0) pick = b + j;
        return j >= 0;
    });
    if (tid == 0) {
        if (pick < 0) pick = keep - 1;
        P.tok[row] = si[pick];
        P.margin[row] = (n >= 2) ? mx - second : 10.0f;
        if (P.ndraws) P.ndraws[row] = draws;
        if (P.keep) P.keep[row] = keep;
    }
    if (P.cand_ids) {
        const int n_out = min(keep, P.cand_ld);
        for (int i = tid; i < n_out; i += kThreads) {
            const int64_t o = (int64_t)row * P.cand_ld + i;
            P.cand_ids[o] = si[i];
            if (P.cand_vals) P.cand_vals[o] = value(i);
            if (P.probs) P.probs[o] = (i >= start) ? wterm(i) / total : 0.0f;
        }
    }
}

template <typename T, bool M, bool PN>
static hipError_t launch_exact_t(const ExactParams &P, int rows, hipStream_t st) {
    if (P.src.cap > 0.0f) hipLaunchKernelGGL((exact_kernel<T, M, PN, true>), dim3(rows), dim3(kThreads), 0, st, P);
    else hipLaunchKernelGGL((exact_kernel<T, M, PN, false>), dim3(rows), dim3(kThreads), 0, st, P);
    return hipGetLastError();
}

template <typename T>
static hipError_t launch_exact_d(const ExactParams &P, int rows, hipStream_t st) {
    const bool m = P.src.mask != nullptr;
    const bool p = (P.src.hist != nullptr) || (P.src.edit_ids != nullptr);
    if (m && p) return launch_exact_t<T, true, true>(P, rows, st);
    if (m) return launch_exact_t<T, true, false>(P, rows, st);
    if (p) return launch_exact_t<T, false, true>(P, rows, st);
    return launch_exact_t<T, false, false>(P, rows, st);
}

hipError_t launch_exact(const ExactParams &P, int dtype, int rows, hipStream_t st) {
    return dtype == 0 ? launch_exact_d<float>(P, rows, st) : launch_exact_d<uint16_t>(P, rows, st);
}

}  // namespace zi
