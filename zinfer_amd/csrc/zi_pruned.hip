// zi_pruned.hip -- Sampler.sampleWithMargin (src/sampler.zig:190-276) on
// pruned-vocabulary rows.
//
// The reference's pruned lm_head (src/model.zig:2036-2140) scores the
// vocabulary coarsely in groups of 8 ids, keeps 64 fixed groups plus the 512
// best others, fills the whole logit row with -inf (:2127-2128) and computes
// only the kept groups (prunedFineWorker, :1144-1160).  Here the -inf fill is
// never written: a row is read only at its listed groups, and every other id
// is -inf by construction.  One 512-thread workgroup per row:
//  1. the group list, deduplicated through an LDS bitset, and each group's 8
//     logits (32 B for f32, 16 B for bf16 per load pair);
//  2. mask, then penalties and edits from an LDS hash filled with the window
//     ids that lie in listed groups (on -inf ids a penalty or an edit leaves
//     -inf, so the others need nothing);
//  3. temp <= 0: the reference argmax (2x8 lane classes, sampler.zig:553-610)
//     over the virtual row; else the exact top-k of the finite entries
//     (threshold from the lane maxima, candidates ranked by counting; an
//     exact 64-bit radix select when ties leave too many candidates), padded
//     to k with the lowest ids whose value is -inf, where the reference's
//     (value desc, id asc) order puts them;
//  4. the reference tail on the k candidates (zi_tail.hpp).
#include "zi_launch.hpp"
#include "zi_rowpass.hpp"
#include "zi_tail.hpp"

namespace zi {

constexpr int kMaxGroups = kMaxGroupsHost;
constexpr int kGroupsPerThread = kMaxGroups / kThreads;
constexpr int kEntries = kGroupsPerThread * 8;  // logits per thread
constexpr int kPrCand = 1024;                   // candidates ranked by counting
constexpr int kGroupWords = kMaxVocab / 8 / 32;
constexpr uint32_t kNoGroup = 0xFFFFFFFFu;
static_assert(kMaxGroups % kThreads == 0, "groups per thread");

struct PrunedLds {
    uint32_t gbits[kGroupWords];  // listed groups
    uint32_t pbits[kMaxVocab / 32];  // ids with a penalty-window occurrence or an edit
    uint32_t key[kHashMax];       // penalty hash over the listed ids (id + 1; 0 = empty)
    uint32_t cnt[kHashMax];
    float delta[kHashMax];
    uint32_t uni[kThreads];
    uint64_t ckeys[kPrCand];
    float cvals[kPrCand];
    uint32_t hist[256];
    uint64_t okey[kMaxTopK];
    float oval[kMaxTopK];
    uint32_t fid[kMaxTopK];  // finite ids ascending (rows with fewer than k)
    TailLds tl;
    uint64_t cls[16];  // argmax: class-max keys
    float cls_v[16];   // the class winners' values (sign of zero kept)
    float tail_v[16];  // argmax: ids past the 16-lane body
    uint32_t s_tau;
    int s_cnt;
    uint64_t s_pref;
    int s_krem;
};

__device__ __forceinline__ bool group_listed(const uint32_t *gbits, uint32_t id) {
    const uint32_t g = id >> 3;
    return (gbits[g >> 5] >> (g & 31)) & 1u;
}

// Hash slot of `id`, or -1 when absent (the table holds < half its slots).
__device__ __forceinline__ int pen_find(const PrunedLds &s, uint32_t id, int hs_log2) {
    uint32_t h = hash_slot(id, hs_log2);
    const uint32_t m = (1u << hs_log2) - 1;
    for (int probe = 0; probe <= (int)m; ++probe) {
        const uint32_t k = s.key[h];
        if (k == id + 1) return (int)h;
        if (k == 0u) return -1;
        h = (h + 1) & m;
    }
    return -1;
}

// Appends every entry for which pred(i) holds to s.ckeys / s.cvals (up to
// kPrCand; the returned count may exceed it): one ballot per entry slot, the
// slots' offsets from their popcounts, one LDS atomic per wave.  Contains two
// barriers.
template <class Pred>
__device__ __forceinline__ int gather(PrunedLds &s, const float (&x)[kEntries], const uint32_t (&gid)[kGroupsPerThread],
                                      const bool (&wl)[kGroupsPerThread], Pred pred) {
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid == 0) s.s_cnt = 0;
    __syncthreads();
    uint64_t bs[kEntries];
    int tot = 0;
#pragma unroll
    for (int i = 0; i < kEntries; ++i) {
        bs[i] = wl[i >> 3] ? ballot(pred(i)) : 0ull;  // wl: wave-uniform
        tot += __popcll(bs[i]);
    }
    if (tot) {
        int base = 0;
        if (lane == 0) base = atomicAdd(&s.s_cnt, tot);
        int off = __shfl(base, 0);
#pragma unroll
        for (int i = 0; i < kEntries; ++i) {
            if (!bs[i]) continue;  // wave-uniform: most slots hold no candidate
            if ((bs[i] >> lane) & 1ull) {
                const int pos = off + lanes_below(bs[i]);
                if (pos < kPrCand) {
                    const uint32_t id = gid[i >> 3] * 8u + (uint32_t)(i & 7);
                    s.ckeys[pos] = ckey(x[i], id);
                    s.cvals[pos] = x[i];
                }
            }
            off += __popcll(bs[i]);
        }
    }
    __syncthreads();
    return s.s_cnt;
}

template <typename T, bool HAS_MASK, bool HAS_PEN>
__global__ __launch_bounds__(kThreads) void pruned_kernel(SampleParams P) {
    constexpr int VEC = VecTraits<T>::VEC;
    constexpr int NL = 8 / VEC;  // 16-byte loads per group
    __shared__ PrunedLds s;
    const RowSource &a = P.src;
    const int tid = threadIdx.x, lane = tid & 63;
    const int row = blockIdx.x;
    const uint32_t V = (uint32_t)a.V;
    const uint32_t ngt = (V + 7) / 8;  // groups of the vocabulary

    // Every load that does not need a group id goes out first, together with
    // the ids and their count (the id slots up to groups_ld, not up to the
    // count, so that the ids do not wait for it): one round trip; then the
    // logits, which need the ids.
    PenRegs pr;
    int hl_raw = 0, ne_raw = 0;
    if (HAS_PEN) {
        pen_prefetch(a, row, pr);
        int rr = row;
        asm volatile("" : "+v"(rr));  // vector loads: their waits are counted with the others
        if (row_pen_window_on(a)) hl_raw = a.hist_len[rr];
        if (a.edit_ids) ne_raw = a.edit_count[rr];
    }
    int ur = 2 * row;
    asm volatile("" : "+v"(ur));
    const float u0 = P.uniforms ? P.uniforms[ur] : 0.0f, u1 = P.uniforms ? P.uniforms[ur + 1] : 0.0f;
    const int gcap = min(P.groups_ld, kMaxGroups);
    uint32_t graw[kGroupsPerThread];
#pragma unroll
    for (int u = 0; u < kGroupsPerThread; ++u) {
        const int j = tid + u * kThreads;
        graw[u] = j < gcap ? P.groups[(int64_t)row * P.groups_ld + j] : kNoGroup;
    }
    int ng = P.group_count[row];
    ng = ng < 0 ? 0 : min(ng, gcap);
    uint32_t gid[kGroupsPerThread];
    const T *base = reinterpret_cast<const T *>(a.logits) + (int64_t)row * a.ld;
    uint4 raw[kGroupsPerThread][NL];
    uint32_t mw[kGroupsPerThread];
#pragma unroll
    for (int u = 0; u < kGroupsPerThread; ++u) {
        const int j = tid + u * kThreads;
        uint32_t g = j < ng ? graw[u] : kNoGroup;
        g = g < ngt ? g : kNoGroup;
        gid[u] = g;
        const uint32_t gl = g == kNoGroup ? 0u : g;  // loads stay in the row either way
#pragma unroll
        for (int q = 0; q < NL; ++q) raw[u][q] = *reinterpret_cast<const uint4 *>(base + gl * 8u + q * VEC);
        mw[u] = HAS_MASK ? a.mask[(int64_t)row * a.mask_ld + ((gl * 8u) >> 5)] : 0xFFFFFFFFu;
    }

    for (int i = tid; i < (int)((ngt + 31) / 32); i += kThreads) s.gbits[i] = 0u;
    RowPen rp;
    if (HAS_PEN) {
        rp = row_pen_from(a, row, hl_raw, ne_raw);
        pen_window(rp, pr);
        for (int i = tid; i < (1 << rp.hs_log2); i += kThreads) {
            s.key[i] = 0u;
            s.cnt[i] = 0u;
            s.delta[i] = 0.0f;
        }
        for (int i = tid; i < (int)((V + 31) / 32); i += kThreads) s.pbits[i] = 0u;
    }
    if (tid < 16) {
        s.cls[tid] = 0ull;
        s.tail_v[tid] = -INFINITY;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kGroupsPerThread; ++u) {  // a group listed twice is taken once
        if (gid[u] != kNoGroup) {
            const uint32_t bit = 1u << (gid[u] & 31);
            if (atomicOr(&s.gbits[gid[u] >> 5], bit) & bit) gid[u] = kNoGroup;
        }
    }
    // wl[u]: some lane of this wave holds a group in slot u (wave-uniform);
    // slots no lane holds are skipped by every per-entry loop
    bool wl[kGroupsPerThread];
#pragma unroll
    for (int u = 0; u < kGroupsPerThread; ++u) wl[u] = ballot(gid[u] != kNoGroup) != 0ull;
    __syncthreads();
    if (HAS_PEN) {
#pragma unroll
        for (int u = 0; u < kWinPerThread; ++u) {
            const uint32_t id = pr.w[u];
            if (id < V && group_listed(s.gbits, id)) {
                atomicAdd(&s.cnt[pen_insert(s, id, rp.hs_log2)], 1u);
                atomicOr(&s.pbits[id >> 5], 1u << (id & 31));
            }
        }
        if (pr.e < V && group_listed(s.gbits, pr.e)) {
            s.delta[pen_insert(s, pr.e, rp.hs_log2)] = pr.d;
            atomicOr(&s.pbits[pr.e >> 5], 1u << (pr.e & 31));
        }
        __syncthreads();
    }

    // values: mask (grammar.zig:446-479), penalty (sampler.zig:91-100), edits
    float x[kEntries];
#pragma unroll
    for (int u = 0; u < kGroupsPerThread; ++u) {
        if (!wl[u]) {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[u * 8 + e] = -INFINITY;
            continue;
        }
#pragma unroll
        for (int q = 0; q < NL; ++q) {
            float v[VEC];
            unpack<T>(raw[u][q], v);
#pragma unroll
            for (int e = 0; e < VEC; ++e) x[u * 8 + q * VEC + e] = v[e];
        }
        // the group's 8 penalty bits (one byte of a word: groups are 8-aligned)
        const uint32_t pb = (HAS_PEN && gid[u] != kNoGroup) ? (s.pbits[gid[u] >> 2] >> ((gid[u] & 3) * 8)) & 0xFFu : 0u;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t id = gid[u] * 8u + (uint32_t)e;
            float v = x[u * 8 + e];
            if (gid[u] == kNoGroup || id >= V) {
                v = -INFINITY;  // not an entry of the row
            } else {
                if (HAS_MASK && !((mw[u] >> (id & 31)) & 1u)) v = -INFINITY;
                if (HAS_PEN && ((pb >> e) & 1u)) {
                    const int h = pen_find(s, id, rp.hs_log2);
                    if (h >= 0) v = pen_apply(v, s.cnt[h], s.delta[h], a);
                }
            }
            x[u * 8 + e] = v;
        }
    }

    if (P.temp <= 0.0f) {
        // argmaxWithMargin (sampler.zig:553-610) over the virtual row, V >= 16:
        // the class of id i < 16*floor(V/16) is i & 15, each class keeps its
        // first maximum; -inf entries never change a class maximum, the
        // reduction or the tail, so only the finite entries take part.
        const uint32_t body = V & ~15u;
#pragma unroll
        for (int i = 0; i < kEntries; ++i) {
            if (!wl[i >> 3]) continue;
            const uint32_t id = gid[i >> 3] * 8u + (uint32_t)(i & 7);
            if (x[i] > -INFINITY) {
                if (id < body)
                    atomicMax(reinterpret_cast<unsigned long long *>(&s.cls[id & 15]),
                              (unsigned long long)ckey(x[i], id));
                else s.tail_v[id - body] = x[i];
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kEntries; ++i) {
            if (!wl[i >> 3]) continue;
            const uint32_t id = gid[i >> 3] * 8u + (uint32_t)(i & 7);
            if (x[i] > -INFINITY && id < body && s.cls[id & 15] == ckey(x[i], id)) s.cls_v[id & 15] = x[i];
        }
        __syncthreads();
        if (tid == 0) {
            float best = -INFINITY, second = -INFINITY;
            uint32_t best_id = 0;
            for (int j = 0; j < 8; ++j) {
                for (int h = 0; h < 2; ++h) {
                    const int c = j + 8 * h;
                    if (!s.cls[c]) continue;  // every entry of the class is -inf
                    const float v = s.cls_v[c];
                    if (v > best) {
                        second = best;
                        best = v;
                        best_id = ckey_id(s.cls[c]);
                    } else if (v > second) {
                        second = v;
                    }
                }
            }
            for (uint32_t t = 0; t < V - body; ++t) {
                const float v = s.tail_v[t];
                if (v > best) {
                    second = best;
                    best = v;
                    best_id = body + t;
                } else if (v > second) {
                    second = v;
                }
            }
            P.tok[row] = best_id;
            P.margin[row] = second > -INFINITY ? best - second : 10.0f;
            if (P.ndraws) P.ndraws[row] = 0;
        }
        return;
    }

    // ---- top-k of the finite entries (value desc, id asc)
    const int k = P.k;
    float m1 = -INFINITY;
#pragma unroll
    for (int i = 0; i < kEntries; ++i) m1 = x[i] > m1 ? x[i] : m1;  // NaN never enters
    const float tau = chunk_tau(m1, k, s.uni, &s.s_tau);
    int nc = gather(s, x, gid, wl, [&](int i) { return x[i] > -INFINITY && x[i] >= tau; });
    if (nc > kPrCand) {
        // Ties keep too many entries at the threshold: find the exact k-th
        // largest 64-bit key (keys are unique) one byte at a time.
        uint64_t pref = 0ull;
        int krem = k;
        for (int sh = 56; sh >= 0; sh -= 8) {
            if (tid < 256) s.hist[tid] = 0u;
            __syncthreads();
            const uint64_t hi = sh == 56 ? 0ull : (~0ull << (sh + 8));
#pragma unroll
            for (int i = 0; i < kEntries; ++i) {
                if (x[i] > -INFINITY) {
                    const uint64_t key = ckey(x[i], gid[i >> 3] * 8u + (uint32_t)(i & 7));
                    if ((key & hi) == pref) atomicAdd(&s.hist[(key >> sh) & 255u], 1u);
                }
            }
            __syncthreads();
            if (tid < 64) {
                // lane l holds bins 4l..4l+3; suffix sums over lanes find the
                // bin where the count from the top reaches krem
                uint32_t c[4];
#pragma unroll
                for (int b = 0; b < 4; ++b) c[b] = s.hist[4 * lane + b];
                const uint32_t own = c[0] + c[1] + c[2] + c[3];
                uint32_t suf = own;
#pragma unroll
                for (int off = 1; off < 64; off <<= 1) {
                    const uint32_t t = __shfl_down(suf, off);
                    if (lane + off < 64) suf += t;
                }
                const uint64_t hit = ballot(suf >= (uint32_t)krem);
                const int L = 63 - __clzll((long long)hit);  // hit is nonempty: lane 0 holds the total >= krem
                if (lane == L) {
                    uint32_t acc = suf - own;
                    int d = 4 * L;
                    for (int b = 3; b >= 0; --b) {
                        if (acc + c[b] >= (uint32_t)krem) {
                            d = 4 * L + b;
                            break;
                        }
                        acc += c[b];
                    }
                    s.s_pref = pref | ((uint64_t)d << sh);
                    s.s_krem = krem - (int)acc;
                }
            }
            __syncthreads();
            pref = s.s_pref;
            krem = s.s_krem;
        }
        nc = gather(s, x, gid, wl, [&](int i) {
            return x[i] > -INFINITY && ckey(x[i], gid[i >> 3] * 8u + (uint32_t)(i & 7)) >= pref;
        });
    }
    // rank by counting: the candidates' keys are distinct
    for (int i = tid; i < nc; i += kThreads) {
        const uint64_t key = s.ckeys[i];
        int r = 0;
#pragma unroll 8
        for (int j = 0; j < nc; ++j) r += s.ckeys[j] > key ? 1 : 0;
        if (r < k) {
            s.okey[r] = key;
            s.oval[r] = s.cvals[i];
        }
    }
    if (nc < k) {
        // Fewer than k finite entries (then every one is a candidate): the
        // list continues with the -inf ids in ascending order, i.e. the ids
        // missing from the finite set.  fid = the finite ids ascending; the
        // j-th missing id is j + #{t : fid[t] - t <= j}.
        for (int i = tid; i < nc; i += kThreads) {
            const uint32_t id = ckey_id(s.ckeys[i]);
            int r = 0;
            for (int j = 0; j < nc; ++j) r += ckey_id(s.ckeys[j]) < id ? 1 : 0;
            s.fid[r] = id;
        }
        __syncthreads();
        for (int j = tid; j < k - nc; j += kThreads) {
            int t = 0;
            for (int q = 0; q < nc; ++q) t += (int)(s.fid[q] - (uint32_t)q) <= j ? 1 : 0;
            const uint32_t id = (uint32_t)(j + t);
            s.okey[nc + j] = ckey(-INFINITY, id);
            s.oval[nc + j] = -INFINITY;
        }
    }
    __syncthreads();
    if (tid >= 64) return;  // the tail runs on wave 0 with all 64 lanes active
    sample_tail<false>(P, row, s.okey, s.oval, k, s.tl, u0, u1);
}

// One 512-thread workgroup per (row, 4096-id block): the block's listed
// groups from the row's list (an LDS bitset), then each thread writes one
// group of 8: copied when listed, -inf otherwise (src/model.zig:2127-2128 then
// :1156-1158).
template <typename T>
__global__ __launch_bounds__(kThreads) void pruned_fill_kernel(const T *src, T *dst, int64_t ld, int64_t dst_ld, int V,
                                                               const uint32_t *groups, const int32_t *group_count,
                                                               int groups_ld) {
    constexpr int VEC = VecTraits<T>::VEC;
    constexpr int NL = 8 / VEC;
    __shared__ uint32_t bits[kThreads / 32];
    const int tid = threadIdx.x, row = blockIdx.y;
    const uint32_t g0 = blockIdx.x * (uint32_t)kThreads;  // first group of this block
    const uint32_t ngt = ((uint32_t)V + 7) / 8;
    if (tid < kThreads / 32) bits[tid] = 0u;
    __syncthreads();
    int ng = group_count[row];
    ng = ng < 0 ? 0 : min(ng, min(groups_ld, kMaxGroups));
    for (int j = tid; j < ng; j += kThreads) {
        const uint32_t g = groups[(int64_t)row * groups_ld + j];
        if (g < ngt && g >= g0 && g < g0 + kThreads) atomicOr(&bits[(g - g0) >> 5], 1u << ((g - g0) & 31));
    }
    __syncthreads();
    const uint32_t g = g0 + tid;
    if (g >= ngt) return;
    const bool listed = (bits[tid >> 5] >> (tid & 31)) & 1u;
    const T *s = src + (int64_t)row * ld + g * 8u;
    T *d = dst + (int64_t)row * dst_ld + g * 8u;
    const uint32_t ninf = sizeof(T) == 4 ? 0xFF800000u : 0xFF80FF80u;  // -inf, as f32 or two bf16
#pragma unroll
    for (int q = 0; q < NL; ++q) {
        const uint4 v = listed ? *reinterpret_cast<const uint4 *>(s + q * VEC) : make_uint4(ninf, ninf, ninf, ninf);
        *reinterpret_cast<uint4 *>(d + q * VEC) = v;
    }
}

hipError_t launch_pruned_fill(const void *logits, void *dense, int64_t ld, int64_t dst_ld, int V, int rows, int dtype,
                              const uint32_t *groups, const int32_t *group_count, int groups_ld, hipStream_t st) {
    const int ngt = (V + 7) / 8;
    dim3 grid((ngt + kThreads - 1) / kThreads, rows), block(kThreads);
    if (dtype == 0)
        hipLaunchKernelGGL(pruned_fill_kernel<float>, grid, block, 0, st, static_cast<const float *>(logits),
                           static_cast<float *>(dense), ld, dst_ld, V, groups, group_count, groups_ld);
    else
        hipLaunchKernelGGL(pruned_fill_kernel<uint16_t>, grid, block, 0, st, static_cast<const uint16_t *>(logits),
                           static_cast<uint16_t *>(dense), ld, dst_ld, V, groups, group_count, groups_ld);
    return hipGetLastError();
}

template <typename T, bool M, bool PN>
static hipError_t launch_pruned_t(const SampleParams &P, int rows, hipStream_t st) {
    hipLaunchKernelGGL((pruned_kernel<T, M, PN>), dim3(rows), dim3(kThreads), 0, st, P);
    return hipGetLastError();
}

template <typename T>
static hipError_t launch_pruned_m(const SampleParams &P, int rows, hipStream_t st) {
    const bool m = P.src.mask != nullptr;
    const bool pn = P.src.hist != nullptr || P.src.edit_ids != nullptr;
    if (m) return pn ? launch_pruned_t<T, true, true>(P, rows, st) : launch_pruned_t<T, true, false>(P, rows, st);
    return pn ? launch_pruned_t<T, false, true>(P, rows, st) : launch_pruned_t<T, false, false>(P, rows, st);
}

hipError_t launch_pruned(const SampleParams &P, int dtype, int rows, hipStream_t st) {
    return dtype == 0 ? launch_pruned_m<float>(P, rows, st) : launch_pruned_m<uint16_t>(P, rows, st);
}

}  // namespace zi
