// zi_dry.hip -- DRY edits (Sampler.applyDry, src/sampler.zig:104-187) for a
// batch of device-resident histories, in the zi_batch.edit_* format that the
// sampling kernels apply.
//
// One 1024-thread workgroup per row, everything in LDS:
//  1. R[k] = the k-th most recent token, k < L = min(hist_len, dry_range,
//     4096) (the reference's ring of max_history = 4096, :31);
//  2. rep_limit = the first k whose token is a sequence breaker (:112-119),
//     an LDS atomicMin;
//  3. z[i] = the common prefix of R[0..] and R[i..], capped at
//     min(L - i, rep_limit), which is what the reference's Z-algorithm
//     (:121-149) yields: its z-box start is a valid match length below the
//     cap and its loop extends to the first mismatch or the cap.  Here the
//     i run in blocks of 1024, one per thread; a block starts from the z-box
//     of the blocks before it (the largest r, then the largest l), so an i
//     inside that box whose mirror i - l is already known starts at
//     min(r - i + 1, z[i - l]) and extends from there, four tokens per
//     step.  A repetition loop then costs its first block, not L^2 / 2
//     compares;
//  4. each i with z[i] >= allowed_length whose continuation R[i-1] is not a
//     breaker contributes (R[i-1], z[i]) (:151-176): an LDS hash keeps, per
//     token, the first i and the longest z;
//  5. the reference keeps the first 128 distinct tokens in order of first
//     appearance (i ascending) and, for those, the longest repeat: rank =
//     the number of distinct tokens that appeared earlier (a bitset over i
//     and its prefix popcounts);
//  6. penalty = mult * pow(base, min(len - allowed, max_exp)) (:178-186),
//     with std.math.pow restated in zi_pow.hpp.
#include "zi_internal.hpp"
#include "zi_launch.hpp"
#include "zi_common.hpp"
#include "zi_pow.hpp"

namespace zi {

constexpr int kDryThreads = 1024;
constexpr int kDryHist = 4096;  // src/sampler.zig:31 max_history
constexpr int kDryBreakers = 16;  // :32 max_breakers
constexpr int kDryPen = 128;      // :152 max_penalized
constexpr int kDryHash = 8192;    // > 2 x the distinct continuations (< 4096)
constexpr int kDryWords = kDryHist / 32;

struct DryParams {
    const uint32_t *hist;
    const int32_t *hist_len;
    int hist_ld;
    const uint32_t *breakers;
    int n_breakers;
    float mult, base;
    uint32_t allowed, range;
    int off;  // DRY disabled (:105): every count is 0
    uint32_t *out_ids;
    float *out_delta;
    int32_t *out_count;
    int edit_ld;
};

struct DryLds {
    uint32_t R[kDryHist];
    uint32_t z[kDryHist];
    uint32_t key[kDryHash];  // token + 1; 0 = empty
    uint32_t first[kDryHash];
    uint32_t len[kDryHash];
    uint32_t kbits[kDryWords];  // first appearances (bit i)
    uint32_t kpre[kDryWords];   // distinct tokens before word w
    uint32_t brk[kDryBreakers];
    int s_rep;
    unsigned long long s_box;  // (r + 1) << 32 | l of the z-box with the largest r (then l); 0: none
};

__device__ __forceinline__ bool dry_is_breaker(const DryLds &s, int nb, uint32_t t) {
    bool b = false;
    for (int j = 0; j < nb; ++j) b |= s.brk[j] == t;
    return b;
}

__global__ __launch_bounds__(kDryThreads) void dry_kernel(DryParams P) {
    __shared__ DryLds s;
    const int tid = threadIdx.x, row = blockIdx.x;
    int n = P.hist_len[row];
    n = n < 0 ? 0 : (n > P.hist_ld ? P.hist_ld : n);
    const int L = min(n, (int)min(P.range, (uint32_t)kDryHist));
    const int allowed = (int)min(P.allowed, (uint32_t)kDryHist + 1u);
    if (P.off || L <= allowed) {  // :105-107
        if (tid == 0) P.out_count[row] = 0;
        return;
    }
    const uint32_t *h = P.hist + (int64_t)row * P.hist_ld;
    for (int k = tid; k < L; k += kDryThreads) s.R[k] = h[n - 1 - k];
    if (tid < P.n_breakers) s.brk[tid] = P.breakers[tid];
    for (int i = tid; i < kDryHash; i += kDryThreads) {
        s.key[i] = 0u;
        s.first[i] = 0xFFFFFFFFu;
        s.len[i] = 0u;
    }
    for (int i = tid; i < kDryWords; i += kDryThreads) s.kbits[i] = 0u;
    if (tid == 0) {
        s.s_rep = L;
        s.s_box = 0ull;
    }
    __syncthreads();
    const int nb = P.n_breakers;
    for (int k = tid; k < L; k += kDryThreads)
        if (dry_is_breaker(s, nb, s.R[k])) atomicMin(&s.s_rep, k);
    __syncthreads();
    const int rep = s.s_rep;
    if (rep < allowed) {  // :120 (uniform)
        if (tid == 0) P.out_count[row] = 0;
        return;
    }
    for (int i0 = 1; i0 < L; i0 += kDryThreads) {
        const int i = i0 + tid;
        const unsigned long long box = s.s_box;  // the blocks before this one
        __syncthreads();                         // every thread has read it before any update
        if (i < L) {
            const int cap = min(L - i, rep);
            int z = 0;
            if (box) {
                const int r = (int)(box >> 32) - 1, l = (int)(box & 0xFFFFFFFFull);
                if (i <= r && i - l < i0) z = min(min(r - i + 1, (int)s.z[i - l]), cap);
            }
            // extend: positions below z match; 4 tokens per step, then one at a time
            while (z + 4 <= cap) {
                const uint32_t a0 = s.R[z], a1 = s.R[z + 1], a2 = s.R[z + 2], a3 = s.R[z + 3];
                const uint32_t b0 = s.R[i + z], b1 = s.R[i + z + 1], b2 = s.R[i + z + 2], b3 = s.R[i + z + 3];
                const uint32_t m =
                    (a0 != b0 ? 1u : 0u) | (a1 != b1 ? 2u : 0u) | (a2 != b2 ? 4u : 0u) | (a3 != b3 ? 8u : 0u);
                if (m) {
                    z += __ffs(m) - 1;
                    break;
                }
                z += 4;
            }
            while (z < cap && s.R[z] == s.R[i + z]) ++z;
            s.z[i] = (uint32_t)z;
            if (z > 0) atomicMax(&s.s_box, ((unsigned long long)(i + z) << 32) | (unsigned long long)i);
            if (z >= allowed) {
                const uint32_t t = s.R[i - 1];
                if (!dry_is_breaker(s, nb, t)) {
                    uint32_t hs = (t * 2654435761u) >> (32 - 13);
                    // at most L - 1 < kDryHash / 2 keys: the probe meets a free slot
                    for (int probe = 0; probe < kDryHash; ++probe) {
                        const uint32_t prev = atomicCAS(&s.key[hs], 0u, t + 1u);
                        if (prev == 0u || prev == t + 1u) break;
                        hs = (hs + 1u) & (kDryHash - 1);
                    }
                    atomicMin(&s.first[hs], (uint32_t)i);
                    atomicMax(&s.len[hs], (uint32_t)z);
                }
            }
        }
        __syncthreads();  // this block's z and box complete
    }
    __syncthreads();
    for (int i = tid; i < kDryHash; i += kDryThreads)
        if (s.key[i]) atomicOr(&s.kbits[s.first[i] >> 5], 1u << (s.first[i] & 31));
    __syncthreads();
    if (tid < 64) {  // exclusive prefix popcount over the 128 words, one wave
        const int w0 = tid * 2;
        const uint32_t c0 = __popc(s.kbits[w0]), c1 = __popc(s.kbits[w0 + 1]);
        uint32_t incl = c0 + c1;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t t = __shfl_up(incl, off);
            if (tid >= off) incl += t;
        }
        const uint32_t excl = incl - c0 - c1;
        s.kpre[w0] = excl;
        s.kpre[w0 + 1] = excl + c0;
        if (tid == 63) P.out_count[row] = (int32_t)min(incl, (uint32_t)kDryPen);
    }
    __syncthreads();
    uint32_t *oid = P.out_ids + (int64_t)row * P.edit_ld;
    float *odl = P.out_delta + (int64_t)row * P.edit_ld;
    for (int i = tid; i < kDryHash; i += kDryThreads) {
        if (!s.key[i]) continue;
        const uint32_t f = s.first[i];
        const uint32_t rank = s.kpre[f >> 5] + __popc(s.kbits[f >> 5] & ((1u << (f & 31)) - 1u));
        if (rank < (uint32_t)kDryPen) {
            oid[rank] = s.key[i] - 1u;
            odl[rank] = dry_penalty(s.len[i], P.mult, P.base, P.allowed);
        }
    }
}

}  // namespace zi

extern "C" int32_t zi_dry_edits_rows(zi_ctx *c, const zi_params *p, const uint32_t *hist, const int32_t *hist_len,
                                     int32_t hist_ld, int32_t rows, const uint32_t *breakers, uint32_t n_breakers,
                                     uint32_t *out_ids, float *out_delta, int32_t *out_count, int32_t edit_ld) {
    const char *fn = "zi_dry_edits_rows";
    if (!c || !p || !hist_len || !out_count || rows < 1 || hist_ld < 0 || (hist_ld > 0 && !hist))
        return zi_fail(ZI_ERR_INVALID, "%s: bad argument", fn);
    if (rows > c->max_rows) return zi_fail(ZI_ERR_CAPACITY, "%s: rows=%d > max_rows %d", fn, rows, c->max_rows);
    if (n_breakers > (uint32_t)zi::kDryBreakers || (n_breakers && !breakers))
        return zi_fail(ZI_ERR_INVALID, "%s: %u breakers (at most %d)", fn, n_breakers, zi::kDryBreakers);
    const bool off = p->dry_multiplier == 0.0f || p->dry_base < 1.0f || p->dry_range == 0;  // :105
    if (!off && (!out_ids || !out_delta || edit_ld < zi::kDryPen))
        return zi_fail(ZI_ERR_INVALID, "%s: out_ids/out_delta NULL or edit_ld=%d < %d", fn, edit_ld, zi::kDryPen);
    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) return zi_hip_fail(e, "hipSetDevice");
    zi::DryParams P;
    P.hist = hist;
    P.hist_len = hist_len;
    P.hist_ld = hist_ld;
    P.breakers = breakers;
    P.n_breakers = (int)n_breakers;
    P.mult = p->dry_multiplier;
    P.base = p->dry_base;
    P.allowed = p->dry_allowed_length;
    P.range = p->dry_range;
    P.off = off ? 1 : 0;
    P.out_ids = out_ids;
    P.out_delta = out_delta;
    P.out_count = out_count;
    P.edit_ld = edit_ld;
    hipLaunchKernelGGL(zi::dry_kernel, dim3(rows), dim3(zi::kDryThreads), 0, c->stream, P);
    e = hipGetLastError();
    if (e != hipSuccess) return zi_hip_fail(e, "dry kernel launch");
    return ZI_OK;
}
