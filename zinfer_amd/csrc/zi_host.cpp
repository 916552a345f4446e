// zi_host.cpp -- host-side mirror of the reference's Zig API around the
// device path: Sampler (src/sampler.zig:38-286), the DRY edit builder
// (:104-187), argmaxWithMargin on a host row (:532-614) and
// Gen.AdaptiveDraft (src/gen.zig:366-432).  Sampling itself always runs on
// the GPU through zi_sample_rows; this file only keeps the reference's state
// (RNG, token ring, breakers) and its in-place side effects.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>

#include "../../include/zinfer_hip.h"
#include "zi_internal.hpp"
#include "zi_launch.hpp"
#include "zi_expf.hpp"
#include "zi_pow.hpp"

namespace {

constexpr uint32_t kMaxHistory = 4096;  // src/sampler.zig:31
constexpr uint32_t kMaxBreakers = 16;   // src/sampler.zig:32

// std.Random.DefaultPrng: xoshiro256++ (Blackman & Vigna) seeded with four
// splitmix64 outputs; Random.float(f32) builds the float from one 64-bit draw
// (23 mantissa bits, exponent from the leading-zero count).
uint64_t splitmix_next(uint64_t &s) {
    uint64_t z = (s += 0x9e3779b97f4a7c15ULL);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
struct Xoshiro {
    uint64_t s[4];
    void seed(uint64_t v) {
        uint64_t st = v;
        for (auto &w : s) w = splitmix_next(st);
    }
    uint64_t next() {
        uint64_t r = rotl(s[0] + s[3], 23) + s[0];
        uint64_t t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }
    float f32() {
        uint64_t r = next();
        uint32_t lz = r ? (uint32_t)__builtin_clzll(r) : 64u;
        if (lz >= 41) {
            uint64_t r2 = next();
            lz = 41 + (r2 ? (uint32_t)__builtin_clzll(r2) : 64u);
            if (lz == 41 + 64) lz += (uint32_t)__builtin_clz((uint32_t)next() | 0x7FFu);
        }
        uint32_t bits = ((126u - lz) << 23) | (uint32_t)(r & 0x7FFFFFu);
        float f;
        std::memcpy(&f, &bits, 4);
        return f;
    }
};

// The final-logit softcap of src/model.zig:2492-2513 on a host row, in place
// (the caller's logits then hold what the reference's forward leaves there).
// Same f32 steps as the device's: the vector body below 32*floor(V/32), the
// scalar tail cap * tanh(l / cap) from there on.
static void host_softcap(float *logits, uint32_t V, float cap) {
    const float inv_cap = 1.0f / cap;
    const uint32_t body = V / 32 * 32;
    for (uint32_t i = 0; i < body; ++i) {
        const float z = std::fmin(std::fmax(logits[i] * inv_cap, -9.0f), 9.0f);
        const float e2z = zi::zexpf(z * 2.0f);
        logits[i] = cap * ((e2z - 1.0f) / (e2z + 1.0f));
    }
    for (uint32_t i = body; i < V; ++i) logits[i] = cap * (float)std::tanh((double)(logits[i] / cap));
}

// src/sampler.zig:91-100 plus the frequency/presence extension, on a host row.
void host_penalty(float *logits, uint32_t V, const uint32_t *win, uint32_t n, const zi_params &p) {
    const bool rep = p.repeat_penalty != 1.0f;
    const bool fp = p.freq_penalty != 0.0f || p.presence_penalty != 0.0f;
    if (!rep && !fp) return;
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t tok = win[i];
        if (std::find(win, win + i, tok) != win + i) continue;
        if (tok >= V) continue;
        float &l = logits[tok];
        if (rep) l = (l > 0.0f) ? l / p.repeat_penalty : l * p.repeat_penalty;
        if (fp) {
            uint32_t cnt = (uint32_t)std::count(win, win + n, tok);
            float t = (float)cnt * p.freq_penalty;
            t = t + p.presence_penalty;
            l = l - t;
        }
    }
}

struct Staging {
    void *h = nullptr;  // pinned host
    void *d = nullptr;  // device
    size_t bytes = 0;
    // Frees both buffers; returns the first failure (hipSuccess if none).
    hipError_t release() {
        hipError_t e = hipSuccess;
        if (h) {
            const hipError_t eh = hipHostFree(h);
            if (eh != hipSuccess) e = eh;
        }
        if (d) {
            const hipError_t ed = hipFree(d);
            if (ed != hipSuccess && e == hipSuccess) e = ed;
        }
        h = d = nullptr;
        bytes = 0;
        return e;
    }
    ~Staging() {
        // a destructor cannot report: a failure is left in zi_last_error()
        const hipError_t e = release();
        if (e != hipSuccess) zi_hip_fail(e, "staging release");
    }
    int32_t ensure(size_t n) {
        if (n <= bytes) return ZI_OK;
        hipError_t e = release();
        if (e != hipSuccess) return zi_hip_fail(e, "staging release");
        e = hipHostMalloc(&h, n, hipHostMallocDefault);
        if (e == hipSuccess) e = hipMalloc(&d, n);
        if (e != hipSuccess) return zi_fail(ZI_ERR_OOM, "staging allocation of %zu bytes: %s", n, hipGetErrorString(e));
        bytes = n;
        return ZI_OK;
    }
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace

uint32_t zi_dry_edits_impl(const uint32_t *hist, uint32_t n_hist, const uint32_t *breakers, uint32_t n_breakers,
                           const zi_params &p, uint32_t *out_ids, float *out_deltas) {
    // src/sampler.zig:104-187 on a linear history (oldest first): R[k] is the
    // k-th most recent token.
    if (p.dry_multiplier == 0.0f || p.dry_base < 1.0f || p.dry_range == 0) return 0;
    uint32_t L = std::min(n_hist, std::min(p.dry_range, kMaxHistory));
    if (L <= p.dry_allowed_length) return 0;
    auto R = [&](uint32_t k) { return hist[n_hist - 1 - k]; };
    auto is_brk = [&](uint32_t t) { return std::find(breakers, breakers + n_breakers, t) != breakers + n_breakers; };
    uint32_t rep_limit = L;
    for (uint32_t k = 0; k < L; ++k)
        if (is_brk(R(k))) {
            rep_limit = k;
            break;
        }
    if (rep_limit < p.dry_allowed_length) return 0;
    static thread_local uint32_t z[kMaxHistory];
    z[0] = 0;
    uint32_t l = 0, r = 0;
    for (uint32_t i = 1; i < L; ++i) {
        z[i] = (i <= r) ? std::min(r - i + 1, z[i - l]) : 0u;
        const uint32_t max_z = std::min(L - i, rep_limit);
        while (z[i] < max_z && R(z[i]) == R(i + z[i])) z[i] += 1;
        if (i + z[i] > 0 && i + z[i] - 1 > r) {
            l = i;
            r = i + z[i] - 1;
        }
    }
    uint32_t n_pen = 0;
    uint32_t lens[128];
    for (uint32_t k = 1; k < L; ++k) {
        const uint32_t rlen = z[k];
        if (rlen < p.dry_allowed_length) continue;
        const uint32_t cont = R(k - 1);
        if (is_brk(cont)) continue;
        uint32_t pi = 0;
        while (pi < n_pen && out_ids[pi] != cont) ++pi;
        if (pi < n_pen) {
            lens[pi] = std::max(lens[pi], rlen);
        } else if (n_pen < 128) {
            out_ids[n_pen] = cont;
            lens[n_pen] = rlen;
            ++n_pen;
        }
    }
    for (uint32_t i = 0; i < n_pen; ++i)
        out_deltas[i] = zi::dry_penalty(lens[i], p.dry_multiplier, p.dry_base, p.dry_allowed_length);
    return n_pen;
}

extern "C" uint32_t zi_dry_edits(const uint32_t *hist, uint32_t n_hist, const uint32_t *breakers,
                                 uint32_t n_breakers, const zi_params *p, uint32_t *out_ids, float *out_deltas) {
    if (!p || !out_ids || !out_deltas || (n_hist && !hist) || (n_breakers && !breakers)) return 0;
    return zi_dry_edits_impl(hist, n_hist, breakers, n_breakers, *p, out_ids, out_deltas);
}

struct zi_sampler {
    zi_ctx *ctx = nullptr;
    uint32_t vocab = 0, ld = 0;
    zi_params p{};
    Xoshiro rng{};
    uint32_t history[kMaxHistory];  // ring, src/sampler.zig:44, :87
    uint64_t n_history = 0;         // accept() also advances the 64-entry ring (:85) in lockstep
    uint32_t breakers[kMaxBreakers];
    uint32_t n_breakers = 0;
    Staging st;
    Staging vst;  // zi_sampler_verify, allocated on first use
    // staging layout (bytes)
    size_t o_logits = 0, o_hist = 0, o_hlen = 0, o_eids = 0, o_edel = 0, o_ecnt = 0, o_u = 0, o_tok = 0,
           o_margin = 0, o_ndraws = 0, total = 0;

    // Last min(n, W) accepted tokens, oldest first.
    uint32_t window(uint32_t W, uint32_t *out) const {
        uint64_t n = std::min<uint64_t>(std::min<uint64_t>(n_history, W), kMaxHistory);
        for (uint64_t i = 0; i < n; ++i) out[i] = history[(n_history - n + i) & (kMaxHistory - 1)];
        return (uint32_t)n;
    }
};

extern "C" int32_t zi_sampler_init(zi_sampler **out, zi_ctx *ctx, uint32_t vocab, const zi_params *p) {
    if (!out || !ctx || !p || vocab == 0) return zi_fail(ZI_ERR_INVALID, "zi_sampler_init: bad argument");
    *out = nullptr;
    if ((int64_t)vocab > ctx->max_vocab)
        return zi_fail(ZI_ERR_CAPACITY, "zi_sampler_init: vocab %u > context max_vocab %d", vocab, ctx->max_vocab);
    zi_sampler *s = new (std::nothrow) zi_sampler();
    if (!s) return zi_fail(ZI_ERR_OOM, "zi_sampler_init: host allocation");
    s->ctx = ctx;
    s->vocab = vocab;
    s->ld = (vocab + 7u) & ~7u;
    s->p = *p;
    s->rng.seed(p->seed);  // :52
    size_t o = 0;
    s->o_logits = o;
    o = align_up(o + (size_t)s->ld * 4, 256);
    s->o_hist = o;
    o = align_up(o + zi::kMaxWinHost * 4, 256);
    s->o_hlen = o;
    o += 16;
    s->o_eids = o;
    o = align_up(o + zi::kMaxEditsHost * 4, 256);
    s->o_edel = o;
    o = align_up(o + zi::kMaxEditsHost * 4, 256);
    s->o_ecnt = o;
    o += 16;
    s->o_u = o;
    o += 16;
    s->o_tok = o;
    o += 16;
    s->o_margin = o;
    o += 16;
    s->o_ndraws = o;
    o += 16;
    s->total = align_up(o, 256);
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) {
        delete s;
        return zi_hip_fail(e, "zi_sampler_init: hipSetDevice");
    }
    int32_t rc = s->st.ensure(s->total);
    if (rc) {
        delete s;
        return rc;
    }
    *out = s;
    return ZI_OK;
}

extern "C" void zi_sampler_deinit(zi_sampler *s) { delete s; }
extern "C" void zi_sampler_reset(zi_sampler *s) {
    if (s) s->n_history = 0;  // :64-67 clears n_recent and n_history only
}
extern "C" void zi_sampler_add_breaker(zi_sampler *s, uint32_t tok) {
    if (s && s->n_breakers < kMaxBreakers) s->breakers[s->n_breakers++] = tok;  // :69-74
}
extern "C" int32_t zi_sampler_is_breaker(const zi_sampler *s, uint32_t tok) {
    if (!s) return 0;
    for (uint32_t i = 0; i < s->n_breakers; ++i)
        if (s->breakers[i] == tok) return 1;
    return 0;
}
extern "C" void zi_sampler_accept(zi_sampler *s, uint32_t tok) {
    if (!s) return;
    s->history[s->n_history & (kMaxHistory - 1)] = tok;  // :84-89
    s->n_history += 1;
}
extern "C" void zi_sampler_get_params(const zi_sampler *s, zi_params *p) {
    if (s && p) *p = s->p;
}
extern "C" void zi_sampler_set_params(zi_sampler *s, const zi_params *p) {
    if (s && p) s->p = *p;
}
extern "C" void zi_sampler_seed(zi_sampler *s, uint64_t seed) {
    if (s) s->rng.seed(seed);
}
extern "C" float zi_sampler_rand_f32(zi_sampler *s) { return s ? s->rng.f32() : 0.0f; }

static uint32_t sampler_dry(const zi_sampler *s, uint32_t *ids, float *deltas) {
    uint32_t lin[kMaxHistory];
    uint32_t n = s->window(kMaxHistory, lin);
    return zi_dry_edits_impl(lin, n, s->breakers, s->n_breakers, s->p, ids, deltas);
}

extern "C" void zi_sampler_apply_dry(const zi_sampler *s, float *logits, uint32_t n) {
    if (!s || !logits) return;
    uint32_t ids[128];
    float d[128];
    uint32_t m = sampler_dry(s, ids, d);
    for (uint32_t i = 0; i < m; ++i)
        if (ids[i] < n) logits[ids[i]] -= d[i];  // :180-185
}

extern "C" int32_t zi_sampler_sample_with_margin(zi_sampler *s, float *logits, uint32_t n, uint32_t *tok,
                                                 float *margin) {
    if (!s || !logits || !tok) return zi_fail(ZI_ERR_INVALID, "zi_sampler_sample_with_margin: bad argument");
    if (n != s->vocab) return zi_fail(ZI_ERR_INVALID, "zi_sampler_sample_with_margin: n=%u != vocab %u", n, s->vocab);
    zi_ctx *c = s->ctx;
    char *h = (char *)s->st.h;
    char *d = (char *)s->st.d;
    zi_params p = s->p;
    if (p.penalty_last_n > (uint32_t)zi::kMaxWinHost)
        return zi_fail(ZI_ERR_UNSUPPORTED, "penalty_last_n %u > %d", p.penalty_last_n, zi::kMaxWinHost);
    if (p.final_logit_softcap > 0.0f) {
        // the caller's row is capped in place, as the reference's forward
        // leaves it, so the device samples it with the cap off
        host_softcap(logits, n, p.final_logit_softcap);
        p.final_logit_softcap = 0.0f;
    }

    std::memcpy(h + s->o_logits, logits, (size_t)n * 4);
    uint32_t *win = (uint32_t *)(h + s->o_hist);
    uint32_t nw = s->window(p.penalty_last_n, win);
    *(int32_t *)(h + s->o_hlen) = (int32_t)nw;
    uint32_t *eids = (uint32_t *)(h + s->o_eids);
    float *edel = (float *)(h + s->o_edel);
    uint32_t ne = sampler_dry(s, eids, edel);
    *(int32_t *)(h + s->o_ecnt) = (int32_t)ne;
    Xoshiro peek = s->rng;  // the draws are peeked, then committed per ndraws
    float *u = (float *)(h + s->o_u);
    u[0] = peek.f32();
    u[1] = peek.f32();
    *(int32_t *)(h + s->o_ndraws) = 0;  // not every path writes ndraws

    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) return zi_hip_fail(e, "sampler: hipSetDevice");
    e = hipMemcpyAsync(d, h, s->o_ndraws + 16, hipMemcpyHostToDevice, c->stream);
    if (e != hipSuccess) return zi_hip_fail(e, "sampler H2D");
    zi_batch b;
    std::memset(&b, 0, sizeof b);
    b.logits = d + s->o_logits;
    b.dtype = ZI_F32;
    b.rows = 1;
    b.vocab = (int32_t)n;
    b.ld = (int32_t)s->ld;
    b.hist = (const uint32_t *)(d + s->o_hist);
    b.hist_len = (const int32_t *)(d + s->o_hlen);
    b.hist_ld = zi::kMaxWinHost;
    if (ne) {
        b.edit_ids = (const uint32_t *)(d + s->o_eids);
        b.edit_delta = (const float *)(d + s->o_edel);
        b.edit_count = (const int32_t *)(d + s->o_ecnt);
        b.edit_ld = zi::kMaxEditsHost;
    }
    zi_sample_out o;
    std::memset(&o, 0, sizeof o);
    o.tok = (uint32_t *)(d + s->o_tok);
    o.margin = (float *)(d + s->o_margin);
    o.ndraws = (int32_t *)(d + s->o_ndraws);
    int32_t rc = zi_sample_rows(c, &p, &b, (const float *)(d + s->o_u), &o);
    if (rc) return rc;
    e = hipMemcpyAsync(h + s->o_tok, d + s->o_tok, s->o_ndraws + 16 - s->o_tok, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return zi_hip_fail(e, "sampler D2H");
    const int32_t nd = *(int32_t *)(h + s->o_ndraws);
    for (int32_t i = 0; i < nd; ++i) (void)s->rng.f32();
    // the reference's in-place side effects: penalty (:191) then DRY (:192)
    host_penalty(logits, n, win, nw, p);
    for (uint32_t i = 0; i < ne; ++i)
        if (eids[i] < n) logits[eids[i]] -= edel[i];
    *tok = *(uint32_t *)(h + s->o_tok);
    if (margin) *margin = *(float *)(h + s->o_margin);
    return ZI_OK;
}

// ------------------------------------------------ batched draft verification
// src/gen.zig:544-587 verifies a draft row by row: row i is sampled with the
// state after take(draft[0..i)) (penalty ring, DRY history, JSON validator)
// and the next draws of the RNG, and acceptance stops at the first row whose
// token differs from the draft (or is end-of-generation); with every draft
// token accepted, row k (the bonus row) gives the next token.  Every row's
// state is known up front, so all k + 1 rows go in one zi_sample_rows launch;
// only the draws need care: a row takes 0 (greedy), 1, or 2 (XTC chance)
// uniforms, decided by its data and not by the uniform values, so when XTC can
// fire a first launch finds each row's count and a second one runs with each
// row's uniforms at its offset in the stream.
constexpr uint32_t kMaxVerify = 16;  // drafted tokens per call (the reference drafts at most 8)

constexpr uint32_t kMaxBranches = 8;  // branches per tree verify (the reference's tree holds 4, sampler.zig:291)
constexpr uint32_t kMaxVerifyRows = kMaxBranches * (kMaxVerify + 1);

// Verification of nbr drafts (branches) from the sampler's current state in
// one zi_sample_rows launch: branch j's rows are b's rows base_j .. base_j +
// k_j, base_j = sum of (k_i + 1) over i < j, each sampled as the reference's
// loop would sample it were branch j verified alone.  With commit, the branch
// with the most accepted tokens (the first on ties) is applied to the sampler
// and *json; *out_best names it.
static int32_t verify_core(zi_sampler *s, const zi_batch *b, const uint32_t *const *drafts, const uint32_t *ks,
                           uint32_t nbr, uint32_t max_accept, const uint32_t *eog, uint32_t n_eog, zi_vocab *v,
                           zi_json_state *json, bool commit, uint32_t *out_accepted, uint32_t *out_next,
                           float *out_margin, uint32_t *out_best, const char *fn) {
    if (!s || !b || !b->logits || !ks || nbr == 0 || (n_eog && !eog) || !out_accepted || !out_next)
        return zi_fail(ZI_ERR_INVALID, "%s: bad argument", fn);
    if (nbr > kMaxBranches) return zi_fail(ZI_ERR_UNSUPPORTED, "%s: %u branches > %u", fn, nbr, kMaxBranches);
    uint32_t base[kMaxBranches + 1];
    base[0] = 0;
    for (uint32_t j = 0; j < nbr; ++j) {
        if (ks[j] > kMaxVerify) return zi_fail(ZI_ERR_UNSUPPORTED, "%s: k=%u > %u", fn, ks[j], kMaxVerify);
        if (ks[j] && !drafts[j]) return zi_fail(ZI_ERR_INVALID, "%s: branch %u has no draft", fn, j);
        base[j + 1] = base[j] + ks[j] + 1;
    }
    const uint32_t R = base[nbr];
    if ((uint32_t)b->vocab != s->vocab || b->rows < (int32_t)R)
        return zi_fail(ZI_ERR_INVALID, "%s: batch of %d x %d for %u rows, vocab %u", fn, b->rows, b->vocab, R, s->vocab);
    if ((v == nullptr) != (json == nullptr)) return zi_fail(ZI_ERR_INVALID, "%s: vocab and json state go together", fn);
    if (v && zi_vocab_size(v) != (int32_t)s->vocab)
        return zi_fail(ZI_ERR_INVALID, "%s: vocab has %d tokens, sampler %u", fn, zi_vocab_size(v), s->vocab);
    zi_ctx *c = s->ctx;
    if ((int32_t)R > c->max_rows) return zi_fail(ZI_ERR_CAPACITY, "%s: %u rows > max_rows", fn, R);
    const zi_params &p = s->p;
    if (p.penalty_last_n > (uint32_t)zi::kMaxWinHost)
        return zi_fail(ZI_ERR_UNSUPPORTED, "penalty_last_n %u > %d", p.penalty_last_n, zi::kMaxWinHost);
    const uint32_t W = (s->vocab + 31) / 32;
    const uint32_t RM = R;
    // window rows only as wide as the window, so the copy to the device stays small
    const uint32_t WP = std::max<uint32_t>(1u, std::min<uint32_t>(p.penalty_last_n, (uint32_t)zi::kMaxWinHost));
    size_t o = 0;
    const size_t o_u = o;
    o = align_up(o + RM * 8, 256);
    const size_t o_hlen = o;
    o = align_up(o + RM * 4, 256);
    const size_t o_hist = o;
    o = align_up(o + (size_t)RM * WP * 4, 256);
    const size_t o_in = o;  // host -> device up to here on every pass
    const size_t o_eids = o;
    o = align_up(o + (size_t)RM * zi::kMaxEditsHost * 4, 256);
    const size_t o_edel = o;
    o = align_up(o + (size_t)RM * zi::kMaxEditsHost * 4, 256);
    const size_t o_ecnt = o;
    o = align_up(o + RM * 4, 256);
    const size_t o_in_edits = o;  // ... and up to here when there are DRY edits
    const size_t o_tok = o;
    o = align_up(o + RM * 4, 256);
    const size_t o_margin = o;
    o = align_up(o + RM * 4, 256);
    const size_t o_nd = o;
    o = align_up(o + RM * 4, 256);
    const size_t o_out = o;  // device -> host from o_tok to here
    const size_t o_mask = o;
    o = align_up(o + (size_t)RM * W * 4, 256);
    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) return zi_hip_fail(e, "verify: hipSetDevice");
    int32_t rc = s->vst.ensure(o);
    if (rc) return rc;
    char *h = (char *)s->vst.h;
    char *d = (char *)s->vst.d;

    // per-row penalty windows and DRY edits: the history plus the branch's draft[0..i)
    static thread_local uint32_t lin[kMaxHistory + kMaxVerify];
    const uint32_t nlin = s->window(kMaxHistory, lin);
    bool any_edits = false;
    for (uint32_t j = 0; j < nbr; ++j) {
        std::memcpy(lin + nlin, drafts[j], (size_t)ks[j] * 4);
        for (uint32_t i = 0; i <= ks[j]; ++i) {
            const uint32_t row = base[j] + i;
            const uint32_t len = nlin + i;
            const uint32_t nw = std::min<uint32_t>(len, std::min<uint32_t>(p.penalty_last_n, WP));
            std::memcpy(h + o_hist + (size_t)row * WP * 4, lin + len - nw, (size_t)nw * 4);
            ((int32_t *)(h + o_hlen))[row] = (int32_t)nw;
            uint32_t ne = 0;
            if (p.dry_multiplier != 0.0f) {
                const uint32_t hl = std::min<uint32_t>(len, kMaxHistory);
                ne = zi_dry_edits_impl(lin + len - hl, hl, s->breakers, s->n_breakers, p,
                                       (uint32_t *)(h + o_eids) + (size_t)row * zi::kMaxEditsHost,
                                       (float *)(h + o_edel) + (size_t)row * zi::kMaxEditsHost);
            }
            ((int32_t *)(h + o_ecnt))[row] = (int32_t)ne;
            any_edits |= ne > 0;
        }
    }
    // per-row JSON states: the validator after consuming the branch's draft[0..i)
    static thread_local zi_json_state states[kMaxVerifyRows];
    if (v) {
        for (uint32_t j = 0; j < nbr; ++j) {
            zi_json_state st = *json;
            for (uint32_t i = 0; i <= ks[j]; ++i) {
                states[base[j] + i] = st;
                if (i < ks[j]) {
                    const uint8_t *pc;
                    uint32_t pn;
                    if (!zi_vocab_piece(v, drafts[j][i], &pc, &pn))
                        return zi_fail(ZI_ERR_INVALID, "%s: draft token %u out of range", fn, drafts[j][i]);
                    zi_json_consume(&st, pc, pn);
                }
            }
        }
    }
    // draws: every branch starts at the sampler's next draw; row i of a
    // branch takes its uniforms at offset off[i] of that stream
    Xoshiro peek = s->rng;
    float stream[2 * (kMaxVerify + 1) + 2];
    for (uint32_t i = 0; i < 2 * (kMaxVerify + 1) + 2; ++i) stream[i] = peek.f32();
    const bool sampled = p.temp > 0.0f;
    const bool xtc = sampled && p.xtc_probability > 0.0f && p.xtc_threshold <= 0.5f;
    static thread_local int32_t nd[kMaxVerifyRows];
    for (uint32_t i = 0; i < R; ++i) nd[i] = sampled ? 1 : 0;

    zi_batch bb = *b;
    bb.rows = (int32_t)R;
    bb.hist = (const uint32_t *)(d + o_hist);
    bb.hist_len = (const int32_t *)(d + o_hlen);
    bb.hist_ld = (int32_t)WP;
    bb.mask = v ? (const uint32_t *)(d + o_mask) : nullptr;
    bb.mask_ld = (int32_t)W;
    bb.edit_ids = any_edits ? (const uint32_t *)(d + o_eids) : nullptr;
    bb.edit_delta = any_edits ? (const float *)(d + o_edel) : nullptr;
    bb.edit_count = any_edits ? (const int32_t *)(d + o_ecnt) : nullptr;
    bb.edit_ld = zi::kMaxEditsHost;
    zi_sample_out so;
    std::memset(&so, 0, sizeof so);
    so.tok = (uint32_t *)(d + o_tok);
    so.margin = (float *)(d + o_margin);
    so.ndraws = (int32_t *)(d + o_nd);
    if (v) {
        rc = zi_json_mask_rows(c, v, states, (int32_t)R, (uint32_t *)(d + o_mask), (int32_t)W);
        if (rc) return rc;
    }
    for (int pass = xtc ? 0 : 1; pass < 2; ++pass) {
        float *u = (float *)(h + o_u);
        for (uint32_t j = 0; j < nbr; ++j) {
            uint32_t off = 0;
            for (uint32_t i = base[j]; i < base[j + 1]; ++i) {
                u[2 * i] = stream[off];
                u[2 * i + 1] = stream[off + 1];
                off += (uint32_t)nd[i];
            }
        }
        e = hipMemcpyAsync(d, h, any_edits && pass == (xtc ? 0 : 1) ? o_in_edits : o_in, hipMemcpyHostToDevice,
                           c->stream);
        if (e != hipSuccess) return zi_hip_fail(e, "verify: H2D");
        rc = zi_sample_rows(c, &p, &bb, (const float *)(d + o_u), &so);
        if (rc) return rc;
        e = hipMemcpyAsync(h + o_tok, d + o_tok, o_out - o_tok, hipMemcpyDeviceToHost, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) return zi_hip_fail(e, "verify: D2H");
        for (uint32_t i = 0; i < R; ++i) nd[i] = ((const int32_t *)(h + o_nd))[i];
    }
    const uint32_t *tok = (const uint32_t *)(h + o_tok);
    const float *mg = (const float *)(h + o_margin);
    uint32_t best = 0;
    for (uint32_t j = 0; j < nbr; ++j) {
        const uint32_t *t = tok + base[j];
        const uint32_t *dr = drafts[j];
        uint32_t a = 0;
        while (a < ks[j] && a < max_accept && t[a] == dr[a] && std::find(eog, eog + n_eog, t[a]) == eog + n_eog) ++a;
        out_accepted[j] = a;
        out_next[j] = t[a];
        if (out_margin) out_margin[j] = mg[base[j] + a];
        if (a > out_accepted[best]) best = j;
    }
    if (out_best) *out_best = best;
    if (!commit) return ZI_OK;
    // side effects of the reference loop for the chosen branch: take() for the
    // accepted tokens, and the draws of rows 0..a (the rows it sampled)
    const uint32_t a = out_accepted[best];
    uint32_t used = 0;
    for (uint32_t i = 0; i <= a; ++i) used += (uint32_t)nd[base[best] + i];
    for (uint32_t i = 0; i < used; ++i) (void)s->rng.f32();
    for (uint32_t i = 0; i < a; ++i) {
        zi_sampler_accept(s, drafts[best][i]);
        if (v) {
            const uint8_t *pc;
            uint32_t pn;
            zi_vocab_piece(v, drafts[best][i], &pc, &pn);
            zi_json_consume(json, pc, pn);
        }
    }
    return ZI_OK;
}

extern "C" int32_t zi_sampler_verify(zi_sampler *s, const zi_batch *b, const uint32_t *draft, uint32_t k,
                                     uint32_t max_accept, const uint32_t *eog, uint32_t n_eog, zi_vocab *v,
                                     zi_json_state *json, uint32_t *out_accepted, uint32_t *out_next,
                                     float *out_margin) {
    if (k && !draft) return zi_fail(ZI_ERR_INVALID, "zi_sampler_verify: bad argument");
    const uint32_t *drafts[1] = {draft};
    return verify_core(s, b, drafts, &k, 1, max_accept, eog, n_eog, v, json, true, out_accepted, out_next,
                       out_margin, nullptr, "zi_sampler_verify");
}

extern "C" int32_t zi_sampler_verify_tree(zi_sampler *s, const zi_batch *b, const uint32_t *drafts, uint32_t draft_ld,
                                          const uint32_t *ks, uint32_t n_branches, uint32_t max_accept,
                                          const uint32_t *eog, uint32_t n_eog, zi_vocab *v, zi_json_state *json,
                                          int32_t commit, uint32_t *out_accepted, uint32_t *out_next,
                                          float *out_margin, uint32_t *out_best) {
    if (!drafts || !ks || n_branches == 0 || n_branches > kMaxBranches)
        return zi_fail(n_branches > kMaxBranches ? ZI_ERR_UNSUPPORTED : ZI_ERR_INVALID,
                       "zi_sampler_verify_tree: %u branches (1..%u) or NULL drafts", n_branches, kMaxBranches);
    const uint32_t *rows[kMaxBranches];
    for (uint32_t j = 0; j < n_branches; ++j) {
        if (ks[j] > draft_ld) return zi_fail(ZI_ERR_INVALID, "zi_sampler_verify_tree: k=%u > draft_ld", ks[j]);
        rows[j] = drafts + (size_t)j * draft_ld;
    }
    return verify_core(s, b, rows, ks, n_branches, max_accept, eog, n_eog, v, json, commit != 0, out_accepted,
                       out_next, out_margin, out_best, "zi_sampler_verify_tree");
}

extern "C" int32_t zi_sampler_sample(zi_sampler *s, float *logits, uint32_t n, uint32_t *tok) {
    return zi_sampler_sample_with_margin(s, logits, n, tok, nullptr);
}

extern "C" int32_t zi_argmax_with_margin(zi_ctx *c, const float *logits, uint32_t n, uint32_t *tok, float *margin) {
    if (!c || !logits || !tok || n == 0) return zi_fail(ZI_ERR_INVALID, "zi_argmax_with_margin: bad argument");
    if ((int64_t)n > c->max_vocab) return zi_fail(ZI_ERR_CAPACITY, "zi_argmax_with_margin: n > max_vocab");
    static thread_local Staging st;
    const uint32_t ld = (n + 7u) & ~7u;
    const size_t o_out = align_up((size_t)ld * 4, 256);
    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) return zi_hip_fail(e, "zi_argmax_with_margin: hipSetDevice");
    int32_t rc = st.ensure(o_out + 256);
    if (rc) return rc;
    std::memcpy(st.h, logits, (size_t)n * 4);
    e = hipMemcpyAsync(st.d, st.h, (size_t)n * 4, hipMemcpyHostToDevice, c->stream);
    if (e != hipSuccess) return zi_hip_fail(e, "argmax H2D");
    zi_batch b;
    std::memset(&b, 0, sizeof b);
    b.logits = st.d;
    b.dtype = ZI_F32;
    b.rows = 1;
    b.vocab = (int32_t)n;
    b.ld = (int32_t)ld;
    char *dout = (char *)st.d + o_out;
    rc = zi_argmax_rows(c, &b, (uint32_t *)dout, (float *)(dout + 16), nullptr, nullptr);
    if (rc) return rc;
    e = hipMemcpyAsync((char *)st.h + o_out, dout, 32, hipMemcpyDeviceToHost, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return zi_hip_fail(e, "argmax D2H");
    *tok = *(uint32_t *)((char *)st.h + o_out);
    if (margin) *margin = *(float *)((char *)st.h + o_out + 16);
    return ZI_OK;
}

// ------------------------------------------------ Gen.AdaptiveDraft mirror
extern "C" void zi_adaptive_draft_init(zi_adaptive_draft *a, uint64_t max_k) {
    if (!a) return;
    a->cur_k = std::min<uint64_t>(max_k, 3);  // gen.zig:374-380
    a->max_k = max_k;
    a->min_k = 1;
    a->consecutive_rejections = 0;
    a->cooldown_steps = 0;
    a->last_margin = 2.0f;
}
extern "C" void zi_adaptive_draft_record_margin(zi_adaptive_draft *a, float m) {
    if (a) a->last_margin = m;
}
// The controller's entropy input (the reference reads the margin only): the
// margin m >= 0 at which the two-token softmax [m, 0] has entropy H (nats),
//   H2(m) = ln(1 + e^-m) + m e^-m / (1 + e^-m),
// strictly decreasing from ln 2 at m = 0 towards 0.  Inverted by bisection
// in f64; H >= ln 2 (or NaN) gives 0, H <= H2(kMaxEquivMargin) gives that cap.
static constexpr double kMaxEquivMargin = 100.0;
static double entropy_two_token(double m) {
    const double e = std::exp(-m);
    return std::log1p(e) + m * e / (1.0 + e);
}
extern "C" float zi_entropy_margin(float entropy) {
    const double H = (double)entropy;
    if (!(H < std::log(2.0))) return 0.0f;  // also NaN
    if (H <= entropy_two_token(kMaxEquivMargin)) return (float)kMaxEquivMargin;
    double lo = 0.0, hi = kMaxEquivMargin;  // H2(lo) > H >= H2(hi)
    for (int i = 0; i < 80; ++i) {
        const double mid = 0.5 * (lo + hi);
        if (entropy_two_token(mid) > H) lo = mid;
        else hi = mid;
    }
    return (float)(0.5 * (lo + hi));
}
extern "C" void zi_adaptive_draft_record_entropy(zi_adaptive_draft *a, float entropy) {
    if (a) a->last_margin = zi_entropy_margin(entropy);
}
extern "C" uint64_t zi_adaptive_draft_next(zi_adaptive_draft *a) {
    if (!a) return 0;
    if (a->cooldown_steps > 0) {  // gen.zig:388-405
        a->cooldown_steps -= 1;
        return 0;
    }
    uint64_t t = a->cur_k;
    if (a->last_margin >= 3.0f)
        t = std::min(a->max_k, std::max<uint64_t>(a->cur_k, 4));
    else if (a->last_margin >= 1.8f)
        t = std::min(a->max_k, std::max<uint64_t>(a->cur_k, 2));
    else if (a->last_margin < 0.9f)
        t = std::min<uint64_t>(t, 1);
    return t;
}
extern "C" void zi_adaptive_draft_update(zi_adaptive_draft *a, uint64_t accepted, uint64_t drafted,
                                         int32_t has_margin, float margin) {
    if (!a) return;
    if (has_margin) a->last_margin = margin;  // gen.zig:408-431
    if (drafted == 0) return;
    if (accepted == drafted) {
        a->consecutive_rejections = 0;
        if (a->cur_k < a->max_k) a->cur_k += 1;
    } else if (accepted > 0) {
        a->consecutive_rejections = 0;
        if (accepted * 2 < drafted && a->cur_k > a->min_k) a->cur_k -= 1;
    } else {
        a->consecutive_rejections += 1;
        if (a->cur_k > a->min_k) a->cur_k -= 1;
        if (a->consecutive_rejections >= 2) {
            a->cooldown_steps = 2;
            a->consecutive_rejections = 0;
            a->cur_k = std::min<uint64_t>(a->max_k, 2);
        }
    }
}
