/*
 * oracle.c -- CPU restatement of zinfer's sampler path.  TEST INFRASTRUCTURE
 * ONLY (see oracle.h for scope and the pinning status of each function).
 *
 * Citations are file:line in the reference repository (pylypenko99/zinfer).
 * All arithmetic is sequential IEEE f32 in the order the Zig source performs
 * it; build with -ffp-contract=off.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

float or_exp32(float x) { return (float)exp((double)x); }
float or_log32(float x) { return (float)log((double)x); }

/* The reference's f32 @exp (src/sampler.zig:219, 222, 230, 240; the softcap
 * body, src/model.zig:2505).  The reference links no libc (build.zig:14), so
 * @exp(f32) is a call to the Zig compiler runtime's expf, a port of musl's
 * expf (FreeBSD e_expf.c).  Restated from that published algorithm, every step
 * an f32 operation in the published order:
 *   |x| > ln2/2 (0x3eb17218): k = (int)(invln2*x + (x < 0 ? -0.5 : 0.5)), or
 *     k = +-1 when |x| <= 1.5 ln2 (0x3f851592); hi = x - k*ln2hi (exact),
 *     lo = k*ln2lo, x = hi - lo;
 *   |x| > 2^-13 (0x39000000): k = 0, hi = x, lo = 0;  else return 1 + x;
 *   c = x - x^2*(P1 + x^2*P2);  y = 1 + (x*c/(2 - c) - lo + hi);
 *   return k ? scalbnf(y, k) : y   (scalbnf: one rounding).
 * Special cases: NaN -> NaN, x >= 88.722839 (0x42b17218) -> inf, x <=
 * -103.972084 (0x42cff1b5) -> 0.  Pinned by tests/test_oracle_expf.py (error
 * within 1 ulp of exp over dense grids, the special cases and boundaries, and
 * the branch identities); that Zig 0.17.1's compiler runtime still carries
 * this port is not checkable here (no Zig toolchain). */
static float zf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t zb(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float or_scalbnf(float y, int n) {
    if (n > 127) {
        y *= 0x1p127f;
        n -= 127;
        if (n > 127) {
            y *= 0x1p127f;
            n -= 127;
            if (n > 127) n = 127;
        }
    } else if (n < -126) {
        y *= 0x1p-102f;
        n += 102;
        if (n < -126) {
            y *= 0x1p-102f;
            n += 102;
            if (n < -126) n = -126;
        }
    }
    return y * zf((uint32_t)(0x7f + n) << 23);
}

float or_zexpf(float x) {
    const float half[2] = {0.5f, -0.5f};
    const float ln2hi = zf(0x3f317200u), ln2lo = zf(0x35bfbe8eu), invln2 = zf(0x3fb8aa3bu);
    const float P1 = 11184783.0f * 0x1p-26f;  /* 0xaaaa8f.0p-26 */
    const float P2 = -11883029.0f * 0x1p-32f; /* -0xb55215.0p-32 */
    uint32_t hx = zb(x);
    const int sign = (int)(hx >> 31);
    hx &= 0x7fffffffu;
    if (hx >= 0x42aeac50u) {
        if (hx > 0x7f800000u) return x;
        if (hx >= 0x42b17218u && !sign) return x * 0x1p127f;
        if (sign && hx >= 0x42cff1b5u) return 0.0f;
    }
    int k;
    float hi, lo;
    if (hx > 0x3eb17218u) {
        if (hx > 0x3f851592u) k = (int)(invln2 * x + half[sign]);
        else k = 1 - sign - sign;
        hi = x - (float)k * ln2hi;
        lo = (float)k * ln2lo;
        x = hi - lo;
    } else if (hx > 0x39000000u) {
        k = 0;
        hi = x;
        lo = 0.0f;
    } else {
        return 1.0f + x;
    }
    const float xx = x * x;
    const float c = x - xx * (P1 + xx * P2);
    const float y = 1.0f + (x * c / (2.0f - c) - lo + hi);
    return k == 0 ? y : or_scalbnf(y, k);
}

void or_zexpf_array(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = or_zexpf(x[i]);
}
/* std.math.tanh(f32) (model.zig:2512, the softcap's scalar tail), as the f64
 * tanh rounded once to f32: within half an ulp plus the f64 error, the same
 * footing as or_exp32. */
float or_tanh32(float x) { return (float)tanh((double)x); }

/* std.math.pow(f32, x, y) as Zig computes it (src/sampler.zig:182 calls it for
 * the DRY penalty).  Zig's lib/std/math/pow.zig (Zig 0.17.1, not in the
 * reference tree) restates Go's math.Pow: special cases; x^yf = exp(yf*log(x))
 * for the fractional part (yf moved into (-0.5, 0.5]); x^yi by repeated
 * squaring of frexp(x)'s significand in f32 with the binary exponent carried
 * separately (overflow guard at |xe| > 2^9 for f32); 1/a for y < 0; scalbn.
 * exp/log: or_exp32 / or_log32.  Last-ulp agreement with Zig is PARITY
 * UNPINNED (no Zig toolchain); the special cases, integer powers and the
 * fractional split are pinned in tests. */
static int pow_odd_int(float y) {
    if (!(fabsf(y) < 16777216.0f)) return 0;
    float t = truncf(y);
    return t == y && fmodf(t, 2.0f) != 0.0f;
}

float or_pow_zig(float x, float y) {
    if (y == 0.0f || x == 1.0f) return 1.0f;
    if (isnan(x) || isnan(y)) return NAN;
    if (y == 1.0f) return x;
    if (x == 0.0f) {
        if (y < 0.0f) return pow_odd_int(y) ? copysignf(INFINITY, x) : INFINITY;
        return pow_odd_int(y) ? x : 0.0f;
    }
    if (isinf(y)) {
        if (x == -1.0f) return 1.0f;
        return ((fabsf(x) < 1.0f) == (y > 0.0f)) ? 0.0f : INFINITY;
    }
    if (isinf(x)) {
        if (x < 0.0f) return or_pow_zig(1.0f / x, -y);
        return y < 0.0f ? 0.0f : INFINITY;
    }
    if (y == 0.5f) return sqrtf(x);
    if (y == -0.5f) return 1.0f / sqrtf(x);
    float yi, yf = modff(fabsf(y), &yi);
    if (yf != 0.0f && x < 0.0f) return NAN;
    if (yi >= 2147483648.0f) {
        if (x == -1.0f) return 1.0f;
        return ((fabsf(x) < 1.0f) == (y > 0.0f)) ? 0.0f : INFINITY;
    }
    float a1 = 1.0f;
    int ae = 0;
    if (yf != 0.0f) {
        if (yf > 0.5f) { yf -= 1.0f; yi += 1.0f; }
        a1 = or_exp32(yf * or_log32(x));
    }
    int xe;
    float x1 = frexpf(x, &xe);
    for (int32_t i = (int32_t)yi; i != 0; i >>= 1) {
        if (xe < -(1 << 9) || (1 << 9) < xe) { ae += xe; break; }
        if (i & 1) { a1 *= x1; ae += xe; }
        x1 *= x1;
        xe <<= 1;
        if (x1 < 0.5f) { x1 += x1; xe -= 1; }
    }
    if (y < 0.0f) { a1 = 1.0f / a1; ae = -ae; }
    return ldexpf(a1, ae);
}

void or_params_default(or_params *p) {
    /* src/sampler.zig:3-27 defaults; the extension fields are neutral and the
     * window is the reference's repeat_last_n = 64 (src/sampler.zig:30). */
    p->temp = 0.8f;
    p->top_k = 40;
    p->top_p = 0.95f;
    p->min_p = 0.05f;
    p->repeat_penalty = 1.0f;
    p->freq_penalty = 0.0f;
    p->presence_penalty = 0.0f;
    p->penalty_last_n = 64;
    p->dry_multiplier = 0.0f;
    p->dry_base = 1.75f;
    p->dry_allowed_length = 2;
    p->dry_range = 1024;
    p->xtc_probability = 0.0f;
    p->xtc_threshold = 0.1f;
    p->xtc_min_keep = 1;
    p->final_logit_softcap = 0.0f;
}

/* The final-logit softcap of src/model.zig:2492-2510 (the vectorized body,
 * i < 32*floor(V/32)): z = l * (1/cap) with 1/cap in f32, clamped to [-9, 9],
 * e = exp(2z), tanh = (e - 1) / (e + 1), l = cap * tanh.  Every sequence step
 * rounds to f32; exp is or_zexpf (the reference's expf). */
/* The scalar tail of the same loop (model.zig:2511-2513, ids >= 32*floor(V/32)):
 * l = cap * tanh(l / cap), a true division and no clamp, so -inf maps to -cap
 * (the body maps it to -cap*tanh(9)). */
float or_softcap_tail(float l, float cap) { return cap * or_tanh32(l / cap); }

float or_softcap(float l, float cap) {
    const float inv_cap = 1.0f / cap;
    /* @min(@max(z, -9), 9) lowers to maxnum/minnum: a NaN operand yields the other */
    const float z = fminf(fmaxf(l * inv_cap, -9.0f), 9.0f);
    const float e2z = or_zexpf(z * 2.0f);
    const float t = (e2z - 1.0f) / (e2z + 1.0f);
    return cap * t;
}

/* src/sampler.zig:91-100.  Each distinct id of the window is penalized once
 * (first-occurrence test, :96): l = l > 0 ? l / rp : l * rp.  The reference
 * returns early when rp == 1 (:92).  Extension (not in the reference): after
 * the repetition step, l -= count * freq + presence for ids with count > 0,
 * evaluated as fl(fl(fl(count) * freq) + presence) then fl(l - that). */
void or_apply_penalty(float *logits, uint32_t V, const uint32_t *window, uint32_t n, float rp,
                      float freq, float pres) {
    int do_rep = rp != 1.0f;
    int do_fp = freq != 0.0f || pres != 0.0f;
    if (!do_rep && !do_fp) return;
    for (uint32_t i = 0; i < n; ++i) {
        uint32_t tok = window[i];
        int seen = 0;
        for (uint32_t j = 0; j < i; ++j)
            if (window[j] == tok) { seen = 1; break; }
        if (seen) continue;
        if (tok >= V) continue; /* out-of-range ids are ignored (Zig would trap) */
        float *l = &logits[tok];
        if (do_rep) *l = (*l > 0.0f) ? *l / rp : *l * rp;
        if (do_fp) {
            uint32_t count = 0;
            for (uint32_t j = 0; j < n; ++j) count += window[j] == tok;
            float c = (float)count;
            float t = c * freq;
            t = t + pres;
            *l = *l - t;
        }
    }
}

void or_apply_edits(float *logits, uint32_t V, const uint32_t *ids, const float *deltas,
                    uint32_t n) {
    for (uint32_t i = 0; i < n; ++i)
        if (ids[i] < V) logits[ids[i]] -= deltas[i]; /* src/sampler.zig:180-184 */
}

static int is_breaker(const uint32_t *b, uint32_t nb, uint32_t tok) {
    for (uint32_t i = 0; i < nb; ++i)
        if (b[i] == tok) return 1; /* src/sampler.zig:76-81 */
    return 0;
}

/* src/sampler.zig:104-187.  hist is the linear history, oldest first; the
 * reference keeps the last max_history = 4096 tokens in a ring (:31, :87), so
 * R[k] = hist[n_hist - 1 - k] for k < min(n_hist, 4096). */
uint32_t or_dry_edits(const uint32_t *hist, uint32_t n_hist, const uint32_t *breakers,
                      uint32_t n_breakers, float mult, float base, uint32_t allowed,
                      uint32_t range, uint32_t *out_ids, float *out_deltas) {
    enum { MAX_HISTORY = 4096, MAX_PENALIZED = 128 };
    if (mult == 0.0f || base < 1.0f || range == 0) return 0; /* :105 */
    uint32_t L = n_hist;
    uint32_t lim = range < MAX_HISTORY ? range : MAX_HISTORY;
    if (L > lim) L = lim; /* :106 */
    if (L <= allowed) return 0; /* :107 */
#define R(k) hist[n_hist - 1 - (k)]
    uint32_t rep_limit = L; /* :112-119 */
    for (uint32_t k = 0; k < L; ++k)
        if (is_breaker(breakers, n_breakers, R(k))) { rep_limit = k; break; }
    if (rep_limit < allowed) return 0; /* :120 */

    static uint32_t z[MAX_HISTORY];
    z[0] = 0; /* :126-147, Z-algorithm over the reversed stream */
    uint32_t l = 0, r = 0;
    for (uint32_t i = 1; i < L; ++i) {
        if (i <= r) {
            uint32_t a = r - i + 1, b = z[i - l];
            z[i] = a < b ? a : b;
        } else {
            z[i] = 0;
        }
        uint32_t max_z = L - i < rep_limit ? L - i : rep_limit;
        while (z[i] < max_z) {
            if (R(z[i]) != R(i + z[i])) break;
            z[i] += 1;
        }
        if (i + z[i] > 0 && i + z[i] - 1 > r) {
            l = i;
            r = i + z[i] - 1;
        }
    }

    uint32_t pen_toks[MAX_PENALIZED]; /* :150-175 */
    uint32_t pen_lens[MAX_PENALIZED];
    uint32_t n_pen = 0;
    for (uint32_t k = 1; k < L; ++k) {
        uint32_t rlen = z[k];
        if (rlen >= allowed) {
            uint32_t cont = R(k - 1);
            if (is_breaker(breakers, n_breakers, cont)) continue;
            int found = 0;
            for (uint32_t pi = 0; pi < n_pen; ++pi) {
                if (pen_toks[pi] == cont) {
                    if (rlen > pen_lens[pi]) pen_lens[pi] = rlen;
                    found = 1;
                    break;
                }
            }
            if (!found && n_pen < MAX_PENALIZED) {
                pen_toks[n_pen] = cont;
                pen_lens[n_pen] = rlen;
                n_pen += 1;
            }
        }
    }
#undef R
    /* :178-186: penalty = mult * pow(base, min(rlen - allowed, max_exp)), with
     * @log and std.math.pow as or_log32 / or_pow_zig */
    float max_exp = (base > 1.0001f) ? 88.0f / or_log32(base) : 100.0f;
    for (uint32_t i = 0; i < n_pen; ++i) {
        float repeat_exp = (float)(pen_lens[i] - allowed);
        float e = repeat_exp < max_exp ? repeat_exp : max_exp;
        out_ids[i] = pen_toks[i];
        out_deltas[i] = mult * or_pow_zig(base, e);
    }
    return n_pen;
}

void or_apply_mask(float *logits, uint32_t V, const uint32_t *words) {
    for (uint32_t id = 0; id < V; ++id)
        if (!((words[id >> 5] >> (id & 31)) & 1u)) logits[id] = -INFINITY;
}

/* src/sampler.zig:532-610. */
or_result or_argmax_with_margin(const float *x, uint32_t n) {
    or_result res;
    if (n == 0) { res.tok = 0; res.margin = 0.0f; return res; } /* :533 */
    if (n == 1) { res.tok = 0; res.margin = 10.0f; return res; } /* :534 */
    if (n < 16) { /* :535-551 */
        uint32_t best = 0, second = 1;
        if (x[1] > x[0]) { best = 1; second = 0; }
        for (uint32_t i = 2; i < n; ++i) {
            if (x[i] > x[best]) { second = best; best = i; }
            else if (x[i] > x[second]) { second = i; }
        }
        res.tok = best;
        res.margin = x[best] - x[second];
        return res;
    }
    /* :553-573: 16 lane classes (two 8-wide vectors), strict > keeps the first max */
    float mx[16];
    uint32_t ix[16];
    for (int c = 0; c < 16; ++c) { mx[c] = x[c]; ix[c] = (uint32_t)c; }
    uint32_t i = 16;
    for (; i + 16 <= n; i += 16)
        for (int c = 0; c < 16; ++c)
            if (x[i + c] > mx[c]) { mx[c] = x[i + c]; ix[c] = i + (uint32_t)c; }
    /* :575-596: reduce lane j of max0 (class j), then lane j of max1 (class j+8) */
    float best_val = -INFINITY, second_val = -INFINITY;
    uint32_t best_idx = 0;
    for (int j = 0; j < 8; ++j) {
        for (int h = 0; h < 2; ++h) {
            int c = j + 8 * h;
            float v = mx[c];
            if (v > best_val) { second_val = best_val; best_val = v; best_idx = ix[c]; }
            else if (v > second_val) { second_val = v; }
        }
    }
    for (; i < n; ++i) { /* :598-606 tail */
        if (x[i] > best_val) { second_val = best_val; best_val = x[i]; best_idx = i; }
        else if (x[i] > second_val) { second_val = x[i]; }
    }
    res.tok = best_idx; /* :608-609 */
    res.margin = (second_val > -INFINITY) ? best_val - second_val : 10.0f;
    return res;
}

or_result or_argmax_true(const float *x, uint32_t n) {
    or_result res;
    if (n == 0) { res.tok = 0; res.margin = 0.0f; return res; }
    uint32_t best = 0;
    for (uint32_t i = 1; i < n; ++i)
        if (x[i] > x[best]) best = i;
    float second = -INFINITY;
    for (uint32_t i = 0; i < n; ++i)
        if (i != best && x[i] > second) second = x[i];
    res.tok = best;
    res.margin = (second > -INFINITY) ? x[best] - second : 10.0f;
    return res;
}

typedef struct { uint32_t id; float v; } cand_t;

/* std.mem.sort(Cand, ..., gt) (src/sampler.zig:201, :283-285) is a stable sort
 * by v descending; restated as a stable bottom-up merge sort. */
static void stable_sort_desc(cand_t *a, uint32_t n) {
    cand_t *tmp = (cand_t *)malloc((size_t)n * sizeof(cand_t));
    for (uint32_t w = 1; w < n; w *= 2) {
        for (uint32_t lo = 0; lo < n; lo += 2 * w) {
            uint32_t mid = lo + w < n ? lo + w : n;
            uint32_t hi = lo + 2 * w < n ? lo + 2 * w : n;
            uint32_t i = lo, j = mid, o = lo;
            while (i < mid && j < hi) {
                /* take from the right only when strictly greater: stable */
                if (a[j].v > a[i].v) tmp[o++] = a[j++];
                else tmp[o++] = a[i++];
            }
            while (i < mid) tmp[o++] = a[i++];
            while (j < hi) tmp[o++] = a[j++];
        }
        memcpy(a, tmp, (size_t)n * sizeof(cand_t));
    }
    free(tmp);
}

/* Sampler.cand (src/sampler.zig:41, :53), one per calling thread so that the
 * CPU baseline can run rows on several threads at once. */
static _Thread_local cand_t *g_cand = NULL;
static _Thread_local uint32_t g_cand_cap = 0;
static _Thread_local float *g_w = NULL;

static void ensure_cand(uint32_t V) {
    if (V > g_cand_cap) {
        free(g_cand);
        free(g_w);
        g_cand = (cand_t *)malloc((size_t)V * sizeof(cand_t));
        g_w = (float *)malloc((size_t)V * sizeof(float));
        g_cand_cap = V;
    }
}

/* src/sampler.zig:193-276 with u[0], u[1] in place of the rng draws. */
or_result or_sample_penalized(const or_params *p, const float *logits, uint32_t V,
                              const float *u, or_sample_diag *diag) {
    or_result res;
    if (diag) { diag->ndraws = 0; diag->n = 0; diag->keep = 0; diag->start = 0; diag->total = 0; }
    if (p->temp <= 0.0f) { /* :193 */
        res = or_argmax_with_margin(logits, V);
        if (diag) { diag->n = 1; diag->keep = 1; }
        return res;
    }
    ensure_cand(V);
    cand_t *c = g_cand;
    uint32_t n = 0; /* :196-210 */
    uint32_t k = (p->top_k == 0 || p->top_k > V) ? V : p->top_k;
    if (k == V) {
        for (uint32_t i = 0; i < V; ++i) { c[i].id = i; c[i].v = logits[i]; }
        n = V;
        stable_sort_desc(c, n);
    } else {
        for (uint32_t i = 0; i < V; ++i) {
            float v = logits[i];
            if (n == k && v <= c[k - 1].v) continue;
            uint32_t j = (n < k) ? n : k - 1;
            if (n < k) n += 1;
            while (j > 0 && c[j - 1].v < v) { c[j] = c[j - 1]; j -= 1; }
            c[j].id = i;
            c[j].v = v;
        }
    }
    float mx = c[0].v; /* :211-213 */
    float margin = (n >= 2) ? mx - c[1].v : 10.0f;

    uint32_t keep = n; /* :215-228 */
    if (p->top_p < 1.0f) {
        float total = 0.0f;
        for (uint32_t i = 0; i < n; ++i) total += or_zexpf(c[i].v - mx);
        float acc = 0.0f;
        for (uint32_t i = 0; i < n; ++i) {
            acc += or_zexpf(c[i].v - mx);
            if (acc >= p->top_p * total) { keep = i + 1; break; }
        }
    }
    if (p->min_p > 0.0f) { /* :229-234 */
        for (uint32_t i = 0; i < keep; ++i)
            if (or_zexpf(c[i].v - mx) < p->min_p) { keep = i > 1 ? i : 1; break; }
    }

    float inv_t = 1.0f / p->temp; /* :236-242 */
    float total = 0.0f;
    float *w = g_w;
    for (uint32_t i = 0; i < keep; ++i) {
        w[i] = or_zexpf((c[i].v - mx) * inv_t);
        total += w[i];
    }

    uint32_t start = 0; /* :244-268 */
    int draws = 0;
    if (p->xtc_probability > 0.0f && p->xtc_threshold <= 0.5f && keep >= 2 && total > 0.0f) {
        float chance = u[draws++];
        if (chance <= p->xtc_probability) {
            float inv_tot = 1.0f / total;
            uint32_t pos_last = 0;
            for (uint32_t i = 0; i < keep; ++i) {
                float prob = w[i] * inv_tot;
                if (prob >= p->xtc_threshold) pos_last = i;
                else break;
            }
            uint32_t min_keep = p->xtc_min_keep > 1 ? p->xtc_min_keep : 1;
            if (keep - pos_last >= min_keep && pos_last > 0) {
                start = pos_last;
                total = 0.0f;
                for (uint32_t i = start; i < keep; ++i) total += w[i];
            }
        }
    }

    float r = u[draws++] * total; /* :270-275 */
    res.tok = c[keep - 1].id;
    res.margin = margin;
    for (uint32_t i = start; i < keep; ++i) {
        r -= w[i];
        if (r <= 0.0f) { res.tok = c[i].id; break; }
    }
    if (diag) {
        diag->ndraws = draws;
        diag->n = (int32_t)n;
        diag->keep = (int32_t)keep;
        diag->start = (int32_t)start;
        diag->total = total;
        uint32_t m = (uint32_t)diag->cap < n ? (uint32_t)diag->cap : n;
        for (uint32_t i = 0; i < m; ++i) {
            if (diag->ids) diag->ids[i] = c[i].id;
            if (diag->vals) diag->vals[i] = c[i].v;
            if (diag->probs) diag->probs[i] = (i >= start && i < keep) ? w[i] / total : 0.0f;
        }
    }
    return res;
}

or_result or_sample_row(const or_params *p, float *logits, uint32_t V, const uint32_t *mask,
                        const uint32_t *window, uint32_t n_window, const uint32_t *edit_ids,
                        const float *edit_deltas, uint32_t n_edits, const float *u,
                        or_sample_diag *diag) {
    if (p->final_logit_softcap > 0.0f) { /* the model's epilogue, model.zig:2492-2514 */
        const float cap = p->final_logit_softcap;
        const uint32_t body = V / 32 * 32;
        for (uint32_t i = 0; i < body; ++i) logits[i] = or_softcap(logits[i], cap);
        /* the scalar tail, ids >= 32*floor(V/32) (:2511-2513) */
        for (uint32_t i = body; i < V; ++i) logits[i] = or_softcap_tail(logits[i], cap);
    }
    if (mask) or_apply_mask(logits, V, mask); /* gen.zig:457-460: mask precedes sample */
    or_apply_penalty(logits, V, window, n_window, p->repeat_penalty, p->freq_penalty,
                     p->presence_penalty); /* sampler.zig:191 */
    if (edit_ids && n_edits) or_apply_edits(logits, V, edit_ids, edit_deltas, n_edits); /* :192 */
    return or_sample_penalized(p, logits, V, u, diag);
}

void or_entropy_topk(const float *x, uint32_t V, uint32_t k, double *entropy, uint32_t *ids,
                     double *probs) {
    double m = -INFINITY;
    for (uint32_t i = 0; i < V; ++i)
        if (x[i] > m) m = x[i];
    double z = 0.0, a = 0.0;
    for (uint32_t i = 0; i < V; ++i) {
        if (x[i] == -INFINITY) continue;
        double d = (double)x[i] - m;
        double e = exp(d);
        z += e;
        a += e * d;
    }
    /* H = -sum p ln p = ln Z - sum e_i d_i / Z with d_i = x_i - max */
    *entropy = log(z) - a / z;
    /* top-k by (value desc, id asc): insertion like sampler.zig:203-209 */
    uint32_t n = 0;
    if (k > V) k = V;
    cand_t buf[1024];
    if (k > 1024) k = 1024;
    for (uint32_t i = 0; i < V; ++i) {
        float v = x[i];
        if (n == k && v <= buf[k - 1].v) continue;
        uint32_t j = (n < k) ? n : k - 1;
        if (n < k) n += 1;
        while (j > 0 && buf[j - 1].v < v) { buf[j] = buf[j - 1]; j -= 1; }
        buf[j].id = i;
        buf[j].v = v;
    }
    for (uint32_t i = 0; i < n; ++i) {
        ids[i] = buf[i].id;
        probs[i] = exp((double)buf[i].v - m) / z;
    }
}

/* gen.zig:366-432 */
void or_adaptive_init(or_adaptive *a, uint64_t max_k) {
    a->cur_k = max_k < 3 ? max_k : 3;
    a->max_k = max_k;
    a->min_k = 1;
    a->consecutive_rejections = 0;
    a->cooldown_steps = 0;
    a->last_margin = 2.0f;
}
void or_adaptive_record_margin(or_adaptive *a, float m) { a->last_margin = m; }
static uint64_t umin(uint64_t a, uint64_t b) { return a < b ? a : b; }
static uint64_t umax(uint64_t a, uint64_t b) { return a > b ? a : b; }
uint64_t or_adaptive_next(or_adaptive *a) {
    if (a->cooldown_steps > 0) { a->cooldown_steps -= 1; return 0; }
    uint64_t t = a->cur_k;
    if (a->last_margin >= 3.0f) t = umin(a->max_k, umax(a->cur_k, 4));
    else if (a->last_margin >= 1.8f) t = umin(a->max_k, umax(a->cur_k, 2));
    else if (a->last_margin < 0.9f) t = umin(t, 1);
    return t;
}
void or_adaptive_update(or_adaptive *a, uint64_t accepted, uint64_t drafted, int has_margin,
                        float margin) {
    if (has_margin) a->last_margin = margin;
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
            a->cur_k = umin(a->max_k, 2);
        }
    }
}

/* splitmix64 (Steele, Lea, Flood 2014; Vigna's public-domain reference). */
uint64_t or_splitmix64_next(uint64_t *state) {
    uint64_t z = (*state += 0x9e3779b97f4a7c15ULL);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
/* xoshiro256++ (Blackman and Vigna 2018), seeded by four splitmix64 outputs. */
void or_xoshiro_seed(uint64_t s[4], uint64_t seed) {
    uint64_t st = seed;
    for (int i = 0; i < 4; ++i) s[i] = or_splitmix64_next(&st);
}
static uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
uint64_t or_xoshiro_next(uint64_t s[4]) {
    uint64_t result = rotl64(s[0] + s[3], 23) + s[0];
    uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl64(s[3], 45);
    return result;
}
/* Random.float(f32): 23 low bits are the mantissa; the exponent is 126 minus
 * the count of leading zeros of the same 64-bit draw (more draws if >= 41). */
float or_rand_f32(uint64_t s[4]) {
    uint64_t rnd = or_xoshiro_next(s);
    uint32_t lz = rnd ? (uint32_t)__builtin_clzll(rnd) : 64;
    if (lz >= 41) {
        uint64_t r2 = or_xoshiro_next(s);
        lz = 41 + (r2 ? (uint32_t)__builtin_clzll(r2) : 64);
        if (lz == 41 + 64) {
            uint32_t r3 = (uint32_t)or_xoshiro_next(s) | 0x7FFu;
            lz += (uint32_t)__builtin_clz(r3);
        }
    }
    uint32_t mant = (uint32_t)(rnd & 0x7FFFFFu);
    uint32_t bits = ((126u - lz) << 23) | mant;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

double or_bench_sample_rows(const or_params *p, const float *logits, uint32_t rows, uint32_t V,
                            uint64_t ld, const uint32_t *hist, const int32_t *hist_len,
                            uint32_t hist_ld, const uint32_t *mask, uint32_t mask_ld,
                            const float *uniforms, uint32_t reps, uint32_t *out_tok,
                            float *out_margin) {
    float *row = (float *)malloc((size_t)V * sizeof(float));
    double t = 0.0;
    for (uint32_t rep = 0; rep < reps; ++rep) {
        for (uint32_t r = 0; r < rows; ++r) {
            memcpy(row, logits + (size_t)r * ld, (size_t)V * sizeof(float));
            const uint32_t *win = NULL;
            uint32_t nw = 0;
            if (hist && hist_len) {
                uint32_t hl = (uint32_t)hist_len[r];
                nw = hl < p->penalty_last_n ? hl : p->penalty_last_n;
                win = hist + (size_t)r * hist_ld + (hl - nw);
            }
            const uint32_t *mk = mask ? mask + (size_t)r * mask_ld : NULL;
            double t0 = now_s();
            or_result res = or_sample_row(p, row, V, mk, win, nw, NULL, NULL, 0,
                                          uniforms + 2 * (size_t)r, NULL);
            t += now_s() - t0;
            if (out_tok) out_tok[r] = res.tok;
            if (out_margin) out_margin[r] = res.margin;
        }
    }
    free(row);
    return t;
}
