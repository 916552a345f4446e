/*
 * oracle.h -- CPU restatement of zinfer's sampling / constrained-decoding path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (zinfer_amd/, include/)
 * links, loads or calls this code.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, as the checker and as the timed CPU
 * baseline ("port").
 *
 * The reference (pylypenko99/zinfer) is Zig 0.17.1; no Zig toolchain exists in
 * this image, so the reference cannot be built (oracle/_ref stays empty).  Each
 * function below restates one reference function, cited file:line relative to
 * the reference repository root, in plain C with the same sequential f32
 * arithmetic.  Compile with -ffp-contract=off (no FMA contraction): every
 * product and sum must round on its own, as in the Zig source.
 *
 * Pinning status (how each function is checked before it is trusted):
 *   or_argmax_with_margin  pinned: reference KAT sampler.zig:616-632, plus an
 *                          independent numpy model of the 2x8-lane reduction on
 *                          tie-heavy inputs.
 *   or_apply_penalty       pinned: closed forms (l/rp, l*rp, count*freq+pres) on
 *                          crafted windows.
 *   or_dry_edits           pinned: reference KAT sampler.zig:634-673 (9.2, 8.4,
 *                          breaker keeps 10.0) and brute-force longest-suffix match.
 *   or_pow_zig             std.math.pow restated (Go math.Pow algorithm): special
 *                          cases, integer powers within the repeated-squaring
 *                          bound of the f64 closed form, the fractional split;
 *                          last-ulp agreement with Zig PARITY UNPINNED (no Zig).
 *   or_sample              pinned: KATs sampler.zig:675-702 (min-p) and :704-748
 *                          (XTC); top-k order vs numpy lexsort; top-p keep vs numpy
 *                          float32 add.accumulate; draw vs inverse-CDF on
 *                          float32 running remainders; empirical draw frequencies.
 *   or_apply_mask          pinned: closed form (bit test -> -inf).
 *   or_entropy_topk        pinned: scipy.stats.entropy(softmax) and brute-force top-k.
 *   or_adaptive_*          pinned: reference KAT gen.zig:845-874.
 *   or_json_*              pinned: reference KATs grammar.zig:482-513; json.dumps
 *                          documents are accepted with every prefix; every text
 *                          accepted to the finished state parses with json.loads;
 *                          hand-derived byte tables per state (the \\u quirk, the
 *                          depth-64 limit, object-only roots).
 *   or_xoshiro_*           linear engine pinned (tests/test_oracle_rng.py): the
 *                          GF(2) update matrix has full period 2^256 - 1 (checked
 *                          against every prime of 2^256 - 1) and reproduces the
 *                          published JUMP / LONG_JUMP polynomials (2^128 and 2^192
 *                          steps); seeding by splitmix64 is pinned by splitmix64's
 *                          published sequence for seed 1234567.  The ++ output
 *                          scrambler rotl(s0 + s3, 23) + s0 is PARITY UNPINNED (no
 *                          Zig and no published output vectors here).
 *   or_rand_f32            pinned: crafted states with chosen outputs give
 *                          2^-(1+lz) * (1 + m/2^23) (m = low 23 bits of the first
 *                          draw; lz extended by the second draw from 41 leading
 *                          zeros on), computed independently with ldexp.  The
 *                          third-draw branch (probability 2^-105) is unpinned.
 *   or_softcap             pinned: within cap*2^-22 of the f64 closed form, odd,
 *                          saturation and special values.
 *   or_softcap_tail        pinned: within two f32 ulps of cap*tanh(fl(l/cap)) in f64,
 *                          odd, +-inf -> +-cap, and applied to exactly the ids at
 *                          and above 32*floor(V/32) (tests/test_oracle_properties.py).
 *   or_zexpf               the reference's @exp(f32) on the sampling path: the
 *                          compiler runtime's expf (the reference links no libc),
 *                          a port of musl's / FreeBSD's expf, restated from that
 *                          published algorithm.  Pinned (tests/test_oracle_expf.py):
 *                          within 1 ulp of exp over dense grids (subnormal results
 *                          included), the special values and thresholds, the
 *                          |x| <= 2^-13 branch (1 + x), both sides of the reduction
 *                          branches' boundaries, and not correctly rounded (it is
 *                          not the f64-rounded exp; planting an f64 evaluation or a
 *                          perturbed P2 fails the tests).  That Zig 0.17.1's
 *                          runtime still ships this port is not checkable here (no
 *                          Zig toolchain).
 *   tanh, pow's exp/log    std.math.tanh (softcap tail) and std.math.pow's exp/log
 *                          last-ulp bits are PARITY UNPINNED; the oracle and the
 *                          device use (float)tanh((double)x), (float)exp((double)x)
 *                          and (float)log((double)x), correctly rounded in practice.
 */
#ifndef ZINFER_ORACLE_H
#define ZINFER_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Params, src/sampler.zig:3-27, plus the frequency/presence extension and the
 * penalty window (fixed at 64 in the reference, src/sampler.zig:30). */
typedef struct or_params {
    float    temp;
    uint32_t top_k;
    float    top_p;
    float    min_p;
    float    repeat_penalty;
    float    freq_penalty;
    float    presence_penalty;
    uint32_t penalty_last_n;
    float    dry_multiplier;
    float    dry_base;
    uint32_t dry_allowed_length;
    uint32_t dry_range;
    float    xtc_probability;
    float    xtc_threshold;
    uint32_t xtc_min_keep;
    float    final_logit_softcap; /* 0 = off; applied to the row before the mask (src/model.zig:2492-2514) */
} or_params;

/* SampleResult, src/sampler.zig:527-530 */
typedef struct or_result {
    uint32_t tok;
    float    margin;
} or_result;

typedef struct or_sample_diag {
    int32_t   ndraws; /* uniforms consumed: 0 (greedy), 1, or 2 (XTC chance drawn) */
    int32_t   n;      /* candidates after top-k */
    int32_t   keep;   /* after top-p and min-p */
    int32_t   start;  /* XTC start index */
    float     total;  /* weight total the draw scales */
    int32_t   cap;    /* capacity of ids/vals/probs (0 = none) */
    uint32_t *ids;    /* candidate ids in order */
    float    *vals;   /* penalized logits in order */
    float    *probs;  /* w_i / total for start <= i < keep, else 0 */
} or_sample_diag;

float or_exp32(float x);
float or_zexpf(float x);
void or_zexpf_array(const float *x, float *y, int64_t n);
float or_log32(float x);
float or_tanh32(float x);
float or_pow_zig(float x, float y);

void or_params_default(or_params *p);

/* src/sampler.zig:91-100 (+ frequency/presence extension, window = caller's). */
void or_apply_penalty(float *logits, uint32_t V, const uint32_t *window, uint32_t n,
                      float rp, float freq, float pres);

/* Subtractive sparse edits: logits[id] -= delta (the DRY step, src/sampler.zig:184). */
void or_apply_edits(float *logits, uint32_t V, const uint32_t *ids, const float *deltas,
                    uint32_t n);

/* src/sampler.zig:104-187: DRY edits from a linear history (oldest first). */
uint32_t or_dry_edits(const uint32_t *hist, uint32_t n_hist, const uint32_t *breakers,
                      uint32_t n_breakers, float mult, float base, uint32_t allowed,
                      uint32_t range, uint32_t *out_ids, float *out_deltas);

/* src/grammar.zig:446-479 restated for a packed allowed-mask:
 * id allowed <=> (words[id >> 5] >> (id & 31)) & 1. */
void or_apply_mask(float *logits, uint32_t V, const uint32_t *words);

/* src/sampler.zig:532-610 (2x8-lane SIMD tie and margin semantics). */
or_result or_argmax_with_margin(const float *x, uint32_t n);

/* Lowest-index argmax with the true top-1 minus top-2 gap (new semantics). */
or_result or_argmax_true(const float *x, uint32_t n);

/* src/sampler.zig:190-276 after the penalty, with injected uniforms u[0], u[1]
 * standing in for the first and second rng.float(f32) draws.  `logits` is the
 * already-penalized row; it is not modified. */
or_result or_sample_penalized(const or_params *p, const float *logits, uint32_t V,
                              const float *u, or_sample_diag *diag);

/* Whole-row pipeline as gen.zig drives it: mask (optional), penalty over the
 * window, sparse edits, then or_sample_penalized.  `logits` is modified in place
 * like the reference's sampleWithMargin. */
or_result or_sample_row(const or_params *p, float *logits, uint32_t V, const uint32_t *mask,
                        const uint32_t *window, uint32_t n_window, const uint32_t *edit_ids,
                        const float *edit_deltas, uint32_t n_edits, const float *u,
                        or_sample_diag *diag);

/* New semantics (entropy of the T=1 full-vocab softmax, nats; top-k ids in
 * (value desc, id asc) order with full-vocab normalized probabilities). */
void or_entropy_topk(const float *x, uint32_t V, uint32_t k, double *entropy, uint32_t *ids,
                     double *probs);

/* gen.zig:366-432 AdaptiveDraft */
typedef struct or_adaptive {
    uint64_t cur_k, max_k, min_k, consecutive_rejections, cooldown_steps;
    float    last_margin;
} or_adaptive;
void     or_adaptive_init(or_adaptive *a, uint64_t max_k);
void     or_adaptive_record_margin(or_adaptive *a, float m);
uint64_t or_adaptive_next(or_adaptive *a);
void     or_adaptive_update(or_adaptive *a, uint64_t accepted, uint64_t drafted, int has_margin,
                            float margin);

/* Zig std.Random.DefaultPrng restated from the published algorithms
 * (xoshiro256++ seeded by splitmix64) and Random.float(f32). */
uint64_t or_splitmix64_next(uint64_t *state);
void     or_xoshiro_seed(uint64_t s[4], uint64_t seed);
uint64_t or_xoshiro_next(uint64_t s[4]);
float    or_rand_f32(uint64_t s[4]);

/* CPU baseline: sample `rows` rows (row stride ld), histories [rows][hist_ld]
 * with hist_len[row] valid entries (window = last penalty_last_n), optional
 * masks [rows][mask_ld], uniforms [rows][2].  Rows are copied into a scratch
 * row before the in-place pipeline so the inputs stay unchanged; the copy is
 * excluded from the returned seconds.  Returns elapsed seconds over `reps`
 * passes. */
double or_bench_sample_rows(const or_params *p, const float *logits, uint32_t rows, uint32_t V,
                            uint64_t ld, const uint32_t *hist, const int32_t *hist_len,
                            uint32_t hist_ld, const uint32_t *mask, uint32_t mask_ld,
                            const float *uniforms, uint32_t reps, uint32_t *out_tok,
                            float *out_margin);

/* JsonValidator, src/grammar.zig:59-480 (grammar_oracle.c).  Fields follow
 * the reference: state / escape / num are the enum positions of State,
 * EscapeState and NumState (:13-57); stack[d] is 0 for .object, 1 for .array. */
typedef struct or_json {
    int32_t state;
    int32_t escape;
    int32_t num;
    uint32_t depth;
    uint8_t stack[64];
    uint8_t lit_expected[8];
    uint8_t lit_len;
    uint8_t lit_idx;
    uint8_t object_only;
    uint8_t pad_;
} or_json;

/* model.zig:2492-2510 final-logit softcap, vectorized-body formula, and the
 * scalar tail (:2511-2513) for ids >= 32*floor(V/32). */
float  or_softcap(float l, float cap);
float  or_softcap_tail(float l, float cap);

void   or_json_init(or_json *j, int object_only);
int    or_json_is_finished(const or_json *j);
int    or_json_step_byte(or_json *j, uint8_t b);
int    or_json_try_consume(const or_json *j, const uint8_t *piece, size_t n, or_json *out);
int    or_json_consume(or_json *j, const uint8_t *piece, size_t n);
void   or_json_mask(const or_json *j, const uint32_t *piece_off, const uint8_t *piece_buf, uint32_t V,
                    const uint32_t *eog, uint32_t n_eog, int64_t eos, uint32_t *out);
double or_bench_json_mask(const or_json *states, uint32_t rows, const uint32_t *piece_off,
                          const uint8_t *piece_buf, uint32_t V, const uint32_t *eog, uint32_t n_eog,
                          int64_t eos, uint32_t *out, uint32_t reps);

#ifdef __cplusplus
}
#endif
#endif
