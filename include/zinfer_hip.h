/*
 * zinfer_hip.h -- C ABI of libzinfer_hip, the MI355X (gfx950) sampling and
 * constrained-decoding path for zinfer.
 *
 * The reference (pylypenko99/zinfer, Zig 0.17.1) has no plugin or FFI layer;
 * its boundary is the Zig API of src/sampler.zig, src/grammar.zig and
 * src/gen.zig.  Each declaration below names the reference symbol it replaces
 * (file:line).  A Zig shim binds these with `extern fn ... callconv(.c)`.
 *
 * Conventions
 *  - Every entry point that can fail returns int32_t: ZI_OK (0) or a negative
 *    zi_status.  zi_last_error() gives a static description of the last error
 *    on the calling thread.
 *  - "device" pointers are HIP device allocations on the context's device;
 *    "host" pointers are ordinary process memory.
 *  - Batched entry points (zi_*_rows) are stream-ordered on the context's
 *    stream and return once the work is enqueued; zi_sync() waits.  Calls on
 *    one context share its scratch memory and must not overlap (one context
 *    per thread, as the reference keeps one Sampler per thread).
 *  - Logit rows are row-major [rows][ld]; the logits pointer must be 16-byte
 *    aligned and ld a multiple of 8 elements.  NaN logits are outside the
 *    contract (the reference's insertion sort gives order-dependent results
 *    for them); the kernels never select a NaN.
 */
#ifndef ZINFER_HIP_H
#define ZINFER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ZI_ABI_VERSION 1

typedef enum zi_status {
    ZI_OK = 0,
    ZI_ERR_INVALID = -1,     /* bad argument (null, size, alignment) */
    ZI_ERR_HIP = -2,         /* HIP runtime error */
    ZI_ERR_OOM = -3,         /* device or host allocation failed */
    ZI_ERR_UNSUPPORTED = -4, /* valid request outside what this build implements */
    ZI_ERR_CAPACITY = -5     /* exceeds the context's max_rows / max_vocab */
} zi_status;

typedef enum zi_dtype { ZI_F32 = 0, ZI_BF16 = 1 } zi_dtype;

/* Params, src/sampler.zig:3-27.  Field meaning and defaults follow the
 * reference; usize fields are uint32_t here.  Extensions (not in the
 * reference): freq_penalty, presence_penalty (l -= count*freq + presence for
 * ids in the window, after the repetition penalty) and penalty_last_n (the
 * reference fixes the window at repeat_last_n = 64, src/sampler.zig:30). */
typedef struct zi_params {
    float    temp;               /* 0.8  (<= 0: greedy argmax, sampler.zig:193) */
    uint32_t top_k;              /* 40   (0: whole vocabulary) */
    float    top_p;              /* 0.95 */
    float    min_p;              /* 0.05 */
    float    repeat_penalty;     /* 1.0  (1 = off) */
    float    freq_penalty;       /* 0    extension */
    float    presence_penalty;   /* 0    extension */
    uint32_t penalty_last_n;     /* 64   extension (reference constant) */
    float    dry_multiplier;     /* 0    (0 = off) */
    float    dry_base;           /* 1.75 */
    uint32_t dry_allowed_length; /* 2 */
    uint32_t dry_range;          /* 1024 */
    float    xtc_probability;    /* 0    (0 = off) */
    float    xtc_threshold;      /* 0.1 */
    uint32_t xtc_min_keep;       /* 1 */
    uint64_t seed;               /* 0    (host Sampler RNG seed) */
    float    final_logit_softcap; /* 0   (0 = off) cap*tanh(l/cap) on each logit before the mask, the
                                     model's epilogue (src/model.zig:2492-2514) fused into the read;
                                     set it when the producer leaves logits uncapped.  Ids below
                                     32*floor(V/32) take the reference's vector body (tanh through
                                     exp, clamped at |l/cap| = 9), the rest its scalar tail
                                     (cap * tanh(l / cap)). */
} zi_params;

/* Fills the reference defaults (src/sampler.zig:4-26). */
void zi_params_default(zi_params *p);

/* ---------------------------------------------------------------- context */

typedef struct zi_ctx zi_ctx;
typedef struct zi_vocab zi_vocab; /* token pieces on the device (JSON grammar masks, below) */

/* Creates a context on HIP device `device` able to serve batches of up to
 * max_rows rows of up to max_vocab logits.  It owns a HIP stream (default
 * priority) and the device scratch the kernels use.  No reference
 * counterpart: the reference samples on the host (Sampler.init allocates
 * cand[vocab], src/sampler.zig:49-58). */
int32_t zi_create(zi_ctx **out, int32_t device, int32_t max_rows, int32_t max_vocab);
void    zi_destroy(zi_ctx *ctx);
/* Make batched calls use `stream` (a hipStream_t) instead of the context's
 * own stream (the default until this is called); NULL selects HIP's default
 * (null) stream. */
int32_t zi_set_stream(zi_ctx *ctx, void *stream);
int32_t zi_sync(zi_ctx *ctx);

/* Allocates now the scratch that some requests otherwise allocate on their
 * first call, so that no later call on the context allocates (code under HIP
 * graph capture, serving loops).  No reference counterpart.  Synchronous.
 *   ZI_RESERVE_WHOLE_ORDER   top_k = 0 or > 256 (whole-order sorting):
 *                            20 B x max_rows x max_vocab (rounded up to 8)
 *                            + 4 B x max_rows
 *   ZI_RESERVE_PRUNED_DENSE  zi_sample_rows_pruned with a softcap or top_k >
 *                            256 (the reference's filled rows):
 *                            4 B x max_rows x max_vocab (rounded up to 8) */
#define ZI_RESERVE_WHOLE_ORDER 1u
#define ZI_RESERVE_PRUNED_DENSE 2u
int32_t zi_reserve(zi_ctx *ctx, uint32_t what);
const char *zi_last_error(void);
int32_t zi_abi_version(void);

/* ------------------------------------------------- batched device entries */

/* Per-row inputs of a batch.  All pointers are device pointers. */
typedef struct zi_batch {
    const void     *logits;     /* [rows][ld], f32 or bf16 */
    int32_t         dtype;      /* zi_dtype */
    int32_t         rows;
    int32_t         vocab;      /* V */
    int32_t         ld;         /* row stride in elements, >= V, multiple of 8 */
    const uint32_t *hist;       /* [rows][hist_ld] accepted token ids, oldest first; NULL = none */
    const int32_t  *hist_len;   /* [rows] valid entries of hist */
    int32_t         hist_ld;
    const uint32_t *mask;       /* [rows][mask_ld] allowed bits: id t allowed <=>
                                   (mask[t >> 5] >> (t & 31)) & 1; NULL = all allowed */
    int32_t         mask_ld;    /* >= ceil(V / 32) */
    const uint32_t *edit_ids;   /* [rows][edit_ld] distinct ids whose penalized logit gets
                                   l -= edit_delta (the DRY step); NULL = none */
    const float    *edit_delta; /* [rows][edit_ld] */
    const int32_t  *edit_count; /* [rows] */
    int32_t         edit_ld;
} zi_batch;

/* Outputs of zi_sample_rows.  tok and margin are required; the rest may be
 * NULL.  All device pointers. */
typedef struct zi_sample_out {
    uint32_t *tok;       /* [rows] sampled token (SampleResult.tok) */
    float    *margin;    /* [rows] c[0].v - c[1].v, 10 if n < 2 (SampleResult.margin) */
    int32_t  *ndraws;    /* [rows] uniforms consumed: 0 greedy, 1, 2 (XTC chance drawn) */
    int32_t  *keep;      /* [rows] survivors after top-p and min-p */
    uint32_t *cand_ids;  /* [rows][cand_ld] candidates in (value desc, id asc) order */
    float    *cand_vals; /* [rows][cand_ld] their penalized logits */
    float    *probs;     /* [rows][cand_ld] w_i / total for kept i (after XTC), else 0 */
    int32_t   cand_ld;   /* >= top_k when the three arrays above are given */
} zi_sample_out;

/* One Sampler.sampleWithMargin (src/sampler.zig:190-276) per row, batched:
 * mask (grammar.zig:446-479) -> repetition/frequency/presence penalty over the
 * last penalty_last_n ids of hist (sampler.zig:91-100) -> edits (the DRY
 * subtraction, sampler.zig:184) -> top-k -> top-p -> min-p -> temperature ->
 * XTC -> draw.  temp <= 0 returns the reference argmax (2x8-lane tie and
 * margin rules, sampler.zig:532-610) of the penalized row.
 * `uniforms` [rows][2] (device) stand in for the Zig rng: the first draw is
 * the XTC chance when XTC draws one, else the main draw; ndraws says how many
 * were used so the caller can advance its own generator.
 * Any top_k: lists of up to 256 candidates take one fused pass; top_k = 0
 * (or >= V) first tries the top-256 prefix with a bounded total and sorts
 * the rows it cannot settle; 256 < top_k < V always sorts.  For top_k > 256
 * (with V > 256) cand_ids/cand_vals/probs hold the first min(keep, cand_ld)
 * candidates (cand_ld >= 1), and the first such call allocates 20 bytes of
 * sort scratch per (max_rows x max_vocab) entry unless zi_reserve did.
 * Penalty window + edits <= 1024 + 128 ids. */
int32_t zi_sample_rows(zi_ctx *ctx, const zi_params *p, const zi_batch *b,
                       const float *uniforms, const zi_sample_out *out);

/* zi_sample_rows without a context and without allocating: for callers that
 * cannot call hipMalloc (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  No counterpart in the reference (its
 * sampler runs on the host).  Same inputs, outputs and results as
 * zi_sample_rows; runs on the calling thread's current HIP device, enqueued
 * on `stream` (a hipStream_t; NULL = the default stream).  Its scratch is one
 * static device array per GPU (about 7 MB, held until the process ends; its
 * address is looked up once per device on the first call).  Each call clears
 * the row tickets with a small kernel on `stream` and keeps nothing else
 * between calls, but every call on a GPU shares that GPU's array, so calls
 * that overlap on one GPU (other streams, other threads) race: serialize
 * them.  Limits, checked before any HIP call: rows <= 512, vocab <= 262144,
 * top_k resolving to <= 256 when temp > 0 (ZI_ERR_UNSUPPORTED otherwise: the
 * whole-order sort needs a context's scratch), hist_ld <= 1024. */
int32_t zi_sample_rows_noalloc(const zi_params *p, const zi_batch *b, const float *uniforms,
                               const zi_sample_out *out, void *stream);

/* zi_sample_rows on pruned-vocabulary rows.  Replaces the reference's -inf
 * fill of the whole logit row (src/model.zig:2127-2128) plus the full read of
 * it: the pruned lm_head (:2036-2140) computes only its candidate groups of 8
 * ids (prunedFineWorker, :1144-1160, writing logits[8g .. 8g + 8)), and this
 * entry reads only those, every other id being -inf.  groups [rows][groups_ld]
 * lists row r's group ids g (ids [8g, 8g + 8) valid in `b`'s row, the rest of
 * the row is never read); group_count [rows] (device) how many, clamped to
 * groups_ld.  Ids g >= ceil(V / 8) are ignored; a group listed twice counts
 * once.  Results are those of zi_sample_rows on the row with the fill
 * written.  With final_logit_softcap (which runs after the fill and moves it
 * to -cap*tanh(9)) or top_k resolving to > 256 (lists that order every id),
 * the filled rows are written to a context scratch (zi_reserve, else
 * allocated on first use) and sampled by zi_sample_rows.  Limits: groups_ld <= 1024 (the reference
 * keeps 576), V >= 16; each returns ZI_ERR_UNSUPPORTED. */
int32_t zi_sample_rows_pruned(zi_ctx *ctx, const zi_params *p, const zi_batch *b,
                              const uint32_t *groups, const int32_t *group_count,
                              int32_t groups_ld, const float *uniforms,
                              const zi_sample_out *out);

/* argmaxWithMargin per row (src/sampler.zig:532-614; greedy decoding, the
 * bench argmax at src/main.zig:690).  out_tok/out_margin follow the reference
 * 2x8-lane rules; out_tok_low/out_margin_true (may be NULL) give the
 * lowest-index argmax and the true top-1 minus top-2 gap.  Only logits,
 * dtype, rows, vocab and ld of `b` are read.  Device outputs [rows]. */
int32_t zi_argmax_rows(zi_ctx *ctx, const zi_batch *b, uint32_t *out_tok, float *out_margin,
                       uint32_t *out_tok_low, float *out_margin_true);

/* Speculative-verify row statistics (the consumer is Gen.AdaptiveDraft and
 * the accept compare, src/gen.zig:366-432, :544-587): Shannon entropy (nats)
 * of the T = 1 full-vocabulary softmax, the top-k ids (k <= 64, value desc,
 * id asc) with full-vocabulary probabilities, the lowest-index argmax and,
 * when draft (device [rows]) is non-NULL, accept[r] = (argmax == draft[r]).
 * The reference has no entropy (it uses the logit margin); this is the new
 * signal.  Only logits, dtype, rows, vocab, ld of `b` are read. */
int32_t zi_entropy_topk_rows(zi_ctx *ctx, const zi_batch *b, int32_t k, const uint32_t *draft,
                             float *out_entropy, uint32_t *out_ids, float *out_probs,
                             int32_t out_ld, uint32_t *out_argmax, uint8_t *out_accept);

/* JsonValidator.applyMask (src/grammar.zig:446-479) for a precomputed packed
 * mask: logits[r][t] = -inf where the bit is clear, in place (f32 or bf16).
 * Only logits, dtype, rows, vocab, ld, mask, mask_ld of `b` are read. */
int32_t zi_apply_mask_rows(zi_ctx *ctx, const zi_batch *b);

/* ------------------------------------------------ JSON grammar mask (GPU) */

/* JsonValidator (src/grammar.zig:59-68) as plain data.  state / escape / num
 * are the positions in State, EscapeState and NumState (:13-57); bit d of
 * stack is 1 when stack[d] is .array, 0 for .object (d < depth <= 64). */
typedef struct zi_json_state {
    uint64_t stack;
    uint8_t  state;
    uint8_t  escape;
    uint8_t  num;
    uint8_t  depth;
    uint8_t  lit_len;
    uint8_t  lit_idx;
    uint8_t  object_only;     /* is_object_only */
    uint8_t  reserved;
    uint8_t  lit_expected[8];
} zi_json_state;

/* Host state machine, same semantics as the reference. */
void    zi_json_init(zi_json_state *s, int32_t object_only);           /* initObjectOnly / initAny :70-76 */
int32_t zi_json_is_finished(const zi_json_state *s);                   /* isFinished :78-80 */
int32_t zi_json_step_byte(zi_json_state *s, uint8_t b);                /* stepByte :195-381 */
/* consume (:437-443): in place; on failure the bytes before the bad one stay
 * applied.  Returns 1 / 0. */
int32_t zi_json_consume(zi_json_state *s, const uint8_t *piece, size_t n);
/* tryConsume (:428-434): 1 and *out = the new state, or 0 (out untouched). */
int32_t zi_json_try_consume(const zi_json_state *s, const uint8_t *piece, size_t n, zi_json_state *out);

/* The token pieces on the device: Tokenizer.piece_off [V+1] / piece_buf
 * (decoded bytes of every token, src/tokenizer.zig:35-36, piece() :274-276),
 * the end-of-generation ids (Tokenizer.eog, isEog :270-272) and the eos id
 * every reference call site passes to applyMask (g.tok.eos, src/gen.zig:458;
 * -1 for none).  Host arrays, copied (synchronous).  cache_states > 0 keeps
 * that many per-state masks on the device (least recently used replaced). */
int32_t zi_vocab_create(zi_vocab **out, zi_ctx *ctx, const uint32_t *piece_off, const uint8_t *piece_buf,
                        uint32_t n_vocab, const uint32_t *eog, uint32_t n_eog, int64_t eos,
                        int32_t cache_states);
void    zi_vocab_destroy(zi_vocab *v);

/* JsonValidator.applyMask (src/grammar.zig:446-479) as a packed mask, one
 * row per validator state: bit t of out_mask[r][t >> 5] is set when the
 * reference leaves logit t unchanged (the layout zi_batch.mask reads); bits
 * at and above V are clear.  states: host [rows]; out_mask: device
 * [rows][mask_ld], mask_ld >= ceil(V / 32).  Stream-ordered. */
int32_t zi_json_mask_rows(zi_ctx *ctx, zi_vocab *v, const zi_json_state *states, int32_t rows,
                          uint32_t *out_mask, int32_t mask_ld);

/* applyMask on one host row, in place (the reference signature): logits of
 * disallowed tokens become -inf.  Synchronous. */
int32_t zi_json_apply_mask(zi_ctx *ctx, zi_vocab *v, const zi_json_state *s, float *logits, uint32_t n);

/* ------------------------------------------ host mirror of the Zig Sampler */

/* The Sampler of src/sampler.zig:38-286 with the same state (params, RNG,
 * 64-entry recent ring, 4096-entry history, breakers) and methods; each
 * sample call runs zi_sample_rows on one host row.  The RNG restates Zig's
 * DefaultPrng (xoshiro256++ seeded by splitmix64) and Random.float(f32). */
typedef struct zi_sampler zi_sampler;

int32_t zi_sampler_init(zi_sampler **out, zi_ctx *ctx, uint32_t vocab, const zi_params *p); /* :49 */
void    zi_sampler_deinit(zi_sampler *s);                                                  /* :60 */
void    zi_sampler_reset(zi_sampler *s);                                                   /* :64 */
void    zi_sampler_add_breaker(zi_sampler *s, uint32_t tok);                               /* :69 */
int32_t zi_sampler_is_breaker(const zi_sampler *s, uint32_t tok);                          /* :76 */
void    zi_sampler_accept(zi_sampler *s, uint32_t tok);                                    /* :84 */
/* Host DRY step on host logits, in place (src/sampler.zig:104-187). */
void    zi_sampler_apply_dry(const zi_sampler *s, float *logits, uint32_t n);
/* sampleWithMargin (src/sampler.zig:190): host logits, modified in place by
 * the penalty and DRY exactly as the reference modifies them. */
int32_t zi_sampler_sample_with_margin(zi_sampler *s, float *logits, uint32_t n, uint32_t *tok,
                                      float *margin);
int32_t zi_sampler_sample(zi_sampler *s, float *logits, uint32_t n, uint32_t *tok); /* :279 */
/* Draft verification (src/gen.zig:544-587) in one batched launch.  Row i of
 * b (device logits, i = 0..k) is the target's output after cur_tok and
 * draft[0..i); it is sampled with the state the reference would have after
 * take(draft[0..i)): penalty window and DRY history with the prefix appended,
 * JSON validator (when v and json are given) after consuming its pieces, and
 * the RNG draws of rows 0..i-1 spent.  Acceptance stops at the first row whose
 * token differs from the draft, is in eog, or once max_accept tokens are taken;
 * with all k accepted, row k (the bonus row) gives the next token.  Returns the
 * accepted count, the next token and its margin, and leaves the sampler (and
 * *json) as the reference leaves them: draft[0..accepted) accepted (pieces
 * consumed), the RNG advanced by the draws of the rows it sampled.  The next
 * token is not accepted.  k <= 16; only logits, dtype, rows (>= k + 1), vocab
 * and ld of b are read.  Synchronous. */
int32_t zi_sampler_verify(zi_sampler *s, const zi_batch *b, const uint32_t *draft, uint32_t k,
                          uint32_t max_accept, const uint32_t *eog, uint32_t n_eog, zi_vocab *v,
                          zi_json_state *json, uint32_t *out_accepted, uint32_t *out_next,
                          float *out_margin);

/* Tree verification (the batched tree verify of the reference's roadmap,
 * ROADMAP.md:134-135, over CandidateTree branches, src/sampler.zig:291-475):
 * n_branches (<= 8) drafts, branch j = drafts[j * draft_ld .. + ks[j]]
 * (ks[j] <= 16), verified in one zi_sample_rows launch.  b holds branch j's
 * rows at base_j .. base_j + ks[j], base_j = sum over i < j of (ks[i] + 1),
 * each row as zi_sampler_verify reads it.  Branch j's results are exactly what
 * zi_sampler_verify would return for that draft alone from the sampler's
 * current state (every branch starts at the same RNG draw).  out_accepted /
 * out_next / out_margin [n_branches]; *out_best = the branch with the most
 * accepted tokens (the first on ties).  With commit != 0 the sampler and
 * *json are left as zi_sampler_verify on that branch leaves them; with 0 they
 * are untouched.  Synchronous. */
int32_t zi_sampler_verify_tree(zi_sampler *s, const zi_batch *b, const uint32_t *drafts,
                               uint32_t draft_ld, const uint32_t *ks, uint32_t n_branches,
                               uint32_t max_accept, const uint32_t *eog, uint32_t n_eog,
                               zi_vocab *v, zi_json_state *json, int32_t commit,
                               uint32_t *out_accepted, uint32_t *out_next, float *out_margin,
                               uint32_t *out_best);
/* Read / replace the params (server.zig:377-415 writes g.smp.p fields). */
void    zi_sampler_get_params(const zi_sampler *s, zi_params *p);
void    zi_sampler_set_params(zi_sampler *s, const zi_params *p);
/* rng = DefaultPrng.init(seed) (sampler.zig:52, server.zig:414). */
void    zi_sampler_seed(zi_sampler *s, uint64_t seed);
/* Next Random.float(f32) of the sampler's generator (advances it). */
float   zi_sampler_rand_f32(zi_sampler *s);

/* argmaxWithMargin on a host row (src/sampler.zig:532-614); synchronous. */
int32_t zi_argmax_with_margin(zi_ctx *ctx, const float *logits, uint32_t n, uint32_t *tok,
                              float *margin);

/* Sampler.applyDry (src/sampler.zig:104-187) for a batch on the device: the
 * DRY edits of each row's history, written in the zi_batch.edit_* format so
 * that zi_sample_rows applies them (logits[id] -= delta).  hist [rows][hist_ld]
 * holds each row's accepted ids oldest first, hist_len [rows] how many (the
 * last min(hist_len, dry_range, 4096) are searched, the reference's ring);
 * breakers (device, <= 16, sampler.zig:32) the sequence breakers.  Writes
 * out_count[r] (<= 128) and, when DRY is on, out_ids / out_delta
 * [rows][edit_ld], edit_ld >= 128, in the reference's order (first
 * appearance).  The same results as zi_dry_edits per row.  Asynchronous on
 * the context's stream. */
int32_t zi_dry_edits_rows(zi_ctx *ctx, const zi_params *p, const uint32_t *hist,
                          const int32_t *hist_len, int32_t hist_ld, int32_t rows,
                          const uint32_t *breakers, uint32_t n_breakers, uint32_t *out_ids,
                          float *out_delta, int32_t *out_count, int32_t edit_ld);

/* DRY edits (src/sampler.zig:104-187) from a linear history (oldest first),
 * as (id, delta) pairs for zi_batch.edit_*; returns the count (<= 128). */
uint32_t zi_dry_edits(const uint32_t *hist, uint32_t n_hist, const uint32_t *breakers,
                      uint32_t n_breakers, const zi_params *p, uint32_t *out_ids,
                      float *out_deltas);

/* Gen.AdaptiveDraft (src/gen.zig:366-432), host-side. */
typedef struct zi_adaptive_draft {
    uint64_t cur_k, max_k, min_k, consecutive_rejections, cooldown_steps;
    float    last_margin;
} zi_adaptive_draft;
void     zi_adaptive_draft_init(zi_adaptive_draft *a, uint64_t max_k);           /* :374 */
void     zi_adaptive_draft_record_margin(zi_adaptive_draft *a, float margin);    /* :382 */
uint64_t zi_adaptive_draft_next(zi_adaptive_draft *a);                           /* :388 */
void     zi_adaptive_draft_update(zi_adaptive_draft *a, uint64_t accepted, uint64_t drafted,
                                  int32_t has_margin, float margin);             /* :408 */
/* The entropy signal for the same controller (no counterpart in the reference,
 * whose controller reads the logit margin only; the entropy comes from
 * zi_entropy_topk_rows).  zi_entropy_margin(H) is the margin m >= 0 at which
 * the two-token softmax [m, 0] has entropy H nats: 0 for H >= ln 2 or NaN,
 * capped at 100 for H near 0.  record_entropy records that margin, so
 * nextDraft's thresholds (3.0, 1.8, 0.9) act at H = 0.191, 0.408, 0.601. */
float    zi_entropy_margin(float entropy);
void     zi_adaptive_draft_record_entropy(zi_adaptive_draft *a, float entropy);

#ifdef __cplusplus
}
#endif
#endif
