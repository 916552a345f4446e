// zi_api.cpp -- C ABI of libzinfer_hip: context, argument checks, chunk
// planning and kernel dispatch for the batched device entry points.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "../../include/zinfer_hip.h"
#include "zi_internal.hpp"
#include "zi_launch.hpp"

namespace {
thread_local char g_err[512] = "no error";
}

int32_t zi_fail(int32_t code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int32_t zi_hip_fail(hipError_t e, const char *what) {
    return zi_fail(ZI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

extern "C" const char *zi_last_error(void) { return g_err; }
extern "C" int32_t zi_abi_version(void) { return ZI_ABI_VERSION; }

extern "C" void zi_params_default(zi_params *p) {
    if (!p) return;
    std::memset(p, 0, sizeof *p);
    p->temp = 0.8f;  // src/sampler.zig:4-26
    p->top_k = 40;
    p->top_p = 0.95f;
    p->min_p = 0.05f;
    p->repeat_penalty = 1.0f;
    p->freq_penalty = 0.0f;
    p->presence_penalty = 0.0f;
    p->penalty_last_n = 64;  // repeat_last_n, src/sampler.zig:30
    p->dry_multiplier = 0.0f;
    p->dry_base = 1.75f;
    p->dry_allowed_length = 2;
    p->dry_range = 1024;
    p->xtc_probability = 0.0f;
    p->xtc_threshold = 0.1f;
    p->xtc_min_keep = 1;
    p->seed = 0;
    p->final_logit_softcap = 0.0f;
}

#define HIP_TRY(call, what)                          \
    do {                                             \
        hipError_t e_ = (call);                      \
        if (e_ != hipSuccess) return zi_hip_fail(e_, what); \
    } while (0)

extern "C" int32_t zi_create(zi_ctx **out, int32_t device, int32_t max_rows, int32_t max_vocab) {
    if (!out) return zi_fail(ZI_ERR_INVALID, "zi_create: out is NULL");
    *out = nullptr;
    if (max_rows < 1 || max_vocab < 1)
        return zi_fail(ZI_ERR_INVALID, "zi_create: max_rows=%d max_vocab=%d", max_rows, max_vocab);
    if (max_vocab > zi::kMaxVocab)
        return zi_fail(ZI_ERR_UNSUPPORTED, "zi_create: max_vocab %d > %d", max_vocab, zi::kMaxVocab);
    int ndev = 0;
    HIP_TRY(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
    if (device < 0 || device >= ndev)
        return zi_fail(ZI_ERR_INVALID, "zi_create: device %d of %d", device, ndev);
    HIP_TRY(hipSetDevice(device), "hipSetDevice");

    zi_ctx *c = new (std::nothrow) zi_ctx();
    if (!c) return zi_fail(ZI_ERR_OOM, "zi_create: host allocation");
    c->device = device;
    c->max_rows = max_rows;
    c->max_vocab = max_vocab;
    hipError_t e = hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        return zi_hip_fail(e, "hipStreamCreate");
    }
    c->stream = c->own_stream;

    const size_t R = (size_t)max_rows, G = zi::kMaxGHost, CAP = zi::kCapAHost;
    struct Buf {
        void **p;
        size_t bytes;
    } bufs[] = {
        {(void **)&c->g_key, R * G * CAP * sizeof(uint64_t)},
        {(void **)&c->g_val, R * G * CAP * sizeof(float)},
        {(void **)&c->g_cnt, R * G * sizeof(int32_t)},
        {(void **)&c->tickets, R * sizeof(int32_t)},
        {(void **)&c->g_stat, R * G * 3 * sizeof(double)},
        {(void **)&c->g_cls, R * G * 16 * sizeof(uint64_t)},
        {(void **)&c->g_raw, R * G * 16 * sizeof(uint32_t)},
        {(void **)&c->g_top2, R * G * 2 * sizeof(float)},
        {(void **)&c->g_tail, R * 16 * sizeof(float)},
        {(void **)&c->win_ids, R * zi::kMaxWinHost * sizeof(uint32_t)},
        {(void **)&c->win_len, R * sizeof(int32_t)},
    };
    for (auto &b : bufs) {
        e = hipMalloc(b.p, b.bytes);
        if (e != hipSuccess) {
            zi_destroy(c);
            return zi_fail(ZI_ERR_OOM, "zi_create: hipMalloc %zu bytes: %s", b.bytes, hipGetErrorString(e));
        }
    }
    e = hipMemset(c->tickets, 0, R * sizeof(int32_t));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        zi_destroy(c);
        return zi_hip_fail(e, "zi_create: clear tickets");
    }
    *out = c;
    return ZI_OK;
}

// zi_destroy cannot report; the first failing HIP call is left in
// zi_last_error() and the rest of the teardown still runs.
extern "C" void zi_destroy(zi_ctx *c) {
    if (!c) return;
    hipError_t first = hipSuccess;
    const char *what = nullptr;
    auto note = [&](hipError_t e, const char *w) {
        if (e != hipSuccess && first == hipSuccess) {
            first = e;
            what = w;
        }
    };
    note(hipSetDevice(c->device), "zi_destroy: hipSetDevice");
    if (c->own_stream) note(hipStreamSynchronize(c->own_stream), "zi_destroy: hipStreamSynchronize");
    void *ptrs[] = {c->g_key,  c->g_val,   c->g_cnt,   c->tickets, c->g_stat,  c->g_cls,   c->g_raw,
                    c->g_top2, c->g_tail,  c->win_ids, c->win_len, c->ex_sort, c->nuc_flag, c->pr_dense};
    for (void *p : ptrs)
        if (p) note(hipFree(p), "zi_destroy: hipFree");
    if (c->own_stream) note(hipStreamDestroy(c->own_stream), "zi_destroy: hipStreamDestroy");
    if (first != hipSuccess) zi_hip_fail(first, what);
    delete c;
}

extern "C" int32_t zi_set_stream(zi_ctx *c, void *stream) {
    if (!c) return zi_fail(ZI_ERR_INVALID, "zi_set_stream: ctx is NULL");
    c->stream = (hipStream_t)stream;  // NULL is HIP's default (null) stream
    return ZI_OK;
}

extern "C" int32_t zi_sync(zi_ctx *c) {
    if (!c) return zi_fail(ZI_ERR_INVALID, "zi_sync: ctx is NULL");
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return ZI_OK;
}

namespace zi {

// Chunking: 512 threads x EPT elements per workgroup, EPT in {16, 32, 64};
// the largest EPT that still gives >= 256 workgroups (one per CU; or EPT 16),
// with at most kMaxG chunks per row.
Plan plan_rows(int rows, int V, int dtype) {
    Plan pl;
    const int vec = dtype == ZI_F32 ? 4 : 8;
    int ept = 64;
    auto chunks = [&](int e) { return (V + kThreadsHost * e - 1) / (kThreadsHost * e); };
    while (ept > 16 && (int64_t)rows * chunks(ept) < 256 && chunks(ept / 2) <= kMaxGHost) ept /= 2;
    int G = chunks(ept);
    int CH = (V + G - 1) / G;
    CH = (CH + 63) / 64 * 64;
    G = (V + CH - 1) / CH;
    pl.G = G;
    pl.CH = CH;
    pl.nv = ept / vec;
    return pl;
}

}  // namespace zi

static int32_t check_batch(const zi_ctx *c, const zi_batch *b, const char *fn) {
    if (!c || !b) return zi_fail(ZI_ERR_INVALID, "%s: NULL ctx or batch", fn);
    if (!b->logits) return zi_fail(ZI_ERR_INVALID, "%s: logits is NULL", fn);
    if (b->dtype != ZI_F32 && b->dtype != ZI_BF16) return zi_fail(ZI_ERR_INVALID, "%s: dtype %d", fn, b->dtype);
    if (b->rows < 1 || b->vocab < 1) return zi_fail(ZI_ERR_INVALID, "%s: rows=%d vocab=%d", fn, b->rows, b->vocab);
    if (b->rows > c->max_rows || b->vocab > c->max_vocab)
        return zi_fail(ZI_ERR_CAPACITY, "%s: rows=%d vocab=%d exceed context (%d, %d)", fn, b->rows, b->vocab,
                       c->max_rows, c->max_vocab);
    if (b->ld < b->vocab || (b->ld % 8) != 0)
        return zi_fail(ZI_ERR_INVALID, "%s: ld=%d must be >= vocab and a multiple of 8", fn, b->ld);
    if (((uintptr_t)b->logits & 15u) != 0) return zi_fail(ZI_ERR_INVALID, "%s: logits not 16-byte aligned", fn);
    return ZI_OK;
}

static int32_t fill_source(const zi_batch *b, const zi_params *p, bool with_inputs, zi::RowSource &s,
                           const zi::Plan &pl, const char *fn) {
    std::memset(&s, 0, sizeof s);
    s.logits = b->logits;
    s.ld = b->ld;
    s.V = b->vocab;
    s.G = pl.G;
    s.CH = pl.CH;
    s.rp = 1.0f;
    if (!with_inputs) return ZI_OK;
    if (b->mask) {
        if (b->mask_ld < (b->vocab + 31) / 32)
            return zi_fail(ZI_ERR_INVALID, "%s: mask_ld=%d < ceil(V/32)", fn, b->mask_ld);
        s.mask = b->mask;
        s.mask_ld = b->mask_ld;
    }
    if (p && p->final_logit_softcap > 0.0f) {
        s.cap = p->final_logit_softcap;
        s.inv_cap = 1.0f / p->final_logit_softcap;
        s.cap_body = b->vocab / 32 * 32;  // the reference's vector body; the rest is its scalar tail
    }
    if (p) {
        s.rp = p->repeat_penalty;
        s.freq = p->freq_penalty;
        s.pres = p->presence_penalty;
        s.do_rep = p->repeat_penalty != 1.0f;
        s.do_fp = (p->freq_penalty != 0.0f || p->presence_penalty != 0.0f);
        if (b->hist && (s.do_rep || s.do_fp) && p->penalty_last_n > 0) {
            if (!b->hist_len || b->hist_ld < 0)
                return zi_fail(ZI_ERR_INVALID, "%s: hist without hist_len/hist_ld", fn);
            if (p->penalty_last_n > (uint32_t)zi::kMaxWinHost)
                return zi_fail(ZI_ERR_UNSUPPORTED, "%s: penalty_last_n %u > %d", fn, p->penalty_last_n,
                               zi::kMaxWinHost);
            s.hist = b->hist;
            s.hist_len = b->hist_len;
            s.hist_ld = b->hist_ld;
            s.win = (int)p->penalty_last_n;
        }
    }
    if (b->edit_ids) {
        if (!b->edit_delta || !b->edit_count || b->edit_ld < 0)
            return zi_fail(ZI_ERR_INVALID, "%s: edit_ids without edit_delta/edit_count", fn);
        s.edit_ids = b->edit_ids;
        s.edit_delta = b->edit_delta;
        s.edit_count = b->edit_count;
        s.edit_ld = b->edit_ld;
    }
    return ZI_OK;
}

namespace {
// The device scratch one call works in: a context's buffers, or the static
// array of zi_sample_rows_noalloc.  Layouts: zi_launch.hpp.
struct Scratch {
    uint64_t *g_key;
    float *g_val;
    int32_t *g_cnt;
    int32_t *tickets;
    uint64_t *g_cls;
    uint32_t *g_raw;
    float *g_top2;
    float *g_tail;
    uint32_t *win_ids;  // NULL: no window compaction (histories up to kMaxWinHost wide only)
    int32_t *win_len;
};

Scratch ctx_scratch(const zi_ctx *c) {
    return Scratch{c->g_key, c->g_val, c->g_cnt, c->tickets, c->g_cls, c->g_raw, c->g_top2, c->g_tail,
                   c->win_ids, c->win_len};
}
}  // namespace

static int32_t run_argmax(const Scratch &S, hipStream_t st, const zi::RowSource &src, const zi_batch *b,
                          const zi::Plan &pl, uint32_t *tok, float *margin, uint32_t *tok_low, float *margin_true,
                          int32_t *ndraws) {
    zi::ArgmaxParams P;
    std::memset(&P, 0, sizeof P);
    P.src = src;
    P.tok = tok;
    P.margin = margin;
    P.tok_low = tok_low;
    P.margin_true = margin_true;
    P.ndraws = ndraws;
    P.g_cls = S.g_cls;
    P.g_raw = S.g_raw;
    P.g_top2 = S.g_top2;
    P.g_tail = S.g_tail;
    P.tickets = S.tickets;
    hipError_t e = zi::launch_argmax(P, b->dtype, pl.nv, b->rows, st);
    if (e != hipSuccess) return zi_hip_fail(e, "argmax kernel launch");
    return ZI_OK;
}

// The whole-order sort scratch: 5 planes of [max_rows][max_vocab rounded up
// to 8] u32 and the per-row settle flags.  Allocated by zi_reserve, or by the
// first request that needs it.
static int32_t ensure_whole_order(zi_ctx *c) {
    if (c->ex_sort) return ZI_OK;
    const int64_t ld = ((int64_t)c->max_vocab + 7) / 8 * 8;
    const size_t bytes = 5 * (size_t)c->max_rows * (size_t)ld * sizeof(uint32_t);
    hipError_t e = hipMalloc((void **)&c->ex_sort, bytes);
    if (e == hipSuccess) e = hipMalloc((void **)&c->nuc_flag, (size_t)c->max_rows * sizeof(int32_t));
    if (e != hipSuccess) {
        if (c->ex_sort) {
            const hipError_t ef = hipFree(c->ex_sort);
            if (ef != hipSuccess) e = ef;
        }
        c->ex_sort = nullptr;
        c->nuc_flag = nullptr;
        return zi_fail(ZI_ERR_OOM, "sort scratch %zu bytes: %s", bytes, hipGetErrorString(e));
    }
    c->ex_ld = ld;
    return ZI_OK;
}

// Dense rows for zi_sample_rows_pruned's dense path, at least `need` bytes
// (zi_reserve takes max_rows x max_vocab rounded up to 8 x 4 bytes, enough
// for every batch).
static int32_t ensure_pruned_dense(zi_ctx *c, size_t need) {
    if (need <= c->pr_dense_bytes) return ZI_OK;
    if (c->pr_dense) {
        const hipError_t ef = hipFree(c->pr_dense);
        c->pr_dense = nullptr;
        c->pr_dense_bytes = 0;
        if (ef != hipSuccess) return zi_hip_fail(ef, "pruned dense scratch release");
    }
    const hipError_t e = hipMalloc(&c->pr_dense, need);
    if (e != hipSuccess) {
        c->pr_dense = nullptr;
        return zi_fail(ZI_ERR_OOM, "pruned dense scratch %zu bytes: %s", need, hipGetErrorString(e));
    }
    c->pr_dense_bytes = need;
    return ZI_OK;
}

extern "C" int32_t zi_reserve(zi_ctx *c, uint32_t what) {
    if (!c) return zi_fail(ZI_ERR_INVALID, "zi_reserve: ctx is NULL");
    if (what & ~(uint32_t)(ZI_RESERVE_WHOLE_ORDER | ZI_RESERVE_PRUNED_DENSE))
        return zi_fail(ZI_ERR_INVALID, "zi_reserve: unknown flags 0x%x", what);
    HIP_TRY(hipSetDevice(c->device), "zi_reserve: hipSetDevice");
    if (what & ZI_RESERVE_WHOLE_ORDER) {
        const int32_t rc = ensure_whole_order(c);
        if (rc) return rc;
    }
    if (what & ZI_RESERVE_PRUNED_DENSE) {
        const size_t ld = ((size_t)c->max_vocab + 7) / 8 * 8;
        const int32_t rc = ensure_pruned_dense(c, (size_t)c->max_rows * ld * sizeof(float));
        if (rc) return rc;
    }
    return ZI_OK;
}

// Candidate lists longer than kMaxTopK.  k = V: nucleus_kernel settles the
// rows whose keep its 256-entry prefix fixes and flags the rest for
// exact_kernel; 256 < k < V: exact_kernel on every row.  The sort scratch
// (20 bytes per row entry) comes from ensure_whole_order.
static int32_t run_whole_order(zi_ctx *c, const zi_params *p, const zi_batch *b, const zi::RowSource &src,
                               const zi::Plan &pl, uint32_t k, const float *uniforms, const zi_sample_out *out) {
    if ((out->cand_ids || out->cand_vals || out->probs) && out->cand_ld < 1)
        return zi_fail(ZI_ERR_INVALID, "zi_sample_rows: cand_ld=%d < 1", out->cand_ld);
    const int32_t rc = ensure_whole_order(c);
    if (rc) return rc;
    const uint32_t V = (uint32_t)b->vocab;
    const bool whole = k >= V;
    if (whole) {
        zi::SampleParams P;
        std::memset(&P, 0, sizeof P);
        P.src = src;
        P.k = zi::kMaxTopK;  // prefix length
        P.temp = p->temp;
        P.top_p = p->top_p;
        P.min_p = p->min_p;
        P.xtc_p = p->xtc_probability;
        P.xtc_thr = p->xtc_threshold;
        P.xtc_min_keep = (int)(p->xtc_min_keep > 0x7FFFFFFFu ? 0x7FFFFFFFu : p->xtc_min_keep);
        P.uniforms = uniforms;
        P.tok = out->tok;
        P.margin = out->margin;
        P.ndraws = out->ndraws;
        P.keep = out->keep;
        P.cand_ids = out->cand_ids;
        P.cand_vals = out->cand_vals;
        P.probs = out->probs;
        P.cand_ld = out->cand_ld;
        P.g_key = c->g_key;
        P.g_val = c->g_val;
        P.g_cnt = c->g_cnt;
        P.tickets = c->tickets;
        P.n_all = (int)V;
        P.g_stat = c->g_stat;
        P.nuc_flag = c->nuc_flag;
        hipError_t e = zi::launch_nucleus(P, b->dtype, pl.nv, b->rows, c->stream);
        if (e != hipSuccess) return zi_hip_fail(e, "nucleus kernel launch");
    }
    zi::ExactParams X;
    std::memset(&X, 0, sizeof X);
    X.src = src;
    X.n = (int)k;
    X.temp = p->temp;
    X.top_p = p->top_p;
    X.min_p = p->min_p;
    X.xtc_p = p->xtc_probability;
    X.xtc_thr = p->xtc_threshold;
    X.xtc_min_keep = (int)(p->xtc_min_keep > 0x7FFFFFFFu ? 0x7FFFFFFFu : p->xtc_min_keep);
    X.uniforms = uniforms;
    X.tok = out->tok;
    X.margin = out->margin;
    X.ndraws = out->ndraws;
    X.keep = out->keep;
    X.cand_ids = out->cand_ids;
    X.cand_vals = out->cand_vals;
    X.probs = out->probs;
    X.cand_ld = out->cand_ld;
    X.flags = whole ? c->nuc_flag : nullptr;
    X.g_stat = whole ? c->g_stat : nullptr;
    X.n_all = (int)V;
    const size_t plane = (size_t)c->max_rows * (size_t)c->ex_ld;
    X.keys = c->ex_sort;
    X.key0 = c->ex_sort + plane;
    X.id0 = c->ex_sort + 2 * plane;
    X.key1 = c->ex_sort + 3 * plane;
    X.id1 = c->ex_sort + 4 * plane;
    X.ldk = c->ex_ld;
    // bf16 rows without a softcap, XTC or candidate outputs: the flagged rows
    // go through the sort-free pass first; what it cannot take (or any other
    // row) stays flagged for the sorting pass
    const bool xtc = p->xtc_probability > 0.0f && p->xtc_threshold <= 0.5f;
    if (whole && b->dtype == ZI_BF16 && src.cap <= 0.0f && !xtc && !out->cand_ids && !out->cand_vals &&
        !out->probs) {
        hipError_t ew = zi::launch_whole(X, b->rows, c->stream);
        if (ew != hipSuccess) return zi_hip_fail(ew, "whole-order kernel launch");
    }
    hipError_t e = zi::launch_exact(X, b->dtype, b->rows, c->stream);
    if (e != hipSuccess) return zi_hip_fail(e, "exact kernel launch");
    return ZI_OK;
}

// zi_sample_rows after the batch checks, on scratch S and stream st.  c (for
// the whole-order path's lazily allocated sort scratch) may be NULL: top_k
// resolving to more than kMaxTopK is then refused.
static int32_t sample_core(zi_ctx *c, const Scratch &S, hipStream_t st, const zi_params *p, const zi_batch *b,
                           const float *uniforms, const zi_sample_out *out, const char *fn) {
    const zi::Plan pl = zi::plan_rows(b->rows, b->vocab, b->dtype);
    zi::RowSource src;
    int32_t rc = fill_source(b, p, true, src, pl, fn);
    if (rc) return rc;
    if (src.hist && src.hist_ld > zi::kMaxWinHost) {  // the kernels prefetch whole history rows
        if (!S.win_ids)
            return zi_fail(ZI_ERR_UNSUPPORTED, "%s: hist_ld %d > %d", fn, src.hist_ld, zi::kMaxWinHost);
        hipError_t e = zi::launch_window_compact(src.hist, src.hist_len, src.hist_ld, src.win, b->rows, S.win_ids,
                                                 S.win_len, st);
        if (e != hipSuccess) return zi_hip_fail(e, "window compaction launch");
        src.hist = S.win_ids;
        src.hist_len = S.win_len;
        src.hist_ld = zi::kMaxWinHost;
    }

    if (p->temp <= 0.0f)  // greedy: argmax of the penalized row (src/sampler.zig:193)
        return run_argmax(S, st, src, b, pl, out->tok, out->margin, nullptr, nullptr, out->ndraws);

    if (!uniforms) return zi_fail(ZI_ERR_INVALID, "%s: uniforms is NULL", fn);
    const uint32_t V = (uint32_t)b->vocab;
    const uint32_t k = (p->top_k == 0 || p->top_k > V) ? V : p->top_k;  // src/sampler.zig:197
    if (k > (uint32_t)zi::kMaxTopK) {
        if (!c) return zi_fail(ZI_ERR_UNSUPPORTED, "%s: top_k resolves to %u > %d", fn, k, zi::kMaxTopK);
        return run_whole_order(c, p, b, src, pl, k, uniforms, out);
    }
    if ((out->cand_ids || out->cand_vals || out->probs) && out->cand_ld < (int32_t)k)
        return zi_fail(ZI_ERR_INVALID, "%s: cand_ld=%d < k=%u", fn, out->cand_ld, k);

    zi::SampleParams P;
    std::memset(&P, 0, sizeof P);
    P.src = src;
    P.k = (int)k;
    P.temp = p->temp;
    P.top_p = p->top_p;
    P.min_p = p->min_p;
    P.xtc_p = p->xtc_probability;
    P.xtc_thr = p->xtc_threshold;
    P.xtc_min_keep = (int)(p->xtc_min_keep > 0x7FFFFFFFu ? 0x7FFFFFFFu : p->xtc_min_keep);
    P.uniforms = uniforms;
    P.tok = out->tok;
    P.margin = out->margin;
    P.ndraws = out->ndraws;
    P.keep = out->keep;
    P.cand_ids = out->cand_ids;
    P.cand_vals = out->cand_vals;
    P.probs = out->probs;
    P.cand_ld = out->cand_ld;
    P.g_key = S.g_key;
    P.g_val = S.g_val;
    P.g_cnt = S.g_cnt;
    P.tickets = S.tickets;
    hipError_t e = zi::launch_sample(P, b->dtype, pl.nv, b->rows, st);
    if (e != hipSuccess) return zi_hip_fail(e, "sample kernel launch");
    return ZI_OK;
}

extern "C" int32_t zi_sample_rows(zi_ctx *c, const zi_params *p, const zi_batch *b, const float *uniforms,
                                  const zi_sample_out *out) {
    int32_t rc = check_batch(c, b, "zi_sample_rows");
    if (rc) return rc;
    if (!p || !out || !out->tok || !out->margin)
        return zi_fail(ZI_ERR_INVALID, "zi_sample_rows: NULL params/out/tok/margin");
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    return sample_core(c, ctx_scratch(c), c->stream, p, b, uniforms, out, "zi_sample_rows");
}

extern "C" int32_t zi_sample_rows_pruned(zi_ctx *c, const zi_params *p, const zi_batch *b, const uint32_t *groups,
                                         const int32_t *group_count, int32_t groups_ld, const float *uniforms,
                                         const zi_sample_out *out) {
    const char *fn = "zi_sample_rows_pruned";
    int32_t rc = check_batch(c, b, fn);
    if (rc) return rc;
    if (!p || !out || !out->tok || !out->margin) return zi_fail(ZI_ERR_INVALID, "%s: NULL params/out/tok/margin", fn);
    if (!groups || !group_count || groups_ld < 1)
        return zi_fail(ZI_ERR_INVALID, "%s: groups/group_count NULL or groups_ld=%d", fn, groups_ld);
    if (groups_ld > zi::kMaxGroupsHost)
        return zi_fail(ZI_ERR_UNSUPPORTED, "%s: groups_ld=%d > %d", fn, groups_ld, zi::kMaxGroupsHost);
    if (b->vocab < 16) return zi_fail(ZI_ERR_UNSUPPORTED, "%s: vocab %d < 16", fn, b->vocab);
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    {
        const uint32_t V0 = (uint32_t)b->vocab;
        const uint32_t k0 = (p->top_k == 0 || p->top_k > V0) ? V0 : p->top_k;
        // The softcap (model.zig:2492) runs after the fill (:2127) and turns it
        // into -cap*tanh(9); whole-vocabulary and long top-k lists order every
        // id.  Both take the dense path on the row the reference builds.
        if (p->final_logit_softcap > 0.0f || (p->temp > 0.0f && k0 > (uint32_t)zi::kMaxTopK)) {
            const size_t elt = b->dtype == ZI_F32 ? 4 : 2;
            const int64_t dld = ((int64_t)b->vocab + 7) / 8 * 8;  // the dense rows' own stride
            rc = ensure_pruned_dense(c, (size_t)b->rows * (size_t)dld * elt);
            if (rc) return rc;
            hipError_t e = zi::launch_pruned_fill(b->logits, c->pr_dense, b->ld, dld, b->vocab, b->rows, b->dtype,
                                                  groups, group_count, groups_ld, c->stream);
            if (e != hipSuccess) return zi_hip_fail(e, "pruned fill launch");
            zi_batch bd = *b;
            bd.logits = c->pr_dense;
            bd.ld = (int32_t)dld;
            return zi_sample_rows(c, p, &bd, uniforms, out);
        }
    }
    const zi::Plan pl = zi::plan_rows(b->rows, b->vocab, b->dtype);
    zi::RowSource src;
    rc = fill_source(b, p, true, src, pl, fn);
    if (rc) return rc;
    if (src.hist && src.hist_ld > zi::kMaxWinHost) {  // the kernel prefetches whole history rows
        hipError_t e = zi::launch_window_compact(src.hist, src.hist_len, src.hist_ld, src.win, b->rows, c->win_ids,
                                                 c->win_len, c->stream);
        if (e != hipSuccess) return zi_hip_fail(e, "window compaction launch");
        src.hist = c->win_ids;
        src.hist_len = c->win_len;
        src.hist_ld = zi::kMaxWinHost;
    }
    const uint32_t V = (uint32_t)b->vocab;
    const uint32_t k = (p->top_k == 0 || p->top_k > V) ? V : p->top_k;  // src/sampler.zig:197
    if (p->temp > 0.0f) {
        if (!uniforms) return zi_fail(ZI_ERR_INVALID, "%s: uniforms is NULL", fn);
        if (k > (uint32_t)zi::kMaxTopK)
            return zi_fail(ZI_ERR_UNSUPPORTED, "%s: top_k resolves to %u > %d", fn, k, zi::kMaxTopK);
        if ((out->cand_ids || out->cand_vals || out->probs) && out->cand_ld < (int32_t)k)
            return zi_fail(ZI_ERR_INVALID, "%s: cand_ld=%d < k=%u", fn, out->cand_ld, k);
    }
    zi::SampleParams P;
    std::memset(&P, 0, sizeof P);
    P.src = src;
    P.k = (int)(k > (uint32_t)zi::kMaxTopK ? (uint32_t)zi::kMaxTopK : k);
    P.temp = p->temp;
    P.top_p = p->top_p;
    P.min_p = p->min_p;
    P.xtc_p = p->xtc_probability;
    P.xtc_thr = p->xtc_threshold;
    P.xtc_min_keep = (int)(p->xtc_min_keep > 0x7FFFFFFFu ? 0x7FFFFFFFu : p->xtc_min_keep);
    P.uniforms = p->temp > 0.0f ? uniforms : nullptr;
    P.tok = out->tok;
    P.margin = out->margin;
    P.ndraws = out->ndraws;
    P.keep = out->keep;
    P.cand_ids = out->cand_ids;
    P.cand_vals = out->cand_vals;
    P.probs = out->probs;
    P.cand_ld = out->cand_ld;
    P.groups = groups;
    P.group_count = group_count;
    P.groups_ld = groups_ld;
    hipError_t e = zi::launch_pruned(P, b->dtype, b->rows, c->stream);
    if (e != hipSuccess) return zi_hip_fail(e, "pruned kernel launch");
    return ZI_OK;
}

extern "C" int32_t zi_argmax_rows(zi_ctx *c, const zi_batch *b, uint32_t *out_tok, float *out_margin,
                                  uint32_t *out_tok_low, float *out_margin_true) {
    int32_t rc = check_batch(c, b, "zi_argmax_rows");
    if (rc) return rc;
    if (!out_tok && !out_margin && !out_tok_low && !out_margin_true)
        return zi_fail(ZI_ERR_INVALID, "zi_argmax_rows: no output");
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    const zi::Plan pl = zi::plan_rows(b->rows, b->vocab, b->dtype);
    zi::RowSource src;
    rc = fill_source(b, nullptr, false, src, pl, "zi_argmax_rows");
    if (rc) return rc;
    return run_argmax(ctx_scratch(c), c->stream, src, b, pl, out_tok, out_margin, out_tok_low, out_margin_true,
                      nullptr);
}

static constexpr int kWalkGroups = 256;  // one workgroup per CU

extern "C" int32_t zi_entropy_topk_rows(zi_ctx *c, const zi_batch *b, int32_t k, const uint32_t *draft,
                                        float *out_entropy, uint32_t *out_ids, float *out_probs, int32_t out_ld,
                                        uint32_t *out_argmax, uint8_t *out_accept) {
    int32_t rc = check_batch(c, b, "zi_entropy_topk_rows");
    if (rc) return rc;
    if (k < 1 || k > zi::kMaxEntropyK)
        return zi_fail(ZI_ERR_INVALID, "zi_entropy_topk_rows: k=%d outside [1, %d]", k, zi::kMaxEntropyK);
    if ((out_ids || out_probs) && out_ld < k)
        return zi_fail(ZI_ERR_INVALID, "zi_entropy_topk_rows: out_ld=%d < k=%d", out_ld, k);
    if (out_accept && !draft) return zi_fail(ZI_ERR_INVALID, "zi_entropy_topk_rows: out_accept needs draft");
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    zi::Plan pl = zi::plan_rows(b->rows, b->vocab, b->dtype);
    // A chunked grid of more than one workgroup per CU would run in rounds
    // that do not overlap; walking workgroups (one round) take such batches.
    const bool walk = (int64_t)b->rows * pl.G > kWalkGroups;
    if (walk) {
        const int gw = std::max(1, std::min(zi::kMaxGHost, kWalkGroups / b->rows));
        int ch = (b->vocab + gw - 1) / gw;
        ch = (ch + 63) / 64 * 64;
        pl.G = (b->vocab + ch - 1) / ch;
        pl.CH = ch;
    }
    zi::EntropyParams P;
    std::memset(&P, 0, sizeof P);
    rc = fill_source(b, nullptr, false, P.src, pl, "zi_entropy_topk_rows");
    if (rc) return rc;
    P.k = k;
    P.draft = draft;
    P.entropy = out_entropy;
    P.ids = out_ids;
    P.probs = out_probs;
    P.out_ld = out_ld;
    P.argmax = out_argmax;
    P.accept = out_accept;
    P.g_key = c->g_key;
    P.g_val = c->g_val;
    P.g_cnt = c->g_cnt;
    P.g_stat = c->g_stat;
    P.tickets = c->tickets;
    hipError_t e = walk ? zi::launch_entropy_walk(P, b->dtype, b->rows, c->stream)
                        : zi::launch_entropy(P, b->dtype, pl.nv, b->rows, c->stream);
    if (e != hipSuccess) return zi_hip_fail(e, "entropy kernel launch");
    return ZI_OK;
}

extern "C" int32_t zi_apply_mask_rows(zi_ctx *c, const zi_batch *b) {
    int32_t rc = check_batch(c, b, "zi_apply_mask_rows");
    if (rc) return rc;
    if (!b->mask || b->mask_ld < (b->vocab + 31) / 32)
        return zi_fail(ZI_ERR_INVALID, "zi_apply_mask_rows: mask missing or mask_ld too small");
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    zi::MaskParams P;
    P.logits = const_cast<void *>(b->logits);
    P.ld = b->ld;
    P.V = b->vocab;
    P.rows = b->rows;
    P.dtype = b->dtype;
    P.mask = b->mask;
    P.mask_ld = b->mask_ld;
    hipError_t e = zi::launch_mask(P, c->stream);
    if (e != hipSuccess) return zi_hip_fail(e, "mask kernel launch");
    return ZI_OK;
}

// ------------------------------------------------ allocation-free sampling
// zi_sample_rows_noalloc works in one file-scope device array per GPU instead
// of a context's hipMalloc'd scratch.  Its layout is a Scratch for up to
// kNaRows rows: chunk lists for the batches that take the chunked kernel
// (rows < kRowLoopRowsHost; larger batches run one workgroup per row and keep
// their lists in LDS), tickets, and the greedy path's per-chunk records.
namespace {
constexpr int kNaRows = 512;
constexpr int kNaListRows = zi::kRowLoopRowsHost - 1;
constexpr size_t na_align(size_t x) { return (x + 255) & ~(size_t)255; }
constexpr size_t kNaKeyOff = 0;
constexpr size_t kNaValOff = kNaKeyOff + na_align((size_t)kNaListRows * zi::kMaxGHost * zi::kCapAHost * 8);
constexpr size_t kNaCntOff = kNaValOff + na_align((size_t)kNaListRows * zi::kMaxGHost * zi::kCapAHost * 4);
constexpr size_t kNaTicketOff = kNaCntOff + na_align((size_t)kNaRows * zi::kMaxGHost * 4);
constexpr size_t kNaClsOff = kNaTicketOff + na_align((size_t)kNaRows * 4);
constexpr size_t kNaRawOff = kNaClsOff + na_align((size_t)kNaRows * zi::kMaxGHost * 16 * 8);
constexpr size_t kNaTop2Off = kNaRawOff + na_align((size_t)kNaRows * zi::kMaxGHost * 16 * 4);
constexpr size_t kNaTailOff = kNaTop2Off + na_align((size_t)kNaRows * zi::kMaxGHost * 2 * 4);
constexpr size_t kNaBytes = kNaTailOff + na_align((size_t)kNaRows * 16 * 4);
static_assert(kNaBytes <= (size_t)8 << 20, "the static scratch stays under 8 MiB");

std::mutex g_na_mu;
constexpr int kNaMaxDevices = 64;
uint8_t *g_na_ptr[kNaMaxDevices];  // device address of `scratch` on each device (hipGetSymbolAddress)
}  // namespace

// The scratch array itself.  In host code its name only stands for the
// symbol; kernels get the per-device address from hipGetSymbolAddress.
static __device__ __align__(256) uint8_t scratch[kNaBytes];

// Zeroes the first n tickets (a kernel, not hipMemsetAsync, so that the call
// can be captured into a HIP graph).
__global__ void na_zero_tickets(int32_t *t, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) t[i] = 0;
}

static int32_t noalloc_scratch(int dev, Scratch &S) {
    if (dev < 0 || dev >= kNaMaxDevices)
        return zi_fail(ZI_ERR_UNSUPPORTED, "zi_sample_rows_noalloc: device %d >= %d", dev, kNaMaxDevices);
    uint8_t *base;
    {
        std::lock_guard<std::mutex> lk(g_na_mu);
        if (!g_na_ptr[dev]) {  // once per device, with that device current
            void *ptr = nullptr;
            hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return zi_hip_fail(e, "zi_sample_rows_noalloc: hipGetSymbolAddress(scratch)");
            if (!ptr) return zi_fail(ZI_ERR_HIP, "zi_sample_rows_noalloc: scratch has no device address");
            g_na_ptr[dev] = (uint8_t *)ptr;
        }
        base = g_na_ptr[dev];
    }
    S.g_key = (uint64_t *)(base + kNaKeyOff);
    S.g_val = (float *)(base + kNaValOff);
    S.g_cnt = (int32_t *)(base + kNaCntOff);
    S.tickets = (int32_t *)(base + kNaTicketOff);
    S.g_cls = (uint64_t *)(base + kNaClsOff);
    S.g_raw = (uint32_t *)(base + kNaRawOff);
    S.g_top2 = (float *)(base + kNaTop2Off);
    S.g_tail = (float *)(base + kNaTailOff);
    S.win_ids = nullptr;  // no compaction buffer: hist_ld <= kMaxWinHost
    S.win_len = nullptr;
    return ZI_OK;
}

extern "C" int32_t zi_sample_rows_noalloc(const zi_params *p, const zi_batch *b, const float *uniforms,
                                          const zi_sample_out *out, void *stream) {
    const char *fn = "zi_sample_rows_noalloc";
    // every size check before any HIP call
    if (!p || !b || !out || !out->tok || !out->margin)
        return zi_fail(ZI_ERR_INVALID, "%s: NULL params/batch/out/tok/margin", fn);
    if (!b->logits) return zi_fail(ZI_ERR_INVALID, "%s: logits is NULL", fn);
    if (b->dtype != ZI_F32 && b->dtype != ZI_BF16) return zi_fail(ZI_ERR_INVALID, "%s: dtype %d", fn, b->dtype);
    if (b->rows < 1 || b->vocab < 1) return zi_fail(ZI_ERR_INVALID, "%s: rows=%d vocab=%d", fn, b->rows, b->vocab);
    if (b->rows > kNaRows) return zi_fail(ZI_ERR_CAPACITY, "%s: rows=%d > %d", fn, b->rows, kNaRows);
    if (b->vocab > zi::kMaxVocab) return zi_fail(ZI_ERR_CAPACITY, "%s: vocab=%d > %d", fn, b->vocab, zi::kMaxVocab);
    if (b->ld < b->vocab || (b->ld % 8) != 0)
        return zi_fail(ZI_ERR_INVALID, "%s: ld=%d must be >= vocab and a multiple of 8", fn, b->ld);
    if (((uintptr_t)b->logits & 15u) != 0) return zi_fail(ZI_ERR_INVALID, "%s: logits not 16-byte aligned", fn);
    if (p->temp > 0.0f) {
        const uint32_t V = (uint32_t)b->vocab;
        const uint32_t k = (p->top_k == 0 || p->top_k > V) ? V : p->top_k;
        if (k > (uint32_t)zi::kMaxTopK)
            return zi_fail(ZI_ERR_UNSUPPORTED, "%s: top_k resolves to %u > %d (whole-order sorting needs a context)",
                           fn, k, zi::kMaxTopK);
    }
    if (b->hist && b->hist_ld > zi::kMaxWinHost)
        return zi_fail(ZI_ERR_UNSUPPORTED, "%s: hist_ld=%d > %d", fn, b->hist_ld, zi::kMaxWinHost);
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
    Scratch S;
    int32_t rc = noalloc_scratch(dev, S);
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(na_zero_tickets, dim3((b->rows + 255) / 256), dim3(256), 0, st, S.tickets, b->rows);
    HIP_TRY(hipGetLastError(), "zi_sample_rows_noalloc: ticket clear launch");
    return sample_core(nullptr, S, st, p, b, uniforms, out, fn);
}
