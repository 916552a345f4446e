// JSON grammar mask generation on the device (JsonValidator.applyMask,
// src/grammar.zig:446-479): one lane per token runs the validator over the
// token's piece from the row's state; a wave ballot gives 64 mask bits.
//
// Piece table layout (built once per vocabulary): one 16-byte record per
// token, bytes 0-11 the piece's first 12 bytes, the last word its length
// (bits 0-23) and an end-of-generation flag (bit 24, isEog or the eos id).
// Bytes 12 and on of longer pieces are packed in 16-byte chunks (tail
// buffer, chunk index per token).  A workgroup loads its tokens' records and
// first four tail chunks into registers once and runs every row of the launch
// over them; only bytes past 76 are loaded inside the byte loop.
#include <string.h>

#include <algorithm>
#include <vector>

#include "zi_internal.hpp"
#include "zi_json.hpp"

namespace zi {

static_assert(sizeof(zi_json_state) == 24, "zi_json_state is 24 bytes in the C ABI");

constexpr int kJsonThreads = 256;
constexpr int kJsonBatch = 16;  // validator states per launch (kernel arguments)
constexpr int kCopyBatch = 32;  // cached masks copied per launch

struct JsonRow {
    uint64_t stack;
    int32_t flat;  // flat state, or -1: the row runs JsonFsm from st[]
    uint32_t depth;
};

struct JsonMaskArgs {
    const uint4 *rec;
    const uint4 *tails;
    const uint32_t *toff;
    const JsonTables *tables;
    int V, W, n;
    uint32_t *dst[kJsonBatch];
    JsonRow row[kJsonBatch];
    zi_json_state st[kJsonBatch];
};

// Walks every lane's piece through step(byte) -> accepted, in lock-step: the
// chunk and byte counters are wave-uniform (the inline 12 bytes, then tail
// chunks 1-4 from registers, then chunks loaded as reached), each lane is
// predicated on having bytes left and no rejection, and the walk ends when no
// lane is left.  Every load stays inside the loading lane's own piece.
template <class Step>
__device__ __forceinline__ bool walk_piece(const uint4 &q, const uint4 &t0, const uint4 &t1, const uint4 &t2,
                                           const uint4 &t3, const uint4 *tail, uint32_t len, bool ok, Step step) {
    uint32_t rem = ok ? len : 0u;
    bool alive = rem > 0;
    uint4 c = q;
#pragma unroll 1
    for (uint32_t k = 0;; ++k) {
        if (!__any(alive)) break;
        if (k == 1) c = t0;
        else if (k == 2) c = t1;
        else if (k == 3) c = t2;
        else if (k == 4) c = t3;
        else if (k > 4 && alive) c = tail[k - 1];
        const uint32_t nw = k == 0 ? 3u : 4u;
        for (uint32_t j = 0; j < nw; ++j) {
            uint32_t w = c.x;
            c.x = c.y;
            c.y = c.z;
            c.z = c.w;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (alive) {
                    ok = step(w & 0xFFu);
                    rem -= 1;
                    alive = ok && rem > 0;
                }
                w >>= 8;
            }
            if (!__any(alive)) break;
        }
    }
    return ok;
}

constexpr int kRowsPerBlock = 4;  // rows of the launch per workgroup (blockIdx.y groups)

// A workgroup covers 256 tokens for up to kRowsPerBlock rows: the records
// and the first tail chunks are loaded once and reused for each row.
__global__ __launch_bounds__(kJsonThreads) void json_mask_kernel(JsonMaskArgs A) {
    __shared__ JsonTables t;
    {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(A.tables);
        uint32_t *d = reinterpret_cast<uint32_t *>(&t);
        for (int i = threadIdx.x; i < (int)(sizeof(JsonTables) / 4); i += kJsonThreads) d[i] = src[i];
    }
    const int lane = threadIdx.x & 63;
    const int base = blockIdx.x * kJsonThreads + (threadIdx.x & ~63);
    const int id = base + lane;
    const bool live = id < A.V;
    const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
    uint4 q = z4, t0 = z4, t1 = z4, t2 = z4, t3 = z4;
    const uint4 *tail = A.tails;
    if (live) {
        q = A.rec[id];
        const uint32_t l = q.w & 0xFFFFFFu;
        if (l > 12) {
            tail += A.toff[id];
            t0 = tail[0];
            if (l > 28) t1 = tail[1];
            if (l > 44) t2 = tail[2];
            if (l > 60) t3 = tail[3];
        }
    }
    const uint32_t len = q.w & 0xFFFFFFu;
    const bool eog = (q.w >> 24) & 1u;
    const int word = base >> 5;
    __syncthreads();
    const int r1 = min(A.n, (int)(blockIdx.y + 1) * kRowsPerBlock);
    for (int r = blockIdx.y * kRowsPerBlock; r < r1; ++r) {
        const JsonRow jr = A.row[r];
        bool ok;
        if (jr.flat == (int)kFFinished && jr.depth == 0) {
            // only end-of-generation ids and all-whitespace pieces (:453-465)
            ok = walk_piece(q, t0, t1, t2, t3, tail, eog ? 0u : len, live && (eog || len > 0),
                            [](uint32_t b) { return JsonFsm::ws(b); });
        } else if (jr.flat >= 0) {
            // eog ids rejected (:468-472); empty pieces pass (:474); else tryConsume (:475-477)
            uint32_t fl = (uint32_t)jr.flat, d = jr.depth;
            uint64_t stk = jr.stack;
            ok = walk_piece(q, t0, t1, t2, t3, tail, len, live && !eog,
                            [&](uint32_t b) { return json_table_step(t.cls, t.tab, fl, d, stk, b); });
        } else {
            JsonFsm f;
            f.load(A.st[r]);
            ok = walk_piece(q, t0, t1, t2, t3, tail, len, live && !eog, [&](uint32_t b) { return f.step(b); });
        }
        const uint64_t m = __ballot(ok);
        if (lane < 2 && word + lane < A.W) A.dst[r][word + lane] = (uint32_t)(m >> (32 * lane));
    }
}

// Tokens whose pieces hold a stack byte ({ } [ ] ,) for rows with a flat
// state: the row's mask already holds the bits of every other token (copied
// from the per-state base masks); accepted list tokens are or-ed in.  The
// list's pieces are stored as byte classes (same record and tail layout,
// list order), so each step is one table lookup.  One row per workgroup
// (blockIdx.y).
struct JsonListArgs {
    const uint4 *rec;    // [S] class records
    const uint4 *tails;  // class tail chunks
    const uint32_t *toff;  // [S]
    const uint32_t *list;  // [S] token ids
    const JsonTables *tables;
    int S, n;
    uint32_t *dst[kJsonBatch];
    JsonRow row[kJsonBatch];
};

__global__ __launch_bounds__(kJsonThreads) void json_list_kernel(JsonListArgs A) {
    __shared__ uint8_t tab[kFCount * kClsStride];
    {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(A.tables->tab);
        uint32_t *d = reinterpret_cast<uint32_t *>(tab);
        for (int i = threadIdx.x; i < (int)(sizeof(tab) / 4); i += kJsonThreads) d[i] = src[i];
    }
    const int j = blockIdx.x * kJsonThreads + threadIdx.x;
    const bool live = j < A.S;
    const uint4 z4 = make_uint4(0u, 0u, 0u, 0u);
    uint4 q = z4, t0 = z4, t1 = z4, t2 = z4, t3 = z4;
    uint32_t id = 0;
    const uint4 *tail = A.tails;
    if (live) {
        id = A.list[j];
        q = A.rec[j];
        const uint32_t l = q.w & 0xFFFFFFu;
        if (l > 12) {
            tail += A.toff[j];
            t0 = tail[0];
            if (l > 28) t1 = tail[1];
            if (l > 44) t2 = tail[2];
            if (l > 60) t3 = tail[3];
        }
    }
    const uint32_t len = q.w & 0xFFFFFFu;
    __syncthreads();
    const int r = blockIdx.y;
    const JsonRow jr = A.row[r];
    uint32_t fl = (uint32_t)jr.flat, d = jr.depth;
    uint64_t stk = jr.stack;
    const bool ok = walk_piece(q, t0, t1, t2, t3, tail, len, live,
                               [&](uint32_t c) { return json_class_step(tab, fl, d, stk, c); });
    if (ok && live) atomicOr(&A.dst[r][id >> 5], 1u << (id & 31u));
}

struct CopyArgs {
    const uint32_t *src[kCopyBatch];
    uint32_t *dst[kCopyBatch];
    int W;
};

__global__ __launch_bounds__(kJsonThreads) void mask_copy_kernel(CopyArgs A) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * kJsonThreads + threadIdx.x;
    if (i < A.W) A.dst[r][i] = A.src[r][i];
}

}  // namespace zi

using namespace zi;

struct zi_vocab {
    zi_ctx *ctx = nullptr;
    int V = 0, W = 0;
    uint4 *rec = nullptr;
    uint4 *tails = nullptr;  // bytes 12.. of longer pieces, 16-byte chunks
    uint32_t *toff = nullptr;  // [V] first tail chunk of each token
    uint32_t *one = nullptr;  // [W] mask of zi_json_apply_mask when no cache is kept
    JsonTables *tables = nullptr;
    // masks of the tokens without stack bytes, one per flat state, plus the
    // finished rule (row kFCount) for every token: [kFCount + 1][W]
    uint32_t *base = nullptr;
    uint32_t *list = nullptr;  // [S] tokens with stack bytes (not end-of-generation), longest first
    uint4 *lrec = nullptr;     // [S] their pieces as byte classes: records ...
    uint4 *ltails = nullptr;   // ... tail chunks
    uint32_t *ltoff = nullptr;  // [S]
    int S = 0;
    // per-state cache: cap masks of W words on the device, keys on the host
    int cap = 0;
    uint32_t *cache = nullptr;
    std::vector<zi_json_state> key;
    std::vector<uint64_t> used;  // last call that used the slot (0: empty)
    uint64_t calls = 0;
    std::vector<uint32_t> host_mask;
    std::vector<uint32_t> h_off;  // host copy of the pieces (for host-side consume)
    std::vector<uint8_t> h_buf;
};

int32_t zi_vocab_size(const zi_vocab *v) { return v ? v->V : 0; }

bool zi_vocab_piece(const zi_vocab *v, uint32_t id, const uint8_t **p, uint32_t *n) {
    if (!v || id >= (uint32_t)v->V) return false;
    *p = v->h_buf.data() + v->h_off[id];
    *n = v->h_off[id + 1] - v->h_off[id];
    return true;
}

// Frees every buffer; the first failure is left in zi_last_error() (the
// callers cannot report it) and the rest still runs.
static void release(zi_vocab *v) {
    if (!v) return;
    void *bufs[] = {v->rec, v->tails, v->toff, v->one, v->tables, v->base, v->list, v->lrec, v->ltails, v->ltoff,
                    v->cache};
    hipError_t first = hipSuccess;
    for (void *p : bufs) {
        if (!p) continue;
        const hipError_t e = hipFree(p);
        if (e != hipSuccess && first == hipSuccess) first = e;
    }
    if (first != hipSuccess) zi_hip_fail(first, "zi_vocab release: hipFree");
    delete v;
}

namespace {

struct MaskJob {
    const zi_json_state *st;
    uint32_t *dst;
};

// The full pass: every token of the vocabulary runs the validator.
int32_t launch_full(zi_vocab *v, const std::vector<MaskJob> &jobs) {
    JsonMaskArgs A{};
    A.rec = v->rec;
    A.tails = v->tails;
    A.toff = v->toff;
    A.tables = v->tables;
    A.V = v->V;
    A.W = v->W;
    const dim3 block(kJsonThreads);
    for (size_t j0 = 0; j0 < jobs.size(); j0 += kJsonBatch) {
        const int n = (int)std::min<size_t>(kJsonBatch, jobs.size() - j0);
        A.n = n;
        for (int i = 0; i < n; ++i) {
            A.dst[i] = jobs[j0 + i].dst;
            A.st[i] = *jobs[j0 + i].st;
            JsonFsm f;
            f.load(A.st[i]);
            A.row[i] = JsonRow{f.stack, json_flat(f), f.depth};
        }
        const dim3 grid((v->V + kJsonThreads - 1) / kJsonThreads, (n + kRowsPerBlock - 1) / kRowsPerBlock);
        hipLaunchKernelGGL(json_mask_kernel, grid, block, 0, v->ctx->stream, A);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return zi_hip_fail(e, "json_mask_kernel");
    }
    return ZI_OK;
}


int32_t launch_copies(zi_vocab *v, const std::vector<std::pair<const uint32_t *, uint32_t *>> &cp) {
    CopyArgs A{};
    A.W = v->W;
    for (size_t j0 = 0; j0 < cp.size(); j0 += kCopyBatch) {
        const int n = (int)std::min<size_t>(kCopyBatch, cp.size() - j0);
        for (int i = 0; i < n; ++i) {
            A.src[i] = cp[j0 + i].first;
            A.dst[i] = cp[j0 + i].second;
        }
        const dim3 grid((v->W + kJsonThreads - 1) / kJsonThreads, n);
        hipLaunchKernelGGL(mask_copy_kernel, grid, dim3(kJsonThreads), 0, v->ctx->stream, A);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return zi_hip_fail(e, "mask_copy_kernel");
    }
    return ZI_OK;
}

int32_t launch_list(zi_vocab *v, const std::vector<std::pair<JsonRow, uint32_t *>> &rows) {
    if (v->S == 0) return ZI_OK;
    JsonListArgs A{};
    A.rec = v->lrec;
    A.tails = v->ltails;
    A.toff = v->ltoff;
    A.list = v->list;
    A.tables = v->tables;
    A.S = v->S;
    for (size_t j0 = 0; j0 < rows.size(); j0 += kJsonBatch) {
        const int n = (int)std::min<size_t>(kJsonBatch, rows.size() - j0);
        A.n = n;
        for (int i = 0; i < n; ++i) {
            A.row[i] = rows[j0 + i].first;
            A.dst[i] = rows[j0 + i].second;
        }
        const dim3 grid((v->S + kJsonThreads - 1) / kJsonThreads, n);
        hipLaunchKernelGGL(json_list_kernel, grid, dim3(kJsonThreads), 0, v->ctx->stream, A);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return zi_hip_fail(e, "json_list_kernel");
    }
    return ZI_OK;
}

// Rows with a flat state: the base mask of the state, then the stack-byte
// tokens; finished rows: the finished-rule base mask; other rows (a literal
// other than true / false / null): the full pass.
int32_t launch_masks(zi_vocab *v, const std::vector<MaskJob> &jobs) {
    std::vector<std::pair<const uint32_t *, uint32_t *>> copies;
    std::vector<std::pair<JsonRow, uint32_t *>> lists;
    std::vector<MaskJob> full;
    for (const MaskJob &j : jobs) {
        JsonFsm f;
        f.load(*j.st);
        const int fl = json_flat(f);
        if (fl < 0) {
            full.push_back(j);
        } else if (fl == (int)kFFinished && f.depth == 0) {
            copies.push_back({v->base + (size_t)kFCount * v->W, j.dst});
        } else {
            copies.push_back({v->base + (size_t)fl * v->W, j.dst});
            lists.push_back({JsonRow{f.stack, fl, f.depth}, j.dst});
        }
    }
    int32_t rc = launch_copies(v, copies);
    if (rc == ZI_OK) rc = launch_list(v, lists);
    if (rc == ZI_OK) rc = launch_full(v, full);
    return rc;
}

// Base masks: the full pass from one state per flat state (depth 1; tokens
// without stack bytes never read the stack) and from the finished state,
// then the stack-byte tokens cleared from the flat-state rows.
int32_t build_base(zi_vocab *v, const std::vector<uint32_t> &nostack) {
    const size_t W = (size_t)v->W;
    std::vector<zi_json_state> st(kFCount + 1);
    std::vector<MaskJob> jobs;
    for (uint32_t fl = 0; fl <= kFCount; ++fl) {
        const JsonFsm f = fl < kFCount ? json_unflat(fl, 1, 0ull) : json_unflat(kFFinished, 0, 0ull);
        st[fl] = zi_json_state{};
        f.store(st[fl]);
        jobs.push_back({&st[fl], v->base + fl * W});
    }
    int32_t rc = launch_full(v, jobs);
    if (rc != ZI_OK) return rc;
    std::vector<uint32_t> h((kFCount + 1) * W);
    hipError_t e = hipMemcpyAsync(h.data(), v->base, sizeof(uint32_t) * h.size(), hipMemcpyDeviceToHost, v->ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(v->ctx->stream);
    if (e != hipSuccess) return zi_hip_fail(e, "zi_vocab_create: read base masks");
    for (uint32_t fl = 0; fl < kFCount; ++fl)
        for (size_t w = 0; w < W; ++w) h[fl * W + w] &= nostack[w];
    e = hipMemcpy(v->base, h.data(), sizeof(uint32_t) * h.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) return zi_hip_fail(e, "zi_vocab_create: write base masks");
    return ZI_OK;
}

bool valid_state(const zi_json_state &s) {
    return s.state < kJStates && s.escape <= kEscHex3 && s.num <= kNumExpDigits && s.depth <= kJsonMaxDepth &&
           s.lit_len <= 8 && s.lit_idx <= s.lit_len;
}

// Masks for `rows` states into dst rows (ld words apart).  Cached states are
// copied; misses are computed into a cache slot (then copied) or, when the
// call needs more distinct states than the cache holds, straight into dst.
int32_t json_masks(zi_vocab *v, const zi_json_state *states, int rows, uint32_t *dst, int64_t ld) {
    std::vector<MaskJob> jobs;
    std::vector<std::pair<const uint32_t *, uint32_t *>> copies;
    std::vector<zi_json_state> canon(rows);
    const uint64_t call = ++v->calls;
    for (int r = 0; r < rows; ++r) {
        canon[r] = json_canonical(states[r]);
        uint32_t *out = dst + (int64_t)r * ld;
        int slot = -1;
        for (int s = 0; s < v->cap; ++s)
            if (v->used[s] && memcmp(&v->key[s], &canon[r], sizeof(zi_json_state)) == 0) {
                slot = s;
                break;
            }
        if (slot < 0 && v->cap) {  // replace the least recently used slot not used by this call
            for (int s = 0; s < v->cap; ++s)
                if (v->used[s] != call && (slot < 0 || v->used[s] < v->used[slot])) slot = s;
            if (slot >= 0) {
                v->key[slot] = canon[r];
                jobs.push_back({&v->key[slot], v->cache + (size_t)slot * v->W});
            }
        }
        if (slot < 0) {
            jobs.push_back({&canon[r], out});
            continue;
        }
        v->used[slot] = call;
        copies.push_back({v->cache + (size_t)slot * v->W, out});
    }
    int32_t rc = launch_masks(v, jobs);
    if (rc == ZI_OK) rc = launch_copies(v, copies);
    if (rc != ZI_OK)  // the cache contents are unknown after a failed launch
        std::fill(v->used.begin(), v->used.end(), 0);
    return rc;
}

}  // namespace

extern "C" {

void zi_json_init(zi_json_state *s, int32_t object_only) {
    if (!s) return;
    memset(s, 0, sizeof *s);
    s->state = kJStart;
    s->escape = kEscNone;
    s->num = kNumZero;
    s->object_only = object_only ? 1 : 0;
}

int32_t zi_json_is_finished(const zi_json_state *s) {
    if (!s) return 0;
    JsonFsm f;
    f.load(*s);
    return f.finished() ? 1 : 0;
}

int32_t zi_json_step_byte(zi_json_state *s, uint8_t b) {
    if (!s) return 0;
    JsonFsm f;
    f.load(*s);
    const bool ok = f.step(b);
    f.store(*s);
    return ok ? 1 : 0;
}

int32_t zi_json_consume(zi_json_state *s, const uint8_t *piece, size_t n) {
    if (!s || (!piece && n)) return 0;
    JsonFsm f;
    f.load(*s);
    bool ok = true;
    for (size_t i = 0; i < n && ok; ++i) ok = f.step(piece[i]);
    f.store(*s);
    return ok ? 1 : 0;
}

int32_t zi_json_try_consume(const zi_json_state *s, const uint8_t *piece, size_t n, zi_json_state *out) {
    if (!s || (!piece && n)) return 0;
    JsonFsm f;
    f.load(*s);
    for (size_t i = 0; i < n; ++i)
        if (!f.step(piece[i])) return 0;
    if (out) {
        *out = *s;
        f.store(*out);
    }
    return 1;
}

int32_t zi_vocab_create(zi_vocab **out, zi_ctx *ctx, const uint32_t *piece_off, const uint8_t *piece_buf,
                        uint32_t n_vocab, const uint32_t *eog, uint32_t n_eog, int64_t eos,
                        int32_t cache_states) {
    if (!out || !ctx || !piece_off) return zi_fail(ZI_ERR_INVALID, "zi_vocab_create: NULL argument");
    *out = nullptr;
    if (n_vocab < 1 || n_vocab > (1u << 30)) return zi_fail(ZI_ERR_INVALID, "zi_vocab_create: n_vocab=%u", n_vocab);
    if (n_eog && !eog) return zi_fail(ZI_ERR_INVALID, "zi_vocab_create: eog is NULL");
    if (cache_states < 0 || cache_states > 4096)
        return zi_fail(ZI_ERR_INVALID, "zi_vocab_create: cache_states=%d (0..4096)", cache_states);
    const uint32_t V = n_vocab;
    for (uint32_t i = 0; i < V; ++i) {
        if (piece_off[i + 1] < piece_off[i])
            return zi_fail(ZI_ERR_INVALID, "zi_vocab_create: piece_off decreases at %u", i);
        if (piece_off[i + 1] - piece_off[i] > 0xFFFFFFu)
            return zi_fail(ZI_ERR_INVALID, "zi_vocab_create: piece %u longer than 2^24 - 1 bytes", i);
    }
    const size_t nbuf = piece_off[V];
    if (nbuf && !piece_buf) return zi_fail(ZI_ERR_INVALID, "zi_vocab_create: piece_buf is NULL");
    static JsonTables tables;
    static const bool tables_ok = json_build_tables(tables);
    if (!tables_ok) return zi_fail(ZI_ERR_UNSUPPORTED, "zi_vocab_create: transition table self-check failed");

    std::vector<uint4> rec(V);
    std::vector<uint32_t> toff(V, 0);
    std::vector<uint4> tails;
    for (uint32_t i = 0; i < V; ++i) {
        const uint32_t len = piece_off[i + 1] - piece_off[i];
        if (len > 12) {
            toff[i] = (uint32_t)tails.size();
            const size_t nch = (len - 12 + 15) / 16;
            if (tails.size() + nch > 0xFFFFFFFFull)
                return zi_fail(ZI_ERR_INVALID, "zi_vocab_create: more than 2^32 tail chunks");
            tails.resize(tails.size() + nch, make_uint4(0u, 0u, 0u, 0u));
            memcpy(&tails[toff[i]], piece_buf + piece_off[i] + 12, len - 12);
        }
        uint8_t b[12] = {0};
        memcpy(b, piece_buf + piece_off[i], std::min<uint32_t>(len, 12));
        uint4 q;
        memcpy(&q.x, b, 4);
        memcpy(&q.y, b + 4, 4);
        memcpy(&q.z, b + 8, 4);
        const bool e = (eos >= 0 && (uint64_t)eos == i) || std::find(eog, eog + n_eog, i) != eog + n_eog;
        q.w = len | (e ? 1u << 24 : 0u);
        rec[i] = q;
    }
    // tokens with stack bytes: the per-row list pass; every other token is in the base masks
    std::vector<uint32_t> list;
    std::vector<uint32_t> nostack((V + 31) / 32, 0u);
    for (uint32_t i = 0; i < V; ++i) {
        const uint8_t *p = piece_buf + piece_off[i];
        const uint32_t len = piece_off[i + 1] - piece_off[i];
        bool stack = false;
        for (uint32_t k = 0; k < len && !stack; ++k)
            stack = p[k] == '{' || p[k] == '}' || p[k] == '[' || p[k] == ']' || p[k] == ',';
        if (!stack) nostack[i >> 5] |= 1u << (i & 31);
        else if (!((rec[i].w >> 24) & 1u)) list.push_back(i);
    }
    std::stable_sort(list.begin(), list.end(), [&](uint32_t a, uint32_t b) {
        return piece_off[a + 1] - piece_off[a] > piece_off[b + 1] - piece_off[b];
    });  // similar lengths share a wave
    std::vector<uint4> lrec(list.size());
    std::vector<uint32_t> ltoff(list.size(), 0);
    std::vector<uint4> ltails;
    for (size_t j = 0; j < list.size(); ++j) {
        const uint32_t i = list[j], len = piece_off[i + 1] - piece_off[i];
        std::vector<uint8_t> c(std::max<uint32_t>(len, 12) + 16, 0);
        for (uint32_t k = 0; k < len; ++k) c[k] = tables.cls[piece_buf[piece_off[i] + k]];
        uint4 q;
        memcpy(&q.x, c.data(), 4);
        memcpy(&q.y, c.data() + 4, 4);
        memcpy(&q.z, c.data() + 8, 4);
        q.w = len;
        lrec[j] = q;
        if (len > 12) {
            ltoff[j] = (uint32_t)ltails.size();
            const size_t nch = (len - 12 + 15) / 16;
            ltails.resize(ltails.size() + nch, make_uint4(0u, 0u, 0u, 0u));
            memcpy(&ltails[ltoff[j]], c.data() + 12, len - 12);
        }
    }

    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return zi_hip_fail(e, "zi_vocab_create: hipSetDevice");
    zi_vocab *v = new (std::nothrow) zi_vocab;
    if (!v) return zi_fail(ZI_ERR_OOM, "zi_vocab_create: host allocation");
    v->ctx = ctx;
    v->V = (int)V;
    v->W = (int)((V + 31) / 32);
    v->cap = cache_states;
    v->host_mask.resize(v->W);
    const size_t W = (size_t)v->W;
    const size_t ntail = std::max<size_t>(tails.size(), 1);
    if (hipMalloc(&v->rec, sizeof(uint4) * V) != hipSuccess || hipMalloc(&v->tails, sizeof(uint4) * ntail) != hipSuccess ||
        hipMalloc(&v->toff, sizeof(uint32_t) * V) != hipSuccess || hipMalloc(&v->one, sizeof(uint32_t) * W) != hipSuccess ||
        hipMalloc(&v->tables, sizeof(JsonTables)) != hipSuccess ||
        hipMalloc(&v->base, sizeof(uint32_t) * W * (kFCount + 1)) != hipSuccess ||
        hipMalloc(&v->list, sizeof(uint32_t) * std::max<size_t>(list.size(), 1)) != hipSuccess ||
        hipMalloc(&v->lrec, sizeof(uint4) * std::max<size_t>(lrec.size(), 1)) != hipSuccess ||
        hipMalloc(&v->ltails, sizeof(uint4) * std::max<size_t>(ltails.size(), 1)) != hipSuccess ||
        hipMalloc(&v->ltoff, sizeof(uint32_t) * std::max<size_t>(ltoff.size(), 1)) != hipSuccess ||
        (v->cap && hipMalloc(&v->cache, sizeof(uint32_t) * W * v->cap) != hipSuccess)) {
        release(v);
        return zi_fail(ZI_ERR_OOM, "zi_vocab_create: device allocation (%u tokens, %zu tail chunks)", V, tails.size());
    }
    e = hipMemcpy(v->rec, rec.data(), sizeof(uint4) * V, hipMemcpyHostToDevice);
    if (e == hipSuccess && !tails.empty())
        e = hipMemcpy(v->tails, tails.data(), sizeof(uint4) * tails.size(), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(v->toff, toff.data(), sizeof(uint32_t) * V, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(v->tables, &tables, sizeof(JsonTables), hipMemcpyHostToDevice);
    if (e == hipSuccess && !list.empty()) {
        e = hipMemcpy(v->list, list.data(), sizeof(uint32_t) * list.size(), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(v->lrec, lrec.data(), sizeof(uint4) * lrec.size(), hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(v->ltoff, ltoff.data(), sizeof(uint32_t) * ltoff.size(), hipMemcpyHostToDevice);
        if (e == hipSuccess && !ltails.empty())
            e = hipMemcpy(v->ltails, ltails.data(), sizeof(uint4) * ltails.size(), hipMemcpyHostToDevice);
    }
    if (e != hipSuccess) {
        release(v);
        return zi_hip_fail(e, "zi_vocab_create: upload");
    }
    v->S = (int)list.size();
    const int32_t rc = build_base(v, nostack);
    if (rc != ZI_OK) {
        release(v);
        return rc;
    }
    v->key.resize(v->cap);
    v->used.assign(v->cap, 0);
    v->h_off.assign(piece_off, piece_off + V + 1);
    v->h_buf.assign(piece_buf, piece_buf + nbuf);
    *out = v;
    return ZI_OK;
}

void zi_vocab_destroy(zi_vocab *v) {
    if (!v) return;
    // failures are recorded for zi_last_error; the memory is released anyway
    hipError_t e = hipSetDevice(v->ctx->device);
    if (e == hipSuccess) e = hipStreamSynchronize(v->ctx->stream);
    if (e != hipSuccess) zi_hip_fail(e, "zi_vocab_destroy: device or stream");
    release(v);
}

}  // extern "C"


extern "C" {

int32_t zi_json_mask_rows(zi_ctx *ctx, zi_vocab *v, const zi_json_state *states, int32_t rows,
                          uint32_t *out_mask, int32_t mask_ld) {
    if (!ctx || !v || !states || !out_mask) return zi_fail(ZI_ERR_INVALID, "zi_json_mask_rows: NULL argument");
    if (v->ctx != ctx) return zi_fail(ZI_ERR_INVALID, "zi_json_mask_rows: vocab belongs to another context");
    if (rows < 1) return zi_fail(ZI_ERR_INVALID, "zi_json_mask_rows: rows=%d", rows);
    if (mask_ld < v->W) return zi_fail(ZI_ERR_INVALID, "zi_json_mask_rows: mask_ld=%d < %d", mask_ld, v->W);
    for (int r = 0; r < rows; ++r)
        if (!valid_state(states[r])) return zi_fail(ZI_ERR_INVALID, "zi_json_mask_rows: state %d out of range", r);
    const hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return zi_hip_fail(e, "zi_json_mask_rows: hipSetDevice");
    return json_masks(v, states, rows, out_mask, mask_ld);
}

int32_t zi_json_apply_mask(zi_ctx *ctx, zi_vocab *v, const zi_json_state *s, float *logits, uint32_t n) {
    if (!ctx || !v || !s || !logits) return zi_fail(ZI_ERR_INVALID, "zi_json_apply_mask: NULL argument");
    if (v->ctx != ctx) return zi_fail(ZI_ERR_INVALID, "zi_json_apply_mask: vocab belongs to another context");
    if (n != (uint32_t)v->V) return zi_fail(ZI_ERR_INVALID, "zi_json_apply_mask: n=%u, vocabulary has %d", n, v->V);
    if (!valid_state(*s)) return zi_fail(ZI_ERR_INVALID, "zi_json_apply_mask: state out of range");
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return zi_hip_fail(e, "zi_json_apply_mask: hipSetDevice");
    const int32_t rc = json_masks(v, s, 1, v->one, v->W);
    if (rc != ZI_OK) return rc;
    e = hipMemcpyAsync(v->host_mask.data(), v->one, sizeof(uint32_t) * v->W, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return zi_hip_fail(e, "zi_json_apply_mask: read mask");
    const float ninf = -__builtin_inff();
    for (uint32_t t = 0; t < n; ++t)
        if (!((v->host_mask[t >> 5] >> (t & 31)) & 1u)) logits[t] = ninf;
    return ZI_OK;
}

}  // extern "C"
