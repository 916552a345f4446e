// JSON grammar mask generation on the device (JsonValidator.applyMask,
// src/grammar.zig:446-479): one lane per token runs the validator over the
// token's piece from the row's state; a wave ballot gives 64 mask bits.
//
// Piece table layout (built once per vocabulary): one 16-byte record per
// token, bytes 0-11 the piece's first 12 bytes, the last word its length
// (bits 0-23) and an end-of-generation flag (bit 24, isEog or the eos id).
// Longer pieces read the rest from the byte buffer at their offset.  A token
// costs one coalesced 16-byte load; the FSM stops at the first rejected byte.
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

struct JsonMaskArgs {
    const uint4 *rec;
    const uint8_t *buf;
    const uint32_t *off;
    int V, W;
    uint32_t *dst[kJsonBatch];
    zi_json_state st[kJsonBatch];
};

__device__ __forceinline__ uint32_t piece_byte(const uint4 &q, const uint8_t *buf, uint32_t off, uint32_t i) {
    if (i < 12) {
        const uint32_t w = i < 4 ? q.x : (i < 8 ? q.y : q.z);
        return (w >> ((i & 3u) * 8u)) & 0xFFu;
    }
    return buf[off + i];
}

__global__ __launch_bounds__(kJsonThreads) void json_mask_kernel(JsonMaskArgs A) {
    const int r = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int base = blockIdx.x * kJsonThreads + (threadIdx.x & ~63);
    const int id = base + lane;
    bool ok = false;
    if (id < A.V) {
        const uint4 q = A.rec[id];
        const uint32_t len = q.w & 0xFFFFFFu;
        const bool eog = (q.w >> 24) & 1u;
        const uint32_t off = len > 12 ? A.off[id] : 0u;
        JsonFsm f;
        f.load(A.st[r]);
        if (f.finished()) {  // only end-of-generation ids and all-whitespace pieces (:453-465)
            ok = eog || len > 0;
            for (uint32_t i = 0; i < len && ok && !eog; ++i) ok = JsonFsm::ws(piece_byte(q, A.buf, off, i));
        } else if (eog) {  // :468-472
            ok = false;
        } else {  // empty pieces pass (:474); else tryConsume (:475-477)
            ok = true;
            for (uint32_t i = 0; i < len && ok; ++i) ok = f.step(piece_byte(q, A.buf, off, i));
        }
    }
    const uint64_t m = __ballot(ok);
    const int word = base >> 5;
    if (lane < 2 && word + lane < A.W) A.dst[r][word + lane] = (uint32_t)(m >> (32 * lane));
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
    uint8_t *buf = nullptr;
    uint32_t *off = nullptr;
    uint32_t *one = nullptr;  // [W] mask of zi_json_apply_mask when no cache is kept
    // per-state cache: cap masks of W words on the device, keys on the host
    int cap = 0;
    uint32_t *cache = nullptr;
    std::vector<zi_json_state> key;
    std::vector<uint64_t> used;  // last call that used the slot (0: empty)
    uint64_t calls = 0;
    std::vector<uint32_t> host_mask;
};

static void release(zi_vocab *v) {
    if (!v) return;
    hipFree(v->rec);
    hipFree(v->buf);
    hipFree(v->off);
    hipFree(v->one);
    hipFree(v->cache);
    delete v;
}

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

    std::vector<uint4> rec(V);
    for (uint32_t i = 0; i < V; ++i) {
        const uint32_t len = piece_off[i + 1] - piece_off[i];
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
    if (hipMalloc(&v->rec, sizeof(uint4) * V) != hipSuccess || hipMalloc(&v->buf, nbuf + 16) != hipSuccess ||
        hipMalloc(&v->off, sizeof(uint32_t) * V) != hipSuccess || hipMalloc(&v->one, sizeof(uint32_t) * W) != hipSuccess ||
        (v->cap && hipMalloc(&v->cache, sizeof(uint32_t) * W * v->cap) != hipSuccess)) {
        release(v);
        return zi_fail(ZI_ERR_OOM, "zi_vocab_create: device allocation (%u tokens, %zu piece bytes)", V, nbuf);
    }
    e = hipMemcpy(v->rec, rec.data(), sizeof(uint4) * V, hipMemcpyHostToDevice);
    if (e == hipSuccess && nbuf) e = hipMemcpy(v->buf, piece_buf, nbuf, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(v->off, piece_off, sizeof(uint32_t) * V, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        release(v);
        return zi_hip_fail(e, "zi_vocab_create: upload");
    }
    v->key.resize(v->cap);
    v->used.assign(v->cap, 0);
    *out = v;
    return ZI_OK;
}

void zi_vocab_destroy(zi_vocab *v) {
    if (!v) return;
    hipSetDevice(v->ctx->device);
    hipStreamSynchronize(v->ctx->stream);
    release(v);
}

}  // extern "C"

namespace {

struct MaskJob {
    const zi_json_state *st;
    uint32_t *dst;
};

int32_t launch_masks(zi_vocab *v, const std::vector<MaskJob> &jobs) {
    JsonMaskArgs A{};
    A.rec = v->rec;
    A.buf = v->buf;
    A.off = v->off;
    A.V = v->V;
    A.W = v->W;
    const dim3 block(kJsonThreads);
    for (size_t j0 = 0; j0 < jobs.size(); j0 += kJsonBatch) {
        const int n = (int)std::min<size_t>(kJsonBatch, jobs.size() - j0);
        for (int i = 0; i < n; ++i) {
            A.dst[i] = jobs[j0 + i].dst;
            A.st[i] = *jobs[j0 + i].st;
        }
        const dim3 grid((v->V + kJsonThreads - 1) / kJsonThreads, n);
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
