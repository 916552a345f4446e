// zi_internal.hpp -- host-side internals shared by the C ABI translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/zinfer_hip.h"

struct zi_ctx {
    int device = 0;
    int max_rows = 0;
    int max_vocab = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    // device scratch (see zi_launch.hpp for layouts)
    uint64_t *g_key = nullptr;
    float *g_val = nullptr;
    int32_t *g_cnt = nullptr;
    int32_t *tickets = nullptr;
    double *g_stat = nullptr;
    uint64_t *g_cls = nullptr;
    uint32_t *g_raw = nullptr;
    float *g_top2 = nullptr;
    float *g_tail = nullptr;
    uint32_t *win_ids = nullptr;  // [max_rows][kMaxWinHost] compacted penalty windows
    int32_t *win_len = nullptr;   // [max_rows]
    // whole-order sampling (top_k > 256), allocated on first use
    uint32_t *ex_sort = nullptr;  // 5 x [max_rows][ex_ld] keys in id order, sort keys / ids
    int64_t ex_ld = 0;
    int32_t *nuc_flag = nullptr;  // [max_rows]
    // pruned rows sampled through the dense path (softcap, top_k > 256), on first use
    void *pr_dense = nullptr;
    size_t pr_dense_bytes = 0;
};

int32_t zi_fail(int32_t code, const char *fmt, ...);
int32_t zi_hip_fail(hipError_t e, const char *what);

// Internal view of a zi_vocab (zi_grammar.hip) for the host drivers: its
// size, and a token's piece bytes (host copy).
int32_t zi_vocab_size(const zi_vocab *v);
bool zi_vocab_piece(const zi_vocab *v, uint32_t id, const uint8_t **p, uint32_t *n);
