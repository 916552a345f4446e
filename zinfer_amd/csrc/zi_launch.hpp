// zi_launch.hpp -- host-visible kernel argument structs and launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zi {

// Limits shared by the host planner and the kernels.
constexpr int kThreadsHost = 512;   // threads per workgroup (8 wave64s)
constexpr int kMaxGHost = 8;        // chunks per row
constexpr int kCapAHost = 256;      // candidates one chunk may publish
constexpr int kMaxChunkElems = 32768;
constexpr int kMaxVocab = kMaxGHost * kMaxChunkElems;  // 262144
constexpr int kMaxWinHost = 1024;   // penalty window
constexpr int kMaxEditsHost = 128;  // sparse edits per row
constexpr int kMaxTopK = 256;
constexpr int kMaxEntropyK = 64;
constexpr int kMaxGroupsHost = 1024;  // listed groups of 8 per pruned row (the reference keeps <= 576)
constexpr int kRowLoopRowsHost = 256;  // sampling batches this large run one workgroup per row (no list scratch)

struct Plan {
    int G, CH, nv;
};
Plan plan_rows(int rows, int V, int dtype);

// One batch of logit rows plus the per-row inputs fused into the streaming
// pass (mask, penalty window, sparse edits).  Device pointers.
struct RowSource {
    const void *logits;
    int64_t ld;
    int V, G, CH;  // vocab, chunks per row, chunk elements (multiple of 64)
    const uint32_t *hist;
    const int32_t *hist_len;
    int hist_ld, win;  // win = penalty window (penalty_last_n)
    const uint32_t *mask;
    int mask_ld;
    const uint32_t *edit_ids;
    const float *edit_delta;
    const int32_t *edit_count;
    int edit_ld;
    float rp, freq, pres;
    int do_rep, do_fp;
    float cap, inv_cap;  // final-logit softcap (cap > 0), applied first
    int cap_body;        // ids below 32*floor(V/32) take the softcap's vector body, the rest its scalar tail
};

struct SampleParams {
    RowSource src;
    int k;
    float temp, top_p, min_p, xtc_p, xtc_thr;
    int xtc_min_keep;
    const float *uniforms;
    uint32_t *tok;
    float *margin;
    int32_t *ndraws;
    int32_t *keep;
    uint32_t *cand_ids;
    float *cand_vals;
    float *probs;
    int cand_ld;
    uint64_t *g_key;  // scratch [rows][G][kCapA]
    float *g_val;
    int32_t *g_cnt;    // [rows][G]
    int32_t *tickets;  // [rows], zero between launches
    // whole-vocabulary rows (nucleus_kernel only)
    int n_all;          // the reference's candidate count (V)
    double *g_stat;     // [rows][G][3]: chunk max, sum exp(x - max)
    int32_t *nuc_flag;  // [rows] out: 1 = keep not fixed by the prefix, run exact_kernel
    // pruned rows (pruned_kernel only): ids [8g, 8g + 8) of the listed groups g
    const uint32_t *groups;      // [rows][groups_ld]
    const int32_t *group_count;  // [rows]
    int groups_ld;
};

// Exact whole-order sampling of one row per workgroup (top_k = 0 rows the
// prefix could not settle, and 256 < top_k < V).
struct ExactParams {
    RowSource src;
    int n;  // candidate count: min(top_k or V, V)
    float temp, top_p, min_p, xtc_p, xtc_thr;
    int xtc_min_keep;
    const float *uniforms;
    uint32_t *tok;
    float *margin;
    int32_t *ndraws;
    int32_t *keep;
    uint32_t *cand_ids;
    float *cand_vals;
    float *probs;
    int cand_ld;
    int32_t *flags;        // [rows]: row r runs iff flags[r] != 0; NULL: every row (whole_kernel clears it)
    const double *g_stat;  // [rows][G][3] chunk (max, sum exp(x - max)) of the prefix pass, or NULL
    int n_all;             // V when g_stat bounds the whole-vocabulary total
    uint32_t *keys, *key0, *id0, *key1, *id1;  // scratch [rows][ldk]: keys in id order, sort buffers
    int64_t ldk;                               // >= V rounded up to 8
};

struct ArgmaxParams {
    RowSource src;
    uint32_t *tok;
    float *margin;
    uint32_t *tok_low;
    float *margin_true;
    int32_t *ndraws;     // greedy sampling writes 0 here when given
    uint64_t *g_cls;     // scratch [rows][G][16] class-max keys (okey << 32 | ~id)
    uint32_t *g_raw;     // scratch [rows][G][16] raw f32 bits of each class winner
    float *g_top2;       // scratch [rows][G][2]
    float *g_tail;       // scratch [rows][16] transformed tail values
    int32_t *tickets;
};

struct EntropyParams {
    RowSource src;
    int k;
    const uint32_t *draft;
    float *entropy;
    uint32_t *ids;
    float *probs;
    int out_ld;
    uint32_t *argmax;
    uint8_t *accept;
    uint64_t *g_key;
    float *g_val;
    int32_t *g_cnt;
    double *g_stat;  // [rows][G][3]: chunk max, sum exp(x - max), sum exp(x - max)(x - max)
    int32_t *tickets;
};

struct MaskParams {
    void *logits;
    int64_t ld;
    int V, rows, dtype;
    const uint32_t *mask;
    int mask_ld;
};

hipError_t launch_sample(const SampleParams &P, int dtype, int nv, int rows, hipStream_t st);
hipError_t launch_nucleus(const SampleParams &P, int dtype, int nv, int rows, hipStream_t st);
hipError_t launch_pruned(const SampleParams &P, int dtype, int rows, hipStream_t st);
// Writes the row the reference's pruned lm_head leaves (-inf, then the listed
// groups' logits) into dense [rows][dst_ld] for the dense sampling path.
hipError_t launch_pruned_fill(const void *logits, void *dense, int64_t ld, int64_t dst_ld, int V, int rows, int dtype,
                              const uint32_t *groups, const int32_t *group_count, int groups_ld, hipStream_t st);
// the final-logit softcap instances of launch_sample / launch_nucleus (zi_sample_cap.hip)
hipError_t launch_sample_capped(const SampleParams &P, int dtype, int nv, int rows, hipStream_t st);
hipError_t launch_nucleus_capped(const SampleParams &P, int dtype, int nv, int rows, hipStream_t st);
hipError_t launch_exact(const ExactParams &P, int dtype, int rows, hipStream_t st);
// bf16 whole-vocabulary rows without a sort (zi_whole.hip); flags required.
hipError_t launch_whole(const ExactParams &P, int rows, hipStream_t st);
hipError_t launch_argmax(const ArgmaxParams &P, int dtype, int nv, int rows, hipStream_t st);
hipError_t launch_entropy(const EntropyParams &P, int dtype, int nv, int rows, hipStream_t st);
// G segments per row, each walked by one workgroup (entropy_walk_kernel).
hipError_t launch_entropy_walk(const EntropyParams &P, int dtype, int rows, hipStream_t st);
hipError_t launch_mask(const MaskParams &P, hipStream_t st);
// Copies each row's penalty window (the last min(hist_len, win) ids) to
// out[row][0, nw) and nw to out_len[row] (rows with hist_ld > kMaxWinHost).
hipError_t launch_window_compact(const uint32_t *hist, const int32_t *hist_len, int hist_ld, int win, int rows,
                                 uint32_t *out, int32_t *out_len, hipStream_t st);

}  // namespace zi
