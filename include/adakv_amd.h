/*
 * adakv_amd.h -- C ABI of the MI355X (gfx950) AdaKV decode hot path.
 *
 * Plain C: device pointers, sizes, strides and a HIP stream passed as void*.
 * No call allocates device memory or synchronises the host; every launch is
 * ordered on the given stream (NULL = the default stream).  Scratch memory is
 * a caller-owned workspace sized by adakv_workspace_bytes().  Its first 64 KiB
 * hold hand-off counters: zero-fill them once before the first use; every
 * call leaves them zeroed again, whatever the geometry of the next call.
 * Calls that share a workspace must not overlap (use one workspace per stream).
 *
 * Layouts (element strides; head_dim is always the contiguous axis):
 *   query    [batch, n_q_heads, head_dim]
 *   K, V     [batch, n_kv_heads, max_seq_len, head_dim]   (one stride set for both)
 *   centroid [batch, n_kv_heads, max_blocks, head_dim]    (contiguous; kind CENTROID)
 *   minmax   [batch, n_kv_heads, max_blocks, 2*head_dim]  (contiguous; kind MINMAX:
 *            per block, the per-dimension max of its keys, then their min)
 *   table    [batch, n_q_heads, table_width] int32, sel_lens [batch, n_q_heads] int32
 *   output   [batch, n_q_heads, head_dim]
 * seq_lens is a device int32 array [batch] of true token counts, or NULL when
 * every sequence holds max_seq_len tokens.  q-head h reads KV head
 * h / (n_q_heads / n_kv_heads) (grouped-query attention).
 *
 * Reference interfaces replaced (liukefan821/adakv):
 *   adakv_centroid_build   <- AdaKVCache.append_prefill          adakv/attention.py:119-139
 *                             build_block_summaries("centroid")  adakv/estimator.py:27-48
 *                             build_block_summaries("minmax")    adakv/estimator.py:50-57
 *                             (kind MINMAX; AdaKVCache.kmin/kmax, adakv/attention.py:131-138)
 *   adakv_centroid_append  <- update_cache_decode                adakv/runtime.py:43-60
 *                             (and the TODO AdaKVCache.append_decode, adakv/attention.py:141-146)
 *   adakv_block_scores     <- block_scores("centroid")           adakv/estimator.py:62-74
 *                             block_scores("minmax")             adakv/estimator.py:76-79
 *   adakv_plan             <- plan_selection                     adakv/attention.py:149-247
 *                             (estimator.py:62-74, budget.py:45-86, selector.py:18-60)
 *   adakv_sparse_decode    <- block_sparse_decode                adakv/kernels/block_sparse_decode.py:103-135
 *   adakv_decode_fused     <- adakv_decode_attention             adakv/attention.py:250-268
 *                             adakv_decode_step                  adakv/runtime.py:85-112
 *   adakv_dense_decode     <- dense_decode                       benchmarks/efficiency/bench_decode_latency.py:40-53
 * Eviction baselines (a retained set frozen at prefill, adakv/baselines_rt.py):
 *   adakv_key_importance   <- h2o_key_importance_torch           adakv/baselines_rt.py:43-64
 *                             snapkv_key_importance_torch (window) adakv/baselines_rt.py:67-78
 *   adakv_importance_pool  <- the max_pool1d of snapkv_key_importance_torch  adakv/baselines_rt.py:79-80
 *   adakv_retain_blocks    <- retain_blocks_torch                adakv/baselines_rt.py:83-127
 *   adakv_frozen_table     <- frozen_decode_block_table          adakv/baselines_rt.py:158-205
 *   adakv_mask_table       <- mask_to_block_table                adakv/baselines_rt.py:139-155
 *                             (and frozen_decode_block_table on a mask)
 */
#ifndef ADAKV_AMD_H
#define ADAKV_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ADAKV_ABI_VERSION 6

/* Status codes.  Argument errors are detected on the host before any launch. */
enum {
  ADAKV_OK = 0,
  ADAKV_ERR_NULL = 1,         /* a required pointer is NULL                        */
  ADAKV_ERR_SHAPE = 2,        /* inconsistent sizes (e.g. n_q_heads % n_kv_heads)  */
  ADAKV_ERR_DTYPE = 3,        /* unsupported or mismatched element type            */
  ADAKV_ERR_UNSUPPORTED = 4,  /* valid but not built: head_dim, group, max_blocks  */
  ADAKV_ERR_WORKSPACE = 5,    /* workspace too small or not 256-byte aligned       */
  ADAKV_ERR_LAUNCH = 6,       /* the HIP runtime reported a launch error           */
  ADAKV_ERR_VALUE = 7,        /* bad parameter value (budget, policy, alignment)   */
  ADAKV_ERR_SCRATCH = 8       /* the step needs more scratch than the static array
                               * of adakv_decode_fused_noalloc holds                */
};

/* Bytes of the static device scratch array behind adakv_decode_fused_noalloc
 * (one per GPU, held by the library until the process ends).  It covers, at
 * block_size 16 and head_dim 128: batch 1 up to 512K tokens (32 q / 8 KV
 * heads), batch 8 at 128K, batch 4 with 64 q heads at 64K. */
#define ADAKV_NOALLOC_SCRATCH_BYTES (16u << 20)

enum { ADAKV_F32 = 0, ADAKV_F16 = 1, ADAKV_BF16 = 2 };

/* Block summary kinds (the reference's estimator argument, adakv/attention.py:185-198). */
enum { ADAKV_SUMMARY_CENTROID = 0, ADAKV_SUMMARY_MINMAX = 1 };

/* Budget policies (adakv/budget.py:45-86): fixed top-k, the entropy weight
 * ("adaptive") and the nucleus weight ("adaptive_nucleus", budget.py:38-41). */
enum { ADAKV_POLICY_FIXED = 0, ADAKV_POLICY_ADAPTIVE = 1, ADAKV_POLICY_NUCLEUS = 2 };

typedef struct {
  int32_t batch;        /* sequences in the batch (<= 4096, batch*n_kv_heads <= 12288) */
  int32_t n_q_heads;
  int32_t n_kv_heads;   /* n_q_heads / n_kv_heads <= 16                            */
  int32_t head_dim;     /* 32, 64, 128 or 256                                      */
  int32_t block_size;   /* tokens per KV block, 1..256                             */
  int32_t max_seq_len;  /* token capacity of the K/V views                         */
  int32_t max_blocks;   /* centroid rows per (sequence, KV head); >= ceil(max_seq_len/block_size), <= 32768 */
} adakv_geometry_t;

typedef struct {        /* query [batch, n_q_heads, head_dim] */
  const void* data;
  int32_t dtype;
  int64_t stride_b, stride_h;
} adakv_query_t;

typedef struct {        /* output [batch, n_q_heads, head_dim] */
  void* data;
  int32_t dtype;
  int64_t stride_b, stride_h;
} adakv_output_t;

typedef struct {        /* K and V caches [batch, n_kv_heads, max_seq_len, head_dim] */
  const void* k;
  const void* v;
  int32_t dtype;        /* same element type for K and V                           */
  int64_t stride_b, stride_h, stride_s;
} adakv_kv_t;

typedef struct {        /* block summaries, contiguous: [batch, n_kv_heads, max_blocks, row]   */
  void* data;
  int32_t dtype;        /* ADAKV_F32 (exact selection parity) or ADAKV_BF16 / ADAKV_F16 */
  int32_t kind;         /* ADAKV_SUMMARY_CENTROID: row = head_dim (the block's mean key);
                         * ADAKV_SUMMARY_MINMAX: row = 2*head_dim, [max | min] of the
                         * block's keys per dimension; head_dim <= 128, dtype the key
                         * dtype or ADAKV_F32 (both exact)                              */
} adakv_centroid_t;

typedef struct {        /* plan_selection keyword arguments (adakv/attention.py:149-162) */
  double avg_budget;
  int32_t k_min, k_max;
  int32_t n_sink_blocks, n_local_blocks, c_min;
  double temperature;
  int32_t policy;
  double nucleus_p;     /* mass target of ADAKV_POLICY_NUCLEUS (compared in fp32)   */
} adakv_budget_t;

typedef struct {        /* block_table [batch, n_q_heads, table_width], sel_lens [batch, n_q_heads] */
  int32_t* block_table;
  int32_t table_width;
  int32_t* sel_lens;
} adakv_selection_t;

const char* adakv_status_string(int status);
int adakv_abi_version(void);

/* Width of the block table a plan writes: the largest per-head count any
 * sequence can receive, max(1, min(max(k_max, sink+local+c_min), max_blocks)).
 * The reference returns width max(sel_lens) after a device->host sync
 * (adakv/attention.py:242); this ABI never syncs and uses the static bound. */
int32_t adakv_table_width(const adakv_geometry_t* g, const adakv_budget_t* p);

/* Workspace bytes for plan / decode / fused / dense calls on this geometry. */
size_t adakv_workspace_bytes(const adakv_geometry_t* g, int32_t table_width);

/* Summary of every block over its real tokens: the mean key (sequential fp32
 * sum / count, stored in the centroid dtype; adakv/estimator.py:27-48,
 * adakv/attention.py:119-139) or, for kind MINMAX, the per-dimension max and
 * min of its keys (adakv/estimator.py:50-57, adakv/attention.py:131-138). */
int adakv_centroid_build(const adakv_geometry_t* g, const adakv_kv_t* kv, const int32_t* seq_lens,
                         const adakv_centroid_t* centroid, void* stream);

/* After n_new tokens were written at positions [len-n_new, len) of every
 * sequence, recompute the summaries of the blocks holding them (O(block_size*D)
 * per KV head; identical bits to a full rebuild).  adakv/runtime.py:43-60. */
int adakv_centroid_append(const adakv_geometry_t* g, const adakv_kv_t* kv, const int32_t* seq_lens,
                          int32_t n_new, const adakv_centroid_t* centroid, void* stream);

/* Block scores for every (sequence, q-head, block), fp32, no 1/sqrt(D):
 * q . centroid (adakv/estimator.py:62-74) or, for kind MINMAX, the Quest bound
 * max(q,0) . kmax + min(q,0) . kmin (adakv/estimator.py:76-79).  scores [batch, n_q_heads, pitch] with
 * pitch >= max_blocks; entries past a sequence's last block are left untouched. */
int adakv_block_scores(const adakv_geometry_t* g, const adakv_query_t* q,
                       const adakv_centroid_t* centroid, const int32_t* seq_lens, float* scores,
                       int32_t pitch, void* stream);

/* Score every block (as adakv_block_scores), split the mean-pinned budget across the
 * heads of each sequence, select sink + local + top-scoring blocks.
 * Rows list forced blocks (ascending) then content blocks by descending score
 * (ties: lower block id first); entries past sel_lens are never read (further
 * ranked candidates, then -1).  adakv/attention.py:149-247. */
int adakv_plan(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_centroid_t* centroid,
               const int32_t* seq_lens, const adakv_budget_t* budget, const adakv_selection_t* sel,
               void* workspace, size_t workspace_bytes, void* stream);

/* Attention of each q-head over exactly the tokens of its listed blocks
 * (duplicates and out-of-range ids ignored, tokens >= seq_len masked), fp32
 * accumulation, output in out->dtype.  Each KV block selected by several heads
 * of a group is read once.  adakv/kernels/block_sparse_decode.py:103-135. */
int adakv_sparse_decode(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_kv_t* kv,
                        const int32_t* seq_lens, const adakv_selection_t* sel, float sm_scale,
                        const adakv_output_t* out, void* workspace, size_t workspace_bytes,
                        void* stream);

/* One decode step: optional summary append of the newest append_new tokens,
 * plan, sparse decode.  sel may be NULL (selection kept in the workspace) or
 * name caller buffers that receive the selection.  adakv/attention.py:250-268. */
int adakv_decode_fused(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_kv_t* kv,
                       const adakv_centroid_t* centroid, const int32_t* seq_lens,
                       const adakv_budget_t* budget, const adakv_selection_t* sel,
                       int32_t append_new, float sm_scale, const adakv_output_t* out,
                       void* workspace, size_t workspace_bytes, void* stream);

/* The first of adakv_decode_fused's two launches, alone and exactly as the step
 * issues it: the optional summary append of the newest append_new tokens, the
 * block scores (adakv/estimator.py:62-74) and their per-workgroup softmax
 * records (the entropy statistics of adakv/budget.py:33-37), left in the
 * workspace.  For timing the step's launches separately. */
int adakv_decode_fused_scan(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_kv_t* kv,
                            const adakv_centroid_t* centroid, const int32_t* seq_lens,
                            const adakv_budget_t* budget, int32_t append_new, void* workspace,
                            size_t workspace_bytes, void* stream);

/* adakv_decode_fused without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops or
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * scratch is a static device array of ADAKV_NOALLOC_SCRATCH_BYTES inside the
 * library, one per GPU, shared by every call on that GPU: calls that overlap
 * on one GPU (different streams or host threads) race and must not be issued;
 * calls ordered on one stream are safe.  A geometry whose workspace
 * (adakv_workspace_bytes) exceeds the array returns ADAKV_ERR_SCRATCH before
 * any launch.  The first call on a GPU looks up the array's device address
 * and clears its hand-off counters with a fill kernel on the stream; no call
 * allocates, frees or memsets memory. */
int adakv_decode_fused_noalloc(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_kv_t* kv,
                               const adakv_centroid_t* centroid, const int32_t* seq_lens,
                               const adakv_budget_t* budget, const adakv_selection_t* sel,
                               int32_t append_new, float sm_scale, const adakv_output_t* out,
                               void* stream);

/* Dense split-K flash-decode over every token (the comparison baseline).
 * benchmarks/efficiency/bench_decode_latency.py:40-53. */
int adakv_dense_decode(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_kv_t* kv,
                       const int32_t* seq_lens, float sm_scale, const adakv_output_t* out,
                       void* workspace, size_t workspace_bytes, void* stream);

/* ---- Eviction baselines (H2O, SnapKV) ----------------------------------------
 * A retained block set is chosen once from the prompt's own attention and
 * frozen; decode steps attend it plus the current sink and local blocks
 * through adakv_sparse_decode.  Prompt of ONE sequence:
 *   q [n_q_heads, n_tokens, head_dim], k [n_kv_heads, n_tokens, head_dim]
 * (q-head h reads KV head h / (n_q_heads / n_kv_heads)); tables are
 * adakv_selection_t rows [n_heads, table_width] (batch 1). */
typedef struct {
  const void* q;
  const void* k;
  int32_t dtype;                 /* shared by q and k                                   */
  int32_t n_q_heads, n_kv_heads;
  int32_t head_dim;              /* 64 or 128                                           */
  int32_t n_tokens;              /* 1 .. 1048576                                        */
  int64_t q_stride_h, q_stride_s;  /* elements; 16-byte aligned rows                    */
  int64_t k_stride_h, k_stride_s;
} adakv_prompt_t;

/* Workspace of adakv_key_importance (256-byte aligned): one fp32 per
 * (q-head, query >= first_query), and when those queries are too few to fill
 * the GPU (a SnapKV window), the partial maxima and sums of a key split. */
size_t adakv_importance_workspace_bytes(const adakv_prompt_t* p, int32_t first_query);

/* importance[h, j] = sum over the queries i in [first_query, n_tokens) with
 * i >= j of softmax_j(q_i . k_j * sm_scale), fp32 [n_q_heads, pitch],
 * pitch >= n_tokens.  first_query 0 is H2O's accumulated attention;
 * n_tokens - obs_window is SnapKV's observation window before its pool
 * (adakv/baselines.py:63-79, 95-115).  Matrix-core dot products with fp32
 * accumulation; deterministic. */
int adakv_key_importance(const adakv_prompt_t* p, int32_t first_query, float sm_scale, float* importance,
                         int32_t pitch, void* workspace, size_t workspace_bytes, void* stream);

/* out[h, t] = max of in[h, u] over |u - t| <= kernel / 2 clipped to
 * [0, n_tokens) (odd kernel; in and out must not overlap).  adakv/baselines.py:82-92. */
int adakv_importance_pool(const float* in, float* out, int32_t n_heads, int32_t n_tokens, int32_t pitch,
                          int32_t kernel, void* stream);

/* The frozen retained set of each head: k = min(max(budget, floor), nb)
 * blocks (nb = ceil(n_real / block_size), floor = min(sink + local + c_min, nb)),
 * the sink and local blocks plus the content blocks of largest importance sum
 * over their real tokens (fp64 sums compared in fp32; ties: lower block first).
 * mask uint8 [n_heads, mask_pitch] gets 1/0 for blocks [0, nb); when sel is not
 * NULL it also receives the retained blocks ascending (table_width >= k,
 * sel_lens = k).  nb <= 16384.  adakv/baselines.py:120-160. */
int adakv_retain_blocks(const float* importance, int32_t n_heads, int32_t pitch, int32_t n_real,
                        int32_t block_size, int32_t budget, int32_t n_sink_blocks, int32_t n_local_blocks,
                        int32_t c_min, uint8_t* mask, int32_t mask_pitch, const adakv_selection_t* sel,
                        void* stream);

/* Decode-step table of a frozen set: per head, the frozen blocks (frozen
 * rows, sel_lens entries each, ids < n_frozen_blocks) united with the sink and
 * local blocks of nb_now >= n_frozen_blocks blocks, ascending, count in
 * out->sel_lens.  out->table_width >= min(nb_now, frozen width + sink + local);
 * nb_now <= 65536. */
int adakv_frozen_table(const adakv_selection_t* frozen, int32_t n_heads, int32_t n_frozen_blocks, int32_t nb_now,
                       int32_t n_sink_blocks, int32_t n_local_blocks, const adakv_selection_t* out,
                       void* stream);

/* Ascending table of the nonzero entries of each mask row [0, n_mask_blocks)
 * united with the sink and local blocks of nb_now >= n_mask_blocks blocks
 * (n_sink_blocks = n_local_blocks = 0, nb_now = n_mask_blocks: the mask
 * alone); table_width >= nb_now, count in sel_lens; nb_now <= 65536. */
int adakv_mask_table(const uint8_t* mask, int32_t n_heads, int32_t mask_pitch, int32_t n_mask_blocks,
                     int32_t nb_now, int32_t n_sink_blocks, int32_t n_local_blocks, const adakv_selection_t* out,
                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ADAKV_AMD_H */
