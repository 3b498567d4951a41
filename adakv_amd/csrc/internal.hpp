// Kernel argument blocks and launcher declarations shared by the translation
// units of libadakv_amd.so.  Host code validates every field before a launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "adakv_amd.h"
#include "common.hpp"

namespace adakv {

struct CentroidArgs {
  const void* k;
  int64_t sb, sh, ss;          // K strides (elements)
  void* c;                     // [B, Hkv, max_blocks, D] (minmax: [..., 2 * D])
  const int32_t* seq_lens;
  int uniform_len;
  int B, Hkv, bs, max_blocks;
  int n_new;                   // 0: every block; > 0: blocks holding the newest n_new tokens
};

struct ScoreArgs {
  const void* q;
  int qdt;
  int64_t qsb, qsh;
  void* c;                     // centroids (rows of appended blocks are rewritten)
  int max_blocks;
  const int32_t* seq_lens;
  int uniform_len, bs;
  int B, Hq, Hkv, G;
  float* scores;               // [B, Hq, sp]
  int sp;
  // fused centroid append: recompute the blocks holding the newest n_new tokens
  int n_new;
  const void* k;
  int kdt;
  int64_t ksb, ksh, kss;
  // softmax records of the scores (nullptr: not wanted), one per (sequence,
  // q-head, score workgroup): group g of record `unit` at part_offset(...)
  float* parts;
  int parts_pitch;
  BudgetCfg cfg;
  int n_app, n_chunks, chunk_rows;   // set by the launcher
  int stream_loads;                  // set by the launcher: non-temporal summary loads
  int q_vec;                   // 1: q has the summary type and 16-byte aligned rows (vector loads)
  int minmax;                  // 1: rows are minmax summaries [max | min] of 2*head_dim elements
};

// Record of a score workgroup's rows for one head (layout in select.hpp):
// the softmax partial of z = score / temperature (m = max z, S = sum
// exp(z - m), T = sum exp(z - m) * (z - m)) and the exact top two content
// blocks of each of its 4 sub-chunks and a bound of the rest.  20 floats (80 bytes).
constexpr int kPartFloats = 20;
constexpr int kPartGroups = kPartFloats / 4;
// Records are stored group-major per (sequence, q-head): the 16-byte group g
// of records 0, 1, 2, ... lies in consecutive words, so a wave whose lane l
// reads group g of record l reads one contiguous KiB (an 80-byte record
// stride would touch a cache line per lane).  Offset in floats.
__host__ __device__ __forceinline__ int64_t part_offset(int b, int Hq, int h, int pitch, int slot, int g) {
  return ((((int64_t)b * Hq + h) * kPartGroups + g) * pitch + slot) * 4;
}

struct SelectArgs {
  const float* scores;
  int sp;
  const int32_t* seq_lens;
  int uniform_len, bs;
  int B, Hq;
  BudgetCfg cfg;
  int32_t* table;              // [B, Hq, T]
  int T;
  double* wbuf;                // [B, Hq] entropy weights (adaptive policy)
  const float* parts;          // softmax records written by the score kernel
  int parts_pitch, n_chunks, chunk_rows;   // records per (sequence, head) row, rows per record
  int chunk_shift;             // log2(chunk_rows) (a power of two)
  int bs_shift;                // log2(bs) when bs is a power of two, else -1
  int n_new;                   // rows >= first appended block are not in any chunk partial
  double lognb_uniform;        // log(max(nb, 2)) of uniform_len, computed on the host (seq_lens null)
};

struct BudgetArgs {
  const double* wbuf;
  const int32_t* seq_lens;
  int uniform_len, bs;
  int B, Hq;
  BudgetCfg cfg;
  int32_t* sel_lens;
};

struct DecodeArgs {
  const void* q;
  int qdt;
  int64_t qsb, qsh;
  const void* k;
  const void* v;
  int64_t sb, sh, ss;
  const int32_t* seq_lens;
  int uniform_len, bs;
  int B, Hq, Hkv, G;
  const int32_t* table;        // nullptr: dense (every block)
  int T;
  const int32_t* sel_lens;     // counts per head, or nullptr: derive them from wbuf / cfg
  const double* wbuf;          // entropy weights when the counts are derived
  BudgetCfg cfg;
  int32_t* sel_lens_out;       // derived counts are written here (may be nullptr)
  float scale_log2;            // sm_scale * log2(e)
  void* out;
  int odt;
  int64_t osb, osh;
  float* partials;             // [B, Hkv, nsplit, G, D + 2]
  int nsplit;
  int min_per;                 // fewest blocks a split takes
  int* counters;               // [B, Hkv]
  int max_blocks;
  int list_cap;                // entries of the per-workgroup block list in LDS
  int merge_in_kernel;         // 1: last split merges (sparse); 0: a merge kernel follows (dense)
  int per_head;                // 1: one workgroup group per q-head (sparse), 0: per KV head
  int table_unique;            // 1: the first sel_lens entries of a row are distinct valid blocks
};

// Fused selection + sparse decode (bf16 / fp16 K/V): the selection fields
// (scores, records, budget, table) and the decode fields (q, K/V, output,
// sel_lens_out) of one step.
struct FusedArgs {
  SelectArgs s;
  DecodeArgs d;
};

struct MergeArgs {
  const float* partials;
  int nsplit;
  int B, Hq, Hkv, G, D;
  const int32_t* seq_lens;
  int uniform_len, bs;
  void* out;
  int odt;
  int64_t osb, osh;
};

// Workspace layout (all offsets 256-byte aligned).
struct WorkspaceLayout {
  size_t scores, weights, counters_plan, counters_dec, partials, table, lens, parts, total;
  int parts_pitch;
  int sp, nsplit_sparse, nsplit_dense, nsplit_max;
};

WorkspaceLayout workspace_layout(const adakv_geometry_t& g, int table_width);

hipError_t launch_centroid(const CentroidArgs& a, int kdt, int cdt, int D, hipStream_t s);
// Per-dimension max and min of every block's keys, rows [max | min] (D <= 128).
hipError_t launch_minmax(const CentroidArgs& a, int kdt, int cdt, int D, hipStream_t s);
// Sets a.n_app, a.n_chunks and a.chunk_rows for the chosen kernel.  D: the
// summary row length (head_dim, or 2 * head_dim when a.minmax).
hipError_t launch_score(ScoreArgs& a, int cdt, int D, hipStream_t s);
hipError_t launch_score_minmax(ScoreArgs& a, int cdt, int D, hipStream_t s);
// Chunks per (sequence, KV head) for any centroid dtype: bound on parts_pitch.
int score_chunks_max(int max_blocks, int D);
hipError_t launch_select(const SelectArgs& a, int max_blocks, hipStream_t s);
// Nucleus weights of every (sequence, q-head) into a.wbuf (ADAKV_POLICY_NUCLEUS).
hipError_t launch_nucleus(const SelectArgs& a, int max_blocks, hipStream_t s);
hipError_t launch_budget(const BudgetArgs& a, hipStream_t s);
hipError_t launch_decode(const DecodeArgs& a, int kvdt, int D, hipStream_t s);
// Threads per workgroup and static LDS bytes of the decode kernel chosen for
// (K/V dtype, head_dim, group size rounded up to a power of two, mode).
int decode_threads(int kvdt, int D, bool sparse);
size_t decode_static_lds(int kvdt, int D, int gmax, bool sparse);
hipError_t launch_merge(const MergeArgs& a, hipStream_t s);
// Fused selection + decode: whether it serves a shape, its LDS bytes (static
// + dynamic) for a head_dim and q-head count, and the launcher.
bool select_decode_supported(int D, int max_blocks, int table_width, int Hq, int sp, int parts_pitch);
size_t select_decode_lds(int D, int Hq, int max_blocks, double avg);
hipError_t launch_select_decode(const FusedArgs& a, int kvdt, int D, int max_blocks, hipStream_t s);

}  // namespace adakv
