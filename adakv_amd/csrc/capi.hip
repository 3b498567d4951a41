// extern "C" entry points of libadakv_amd.so: argument validation on the host,
// workspace carving, kernel launches on the caller's stream.  Nothing here
// allocates device memory or waits on the device.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>

#include "adakv_amd.h"
#include "internal.hpp"

namespace adakv {
namespace {

constexpr size_t kAlign = 256;
constexpr int kMaxBlocks = 32768;
constexpr int kMaxSparseSplits = 16;      // the in-kernel merge reads at most 16 partials
constexpr int kSparseMinPer = 32;         // blocks a sparse split takes at least
constexpr int kMaxDenseSplits = 256;
constexpr int kDenseMinBlocksPerSplit = 8;
constexpr int kDenseTargetGroups = 512;   // dense workgroups to aim for: two per CU
constexpr size_t kLdsLimit = 65536;
constexpr int kMaxPlanCounters = 4096;                  // one per sequence
constexpr int kMaxDecodeCounters = 12288;               // one per (sequence, KV head)
constexpr size_t kCounterBytes = (size_t)(kMaxPlanCounters + kMaxDecodeCounters) * 4;

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }
int ceil_div_h(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }
bool valid_dtype(int dt) { return dt == ADAKV_F32 || dt == ADAKV_F16 || dt == ADAKV_BF16; }
int elt_bytes(int dt) { return dt == ADAKV_F32 ? 4 : 2; }
int per_vec(int dt) { return 16 / elt_bytes(dt); }
int gmax_of(int G) { return G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : G <= 8 ? 8 : 16; }
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Summary element type per key element type: the key type itself or fp32;
// fp32 keys may also have bf16 centroids (a rounded mean), but minmax rows
// are kept exact (a rounded max or min would no longer bound the keys).
bool centroid_pair_ok(int kdt, const adakv_centroid_t* c) {
  if (c->dtype == ADAKV_F32) return true;
  if (kdt == ADAKV_F32) return c->kind == ADAKV_SUMMARY_CENTROID && c->dtype == ADAKV_BF16;
  return kdt == c->dtype;
}

// Elements per summary row: head_dim (centroid) or 2 * head_dim (minmax).
int row_len(const adakv_geometry_t* g, const adakv_centroid_t* c) {
  return c->kind == ADAKV_SUMMARY_MINMAX ? 2 * g->head_dim : g->head_dim;
}

int check_geometry(const adakv_geometry_t* g) {
  if (!g) return ADAKV_ERR_NULL;
  if (g->batch < 1 || g->n_q_heads < 1 || g->n_kv_heads < 1 || g->block_size < 1 ||
      g->max_seq_len < 1 || g->max_blocks < 1)
    return ADAKV_ERR_SHAPE;
  if (g->n_q_heads % g->n_kv_heads) return ADAKV_ERR_SHAPE;
  if ((int64_t)g->max_blocks * g->block_size < g->max_seq_len) return ADAKV_ERR_SHAPE;
  if (g->n_q_heads / g->n_kv_heads > 16) return ADAKV_ERR_UNSUPPORTED;
  const int D = g->head_dim;
  if (D != 32 && D != 64 && D != 128 && D != 256) return ADAKV_ERR_UNSUPPORTED;
  if (g->max_blocks > kMaxBlocks || g->block_size > 4096) return ADAKV_ERR_UNSUPPORTED;
  if (g->batch > kMaxPlanCounters || (int64_t)g->batch * g->n_kv_heads > kMaxDecodeCounters)
    return ADAKV_ERR_UNSUPPORTED;
  return ADAKV_OK;
}

int check_kv(const adakv_geometry_t* g, const adakv_kv_t* kv, bool need_v) {
  if (!kv || !kv->k || (need_v && !kv->v)) return ADAKV_ERR_NULL;
  if (!valid_dtype(kv->dtype)) return ADAKV_ERR_DTYPE;
  const int e = per_vec(kv->dtype);
  if (!aligned16(kv->k) || (need_v && !aligned16(kv->v))) return ADAKV_ERR_VALUE;
  if (kv->stride_b % e || kv->stride_h % e || kv->stride_s % e) return ADAKV_ERR_VALUE;
  if (kv->stride_b < 0 || kv->stride_h < 0 || kv->stride_s < 0) return ADAKV_ERR_VALUE;
  (void)g;
  return ADAKV_OK;
}

int check_q(const adakv_query_t* q) {
  if (!q || !q->data) return ADAKV_ERR_NULL;
  if (!valid_dtype(q->dtype)) return ADAKV_ERR_DTYPE;
  return ADAKV_OK;
}

int check_out(const adakv_output_t* o) {
  if (!o || !o->data) return ADAKV_ERR_NULL;
  if (!valid_dtype(o->dtype)) return ADAKV_ERR_DTYPE;
  return ADAKV_OK;
}

int check_centroid(const adakv_geometry_t* g, const adakv_centroid_t* c) {
  if (!c || !c->data) return ADAKV_ERR_NULL;
  if (!valid_dtype(c->dtype)) return ADAKV_ERR_DTYPE;
  if (c->kind != ADAKV_SUMMARY_CENTROID && c->kind != ADAKV_SUMMARY_MINMAX) return ADAKV_ERR_VALUE;
  if (c->kind == ADAKV_SUMMARY_MINMAX && g->head_dim > 128) return ADAKV_ERR_UNSUPPORTED;
  if (!aligned16(c->data)) return ADAKV_ERR_VALUE;
  return ADAKV_OK;
}

int check_budget(const adakv_budget_t* p) {
  if (!p) return ADAKV_ERR_NULL;
  if (p->policy != ADAKV_POLICY_FIXED && p->policy != ADAKV_POLICY_ADAPTIVE && p->policy != ADAKV_POLICY_NUCLEUS)
    return ADAKV_ERR_VALUE;
  if (!isfinite(p->avg_budget) || !isfinite(p->temperature)) return ADAKV_ERR_VALUE;
  if (p->policy == ADAKV_POLICY_NUCLEUS && !isfinite(p->nucleus_p)) return ADAKV_ERR_VALUE;
  if (p->k_min < 0 || p->k_max < 0 || p->n_sink_blocks < 0 || p->n_local_blocks < 0 || p->c_min < 0)
    return ADAKV_ERR_VALUE;
  return ADAKV_OK;
}

int check_ws(const adakv_geometry_t* g, int T, void* ws, size_t bytes) {
  if (!ws) return ADAKV_ERR_NULL;
  if (((uintptr_t)ws & (kAlign - 1)) != 0) return ADAKV_ERR_WORKSPACE;
  if (bytes < workspace_layout(*g, T).total) return ADAKV_ERR_WORKSPACE;
  return ADAKV_OK;
}

int table_width_of(const adakv_geometry_t* g, const adakv_budget_t* p) {
  int64_t w = p->k_max;
  const int64_t f = (int64_t)p->n_sink_blocks + p->n_local_blocks + p->c_min;
  if (f > w) w = f;
  if (w > g->max_blocks) w = g->max_blocks;
  if (w < 1) w = 1;
  return (int)w;
}

int64_t union_max(const adakv_geometry_t& g, int T) {
  return std::min<int64_t>((int64_t)(g.n_q_heads / g.n_kv_heads) * T, g.max_blocks);
}

int list_cap_of(const adakv_geometry_t& g, int T, int nsplit) {
  const int64_t umax = union_max(g, T);
  return (int)std::max<int64_t>(1, std::max<int64_t>(ceil_div_h(umax, nsplit),
                                                     std::min<int64_t>(kSparseMinPer, umax)));
}

// LDS of the decode kernel: its static arrays plus, in sparse mode, the
// weights, the union bitmap and the block list.
size_t decode_lds_bytes(const adakv_geometry_t& g, int kvdt, int list_cap, bool sparse) {
  const int GM = gmax_of(g.n_q_heads / g.n_kv_heads);
  const size_t stat = decode_static_lds(kvdt, g.head_dim, GM, sparse);
  const size_t dyn = sparse ? ((size_t)g.n_q_heads * 8 + 15) / 16 * 16 +
                                  (size_t)(((g.max_blocks + 3) / 4 + 3) / 4 * 4 + list_cap) * 4
                            : 16;
  return stat + dyn;
}

BudgetCfg budget_cfg(const adakv_budget_t* p) {
  BudgetCfg c;
  c.avg = p->avg_budget;
  c.k_min = p->k_min; c.k_max = p->k_max;
  c.sink = p->n_sink_blocks; c.local = p->n_local_blocks; c.c_min = p->c_min;
  c.policy = p->policy;
  c.temperature = p->temperature;
  c.nucleus_p = (float)p->nucleus_p;
  return c;
}

int status_of(hipError_t e) { return e == hipSuccess ? ADAKV_OK : ADAKV_ERR_LAUNCH; }

hipError_t run_summary(const CentroidArgs& a, int kdt, const adakv_centroid_t* c, int D, hipStream_t s) {
  if (c->kind == ADAKV_SUMMARY_MINMAX) return launch_minmax(a, kdt, c->dtype, D, s);
  return launch_centroid(a, kdt, c->dtype, D, s);
}

CentroidArgs centroid_args(const adakv_geometry_t* g, const adakv_kv_t* kv, const int32_t* lens,
                           const adakv_centroid_t* c, int n_new) {
  CentroidArgs a{};
  a.k = kv->k;
  a.sb = kv->stride_b; a.sh = kv->stride_h; a.ss = kv->stride_s;
  a.c = c->data;
  a.seq_lens = lens;
  a.uniform_len = g->max_seq_len;
  a.B = g->batch; a.Hkv = g->n_kv_heads; a.bs = g->block_size; a.max_blocks = g->max_blocks;
  a.n_new = n_new;
  return a;
}

// Blocks any sequence can have: lengths are clamped to max_seq_len on the
// device, so the selection kernels' shapes (scores per thread, the fused
// kernel's eligibility) follow this bound, not the summary buffer's capacity.
int rows_bound(const adakv_geometry_t* g) {
  return std::min(g->max_blocks, (g->max_seq_len + g->block_size - 1) / g->block_size);
}

ScoreArgs score_args(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_centroid_t* c,
                     const int32_t* lens, float* scores, int sp) {
  ScoreArgs sa{};
  sa.q = q->data; sa.qdt = q->dtype; sa.qsb = q->stride_b; sa.qsh = q->stride_h;
  sa.c = c->data; sa.max_blocks = g->max_blocks;
  sa.seq_lens = lens; sa.uniform_len = g->max_seq_len; sa.bs = g->block_size;
  sa.B = g->batch; sa.Hq = g->n_q_heads; sa.Hkv = g->n_kv_heads; sa.G = g->n_q_heads / g->n_kv_heads;
  sa.scores = scores; sa.sp = sp;
  sa.q_vec = q->dtype == c->dtype && q->dtype != ADAKV_F32 && aligned16(q->data) && q->stride_b % 8 == 0 &&
             q->stride_h % 8 == 0;
  sa.minmax = c->kind == ADAKV_SUMMARY_MINMAX;
  return sa;
}

// Scores (with an optional fused centroid append) and their softmax records;
// returns the selection arguments that consume them.
int run_scores(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_centroid_t* c,
               const adakv_kv_t* kv_append, int n_new, const int32_t* lens, const adakv_budget_t* p,
               int32_t* table, int T, char* ws, hipStream_t s, SelectArgs* se_out) {
  const WorkspaceLayout L = workspace_layout(*g, T);
  ScoreArgs sa = score_args(g, q, c, lens, reinterpret_cast<float*>(ws + L.scores), L.sp);
  if (n_new > 0) {
    sa.n_new = n_new;
    sa.k = kv_append->k; sa.kdt = kv_append->dtype;
    sa.ksb = kv_append->stride_b; sa.ksh = kv_append->stride_h; sa.kss = kv_append->stride_s;
  }
  sa.parts = reinterpret_cast<float*>(ws + L.parts);
  sa.parts_pitch = L.parts_pitch;
  sa.cfg = budget_cfg(p);
  if (launch_score(sa, c->dtype, row_len(g, c), s) != hipSuccess) return ADAKV_ERR_LAUNCH;
  SelectArgs& se = *se_out;
  se = SelectArgs{};
  se.scores = sa.scores; se.sp = L.sp;
  se.seq_lens = lens; se.uniform_len = g->max_seq_len; se.bs = g->block_size;
  se.B = g->batch; se.Hq = g->n_q_heads;
  se.cfg = sa.cfg;
  se.table = table; se.T = T;
  se.wbuf = reinterpret_cast<double*>(ws + L.weights);
  se.parts = sa.parts; se.parts_pitch = sa.parts_pitch;
  se.n_chunks = sa.n_chunks; se.chunk_rows = sa.chunk_rows;
  se.chunk_shift = __builtin_ctz((unsigned)sa.chunk_rows);
  se.bs_shift = (g->block_size & (g->block_size - 1)) == 0 ? __builtin_ctz((unsigned)g->block_size) : -1;
  se.n_new = n_new;
  // the entropy weight's divisor np.log(nb) (adakv/budget.py:35), by the host's
  // libm as NumPy computes it, for the one length every sequence has
  if (lens == nullptr) {
    const int nbu = (g->max_seq_len + g->block_size - 1) / g->block_size;
    se.lognb_uniform = std::log((double)std::max(nbu, 2));
  }
  return ADAKV_OK;
}

// Scores and the per-head selection; sel_lens come from the budget kernel
// when requested, otherwise the decode kernel derives them from the weights
// left in the workspace.
int run_plan(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_centroid_t* c,
             const adakv_kv_t* kv_append, int n_new, const int32_t* lens, const adakv_budget_t* p,
             int32_t* table, int T, int32_t* sel_lens, char* ws, hipStream_t s) {
  SelectArgs se;
  int st;
  if ((st = run_scores(g, q, c, kv_append, n_new, lens, p, table, T, ws, s, &se))) return st;
  if (p->policy == ADAKV_POLICY_NUCLEUS && launch_nucleus(se, rows_bound(g), s) != hipSuccess)
    return ADAKV_ERR_LAUNCH;
  if (launch_select(se, rows_bound(g), s) != hipSuccess) return ADAKV_ERR_LAUNCH;
  if (!sel_lens) return ADAKV_OK;
  BudgetArgs ba{};
  ba.wbuf = se.wbuf;
  ba.seq_lens = lens; ba.uniform_len = g->max_seq_len; ba.bs = g->block_size;
  ba.B = g->batch; ba.Hq = g->n_q_heads;
  ba.cfg = se.cfg;
  ba.sel_lens = sel_lens;
  return status_of(launch_budget(ba, s));
}

// Decode fields shared by every decode launch: q, K/V, lengths, scale, output.
DecodeArgs decode_args(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_kv_t* kv,
                       const int32_t* lens, float sm_scale, const adakv_output_t* out) {
  DecodeArgs d{};
  d.q = q->data; d.qdt = q->dtype; d.qsb = q->stride_b; d.qsh = q->stride_h;
  d.k = kv->k; d.v = kv->v; d.sb = kv->stride_b; d.sh = kv->stride_h; d.ss = kv->stride_s;
  d.seq_lens = lens; d.uniform_len = g->max_seq_len; d.bs = g->block_size;
  d.B = g->batch; d.Hq = g->n_q_heads; d.Hkv = g->n_kv_heads; d.G = g->n_q_heads / g->n_kv_heads;
  d.scale_log2 = sm_scale * 1.4426950408889634f;
  d.out = out->data; d.odt = out->dtype; d.osb = out->stride_b; d.osh = out->stride_h;
  return d;
}

// Largest LDS a workgroup may hold on the current device (cached per device).
size_t max_lds_per_block() {
  static int cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return kLdsLimit;
  if (dev < 64 && cache[dev] > 0) return (size_t)cache[dev];
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
    return kLdsLimit;
  if (dev < 64) cache[dev] = v;
  return (size_t)v;
}

// Table-driven sparse decode (table != nullptr) or dense decode (+ merge).
// With sel_lens == nullptr the per-head counts are derived from the budget
// weights in the workspace and written to sel_lens_out.
int run_decode(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_kv_t* kv,
               const int32_t* lens, const int32_t* table, int T, const int32_t* sel_lens,
               const adakv_budget_t* p, int32_t* sel_lens_out, float sm_scale,
               const adakv_output_t* out, char* ws, int T_layout, bool table_unique, hipStream_t s) {
  const WorkspaceLayout L = workspace_layout(*g, T_layout);
  DecodeArgs d = decode_args(g, q, kv, lens, sm_scale, out);
  d.table = table; d.T = T; d.sel_lens = sel_lens;
  d.wbuf = reinterpret_cast<const double*>(ws + L.weights);
  if (p) d.cfg = budget_cfg(p);
  d.sel_lens_out = sel_lens_out;
  d.partials = reinterpret_cast<float*>(ws + L.partials);
  d.counters = reinterpret_cast<int*>(ws + L.counters_dec);
  d.max_blocks = g->max_blocks;
  if (table) {
    // Sparse: one workgroup group per q-head when the hand-off counters allow
    // (each head streams only its own blocks, so a KV head's union is spread
    // over G workgroups instead of one); per KV head otherwise.
    d.per_head = (int64_t)g->batch * g->n_q_heads <= kMaxDecodeCounters;
    d.table_unique = table_unique;
    const int64_t umax = d.per_head ? std::min<int64_t>(T, g->max_blocks) : union_max(*g, T);
    d.nsplit = (int)std::max<int64_t>(1, std::min<int64_t>(ceil_div_h(umax, kSparseMinPer), kMaxSparseSplits));
    d.min_per = kSparseMinPer;
    d.list_cap = (int)std::max<int64_t>(1, std::max<int64_t>(ceil_div_h(umax, d.nsplit),
                                                             std::min<int64_t>(kSparseMinPer, umax)));
    d.merge_in_kernel = 1;
  } else {
    d.nsplit = L.nsplit_dense;
    d.min_per = 1;
    d.list_cap = 0;
    d.merge_in_kernel = 0;
  }
  if (decode_lds_bytes(*g, kv->dtype, d.list_cap, table != nullptr) > kLdsLimit) return ADAKV_ERR_UNSUPPORTED;
  if (launch_decode(d, kv->dtype, g->head_dim, s) != hipSuccess) return ADAKV_ERR_LAUNCH;
  if (table) return ADAKV_OK;
  MergeArgs m{};
  m.partials = d.partials; m.nsplit = d.nsplit;
  m.B = d.B; m.Hq = d.Hq; m.Hkv = d.Hkv; m.G = d.G; m.D = g->head_dim;
  m.seq_lens = lens; m.uniform_len = g->max_seq_len; m.bs = g->block_size;
  m.out = out->data; m.odt = out->dtype; m.osb = out->stride_b; m.osh = out->stride_h;
  return status_of(launch_merge(m, s));
}

}  // namespace

WorkspaceLayout workspace_layout(const adakv_geometry_t& g, int T) {
  WorkspaceLayout L{};
  const int G = g.n_q_heads / g.n_kv_heads;
  L.sp = (g.max_blocks + 3) / 4 * 4;
  const int64_t umax = union_max(g, T);
  L.nsplit_sparse = (int)std::max<int64_t>(1, std::min<int64_t>(ceil_div_h(umax, kSparseMinPer),
                                                                kMaxSparseSplits));
  // dense splits: about kDenseTargetGroups workgroups over the (sequence, KV head)
  // pairs, at least kDenseMinBlocksPerSplit blocks each
  L.nsplit_dense = std::max(1, std::min({ceil_div_h(g.max_blocks, kDenseMinBlocksPerSplit),
                                         ceil_div_h(kDenseTargetGroups, (int64_t)g.batch * g.n_kv_heads),
                                         kMaxDenseSplits}));
  L.nsplit_max = std::max(L.nsplit_sparse, L.nsplit_dense);
  // The counters sit at fixed offsets so that they stay zero however the
  // geometry of successive calls on one workspace changes; everything after
  // them is scratch that every call fully rewrites before reading.
  L.counters_plan = 0;
  L.counters_dec = (size_t)kMaxPlanCounters * 4;
  size_t off = kCounterBytes;
  L.scores = off;        off = align_up(off + (size_t)g.batch * g.n_q_heads * L.sp * 4);
  L.weights = off;       off = align_up(off + (size_t)g.batch * g.n_q_heads * 8);
  L.partials = off;
  off = align_up(off + (size_t)g.batch * g.n_kv_heads * L.nsplit_max * G * (g.head_dim + 2) * 4);
  L.table = off;         off = align_up(off + (size_t)g.batch * g.n_q_heads * T * 4);
  L.lens = off;          off = align_up(off + (size_t)g.batch * g.n_q_heads * 4);
  // records per row for either summary kind (a minmax row is 2 * head_dim long)
  L.parts_pitch = score_chunks_max(g.max_blocks, std::min(2 * g.head_dim, 256));
  L.parts = off;
  off = align_up(off + (size_t)g.batch * g.n_q_heads * L.parts_pitch * kPartFloats * 4);
  L.total = off;
  return L;
}

}  // namespace adakv

// ---- static scratch of adakv_decode_fused_noalloc ---------------------------
// The workspace of the allocation-free entry point: a file-scope device array,
// one copy per GPU, held until the process ends.  Host code never passes the
// array's name to a kernel (in host code it is a host-side stand-in); it uses
// the per-device address from hipGetSymbolAddress, looked up once per device.
static __device__ __align__(256) unsigned char scratch[ADAKV_NOALLOC_SCRATCH_BYTES];

namespace adakv {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

__global__ void zero_words_kernel(uint32_t* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// The device address of `scratch` on the stream's device.  The first call on a
// device looks it up (that device current) and clears the hand-off counters at
// its front with a fill kernel on the stream (every call leaves them zero).
int static_scratch(hipStream_t s, void** out) {
  int dev = -1;
  if (s == nullptr || hipStreamGetDevice(s, &dev) != hipSuccess) {
    if (hipGetDevice(&dev) != hipSuccess) return ADAKV_ERR_LAUNCH;
  }
  if (dev < 0 || dev >= kMaxDevices) return ADAKV_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return ADAKV_ERR_LAUNCH;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return ADAKV_ERR_LAUNCH;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess && p != nullptr) {
      hipLaunchKernelGGL(zero_words_kernel, dim3(16), dim3(256), 0, s, reinterpret_cast<uint32_t*>(p),
                         (int)(kCounterBytes / 4));
    }
    const hipError_t e2 = hipGetLastError();
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || p == nullptr || e2 != hipSuccess) return ADAKV_ERR_LAUNCH;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ADAKV_OK;
}

int decode_fused_impl(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_kv_t* kv,
                       const adakv_centroid_t* c, const int32_t* seq_lens,
                       const adakv_budget_t* p, const adakv_selection_t* sel, int32_t append_new,
                       float sm_scale, const adakv_output_t* out, void* ws, size_t ws_bytes,
                       void* stream, bool static_ws) {
  int st;
  if ((st = check_geometry(g)) || (st = check_q(q)) || (st = check_kv(g, kv, true)) ||
      (st = check_centroid(g, c)) || (st = check_budget(p)) || (st = check_out(out)))
    return st;
  if (append_new < 0 || append_new > g->max_seq_len) return ADAKV_ERR_VALUE;
  if (!isfinite(sm_scale)) return ADAKV_ERR_VALUE;
  const int T = table_width_of(g, p);
  int Tl = T;
  if (sel) {
    if (!sel->block_table || !sel->sel_lens) return ADAKV_ERR_NULL;
    if (sel->table_width < T) return ADAKV_ERR_SHAPE;
    Tl = sel->table_width;
  }
  if (static_ws) {
    // every argument is checked before the scratch is looked up (the first
    // call on a device launches its counter fill)
    if (append_new > 0 && !centroid_pair_ok(kv->dtype, c)) return ADAKV_ERR_DTYPE;
    if (workspace_layout(*g, Tl).total > ADAKV_NOALLOC_SCRATCH_BYTES) return ADAKV_ERR_SCRATCH;
    if ((st = static_scratch((hipStream_t)stream, &ws))) return st;
  } else if ((st = check_ws(g, Tl, ws, ws_bytes))) {
    return st;
  }
  char* w = reinterpret_cast<char*>(ws);
  const WorkspaceLayout L = workspace_layout(*g, Tl);
  int32_t* table = sel ? sel->block_table : reinterpret_cast<int32_t*>(w + L.table);
  int32_t* lens = sel ? sel->sel_lens : reinterpret_cast<int32_t*>(w + L.lens);
  const hipStream_t s = (hipStream_t)stream;
  if (append_new > 0 && !centroid_pair_ok(kv->dtype, c)) return ADAKV_ERR_DTYPE;
  // bf16 / fp16 K/V (and q of the same type, 16-byte aligned rows) on a shape the fused kernel
  // serves: scores, then one kernel for the budget, the selection and the
  // decode of every head (the nucleus policy adds its weight kernel in between)
  if (kv->dtype != ADAKV_F32 && q->dtype == kv->dtype && aligned16(q->data) && q->stride_b % 8 == 0 &&
      q->stride_h % 8 == 0 &&
      select_decode_supported(g->head_dim, rows_bound(g), T, g->n_q_heads, L.sp, L.parts_pitch) &&
      select_decode_lds(g->head_dim, g->n_q_heads, rows_bound(g), p->avg_budget) <= max_lds_per_block()) {
    FusedArgs fa{};
    if ((st = run_scores(g, q, c, kv, append_new, seq_lens, p, table, Tl, w, s, &fa.s))) return st;
    if (p->policy == ADAKV_POLICY_NUCLEUS && launch_nucleus(fa.s, rows_bound(g), s) != hipSuccess)
      return ADAKV_ERR_LAUNCH;
    fa.d = decode_args(g, q, kv, seq_lens, sm_scale, out);
    fa.d.sel_lens_out = lens;
    return status_of(launch_select_decode(fa, kv->dtype, g->head_dim, rows_bound(g), s));
  }
  if ((st = run_plan(g, q, c, kv, append_new, seq_lens, p, table, Tl, nullptr, w, s))) return st;
  // the selection kernel lists distinct valid blocks: no union needed per head
  return run_decode(g, q, kv, seq_lens, table, Tl, nullptr, p, lens, sm_scale, out, w, Tl, true, s);
}

}  // namespace
}  // namespace adakv

using namespace adakv;

extern "C" {

const char* adakv_status_string(int status) {
  switch (status) {
    case ADAKV_OK: return "ok";
    case ADAKV_ERR_NULL: return "a required pointer is NULL";
    case ADAKV_ERR_SHAPE: return "inconsistent shapes";
    case ADAKV_ERR_DTYPE: return "unsupported or mismatched dtype";
    case ADAKV_ERR_UNSUPPORTED: return "configuration not supported by the built kernels";
    case ADAKV_ERR_WORKSPACE: return "workspace too small or misaligned";
    case ADAKV_ERR_LAUNCH: return "HIP kernel launch failed";
    case ADAKV_ERR_VALUE: return "invalid parameter value or alignment";
    case ADAKV_ERR_SCRATCH: return "the step needs more scratch than ADAKV_NOALLOC_SCRATCH_BYTES";
    default: return "unknown status";
  }
}

int adakv_abi_version(void) { return ADAKV_ABI_VERSION; }

int32_t adakv_table_width(const adakv_geometry_t* g, const adakv_budget_t* p) {
  if (check_geometry(g) != ADAKV_OK || check_budget(p) != ADAKV_OK) return -1;
  return table_width_of(g, p);
}

size_t adakv_workspace_bytes(const adakv_geometry_t* g, int32_t table_width) {
  if (check_geometry(g) != ADAKV_OK || table_width < 1) return 0;
  return workspace_layout(*g, table_width).total;
}

int adakv_centroid_build(const adakv_geometry_t* g, const adakv_kv_t* kv, const int32_t* seq_lens,
                         const adakv_centroid_t* c, void* stream) {
  int st;
  if ((st = check_geometry(g)) || (st = check_kv(g, kv, false)) || (st = check_centroid(g, c))) return st;
  if (!centroid_pair_ok(kv->dtype, c)) return ADAKV_ERR_DTYPE;
  CentroidArgs a = centroid_args(g, kv, seq_lens, c, 0);
  return status_of(run_summary(a, kv->dtype, c, g->head_dim, (hipStream_t)stream));
}

int adakv_centroid_append(const adakv_geometry_t* g, const adakv_kv_t* kv, const int32_t* seq_lens,
                          int32_t n_new, const adakv_centroid_t* c, void* stream) {
  int st;
  if ((st = check_geometry(g)) || (st = check_kv(g, kv, false)) || (st = check_centroid(g, c))) return st;
  if (n_new < 1 || n_new > g->max_seq_len) return ADAKV_ERR_VALUE;
  if (!centroid_pair_ok(kv->dtype, c)) return ADAKV_ERR_DTYPE;
  CentroidArgs a = centroid_args(g, kv, seq_lens, c, n_new);
  return status_of(run_summary(a, kv->dtype, c, g->head_dim, (hipStream_t)stream));
}

int adakv_block_scores(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_centroid_t* c,
                       const int32_t* seq_lens, float* scores, int32_t pitch, void* stream) {
  int st;
  if ((st = check_geometry(g)) || (st = check_q(q)) || (st = check_centroid(g, c))) return st;
  if (!scores) return ADAKV_ERR_NULL;
  if (pitch < g->max_blocks) return ADAKV_ERR_SHAPE;
  ScoreArgs sa = score_args(g, q, c, seq_lens, scores, pitch);
  return status_of(launch_score(sa, c->dtype, row_len(g, c), (hipStream_t)stream));
}

int adakv_plan(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_centroid_t* c,
               const int32_t* seq_lens, const adakv_budget_t* p, const adakv_selection_t* sel,
               void* ws, size_t ws_bytes, void* stream) {
  int st;
  if ((st = check_geometry(g)) || (st = check_q(q)) || (st = check_centroid(g, c)) ||
      (st = check_budget(p)))
    return st;
  if (!sel || !sel->block_table || !sel->sel_lens) return ADAKV_ERR_NULL;
  const int T = table_width_of(g, p);
  if (sel->table_width < T) return ADAKV_ERR_SHAPE;
  if ((st = check_ws(g, sel->table_width, ws, ws_bytes))) return st;
  return run_plan(g, q, c, nullptr, 0, seq_lens, p, sel->block_table, sel->table_width,
                  sel->sel_lens, reinterpret_cast<char*>(ws), (hipStream_t)stream);
}

int adakv_sparse_decode(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_kv_t* kv,
                        const int32_t* seq_lens, const adakv_selection_t* sel, float sm_scale,
                        const adakv_output_t* out, void* ws, size_t ws_bytes, void* stream) {
  int st;
  if ((st = check_geometry(g)) || (st = check_q(q)) || (st = check_kv(g, kv, true)) ||
      (st = check_out(out)))
    return st;
  if (!sel || !sel->block_table || !sel->sel_lens) return ADAKV_ERR_NULL;
  if (sel->table_width < 1) return ADAKV_ERR_SHAPE;
  if (!isfinite(sm_scale)) return ADAKV_ERR_VALUE;
  if ((st = check_ws(g, sel->table_width, ws, ws_bytes))) return st;
  return run_decode(g, q, kv, seq_lens, sel->block_table, sel->table_width, sel->sel_lens,
                    nullptr, nullptr, sm_scale, out, reinterpret_cast<char*>(ws),
                    sel->table_width, false, (hipStream_t)stream);
}

int adakv_decode_fused(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_kv_t* kv,
                       const adakv_centroid_t* c, const int32_t* seq_lens,
                       const adakv_budget_t* p, const adakv_selection_t* sel, int32_t append_new,
                       float sm_scale, const adakv_output_t* out, void* ws, size_t ws_bytes,
                       void* stream) {
  return decode_fused_impl(g, q, kv, c, seq_lens, p, sel, append_new, sm_scale, out, ws, ws_bytes, stream,
                           false);
}

int adakv_decode_fused_scan(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_kv_t* kv,
                            const adakv_centroid_t* c, const int32_t* seq_lens, const adakv_budget_t* p,
                            int32_t append_new, void* ws, size_t ws_bytes, void* stream) {
  int st;
  if ((st = check_geometry(g)) || (st = check_q(q)) || (st = check_kv(g, kv, true)) ||
      (st = check_centroid(g, c)) || (st = check_budget(p)))
    return st;
  if (append_new < 0 || append_new > g->max_seq_len) return ADAKV_ERR_VALUE;
  const int T = table_width_of(g, p);
  if ((st = check_ws(g, T, ws, ws_bytes))) return st;
  if (append_new > 0 && !centroid_pair_ok(kv->dtype, c)) return ADAKV_ERR_DTYPE;
  char* w = reinterpret_cast<char*>(ws);
  const WorkspaceLayout L = workspace_layout(*g, T);
  SelectArgs se;
  return run_scores(g, q, c, kv, append_new, seq_lens, p, reinterpret_cast<int32_t*>(w + L.table), T, w,
                    (hipStream_t)stream, &se);
}

int adakv_decode_fused_noalloc(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_kv_t* kv,
                               const adakv_centroid_t* c, const int32_t* seq_lens,
                               const adakv_budget_t* p, const adakv_selection_t* sel, int32_t append_new,
                               float sm_scale, const adakv_output_t* out, void* stream) {
  return decode_fused_impl(g, q, kv, c, seq_lens, p, sel, append_new, sm_scale, out, nullptr,
                           ADAKV_NOALLOC_SCRATCH_BYTES, stream, true);
}

int adakv_dense_decode(const adakv_geometry_t* g, const adakv_query_t* q, const adakv_kv_t* kv,
                       const int32_t* seq_lens, float sm_scale, const adakv_output_t* out, void* ws,
                       size_t ws_bytes, void* stream) {
  int st;
  if ((st = check_geometry(g)) || (st = check_q(q)) || (st = check_kv(g, kv, true)) ||
      (st = check_out(out)))
    return st;
  if (!isfinite(sm_scale)) return ADAKV_ERR_VALUE;
  if ((st = check_ws(g, 1, ws, ws_bytes))) return st;
  return run_decode(g, q, kv, seq_lens, nullptr, 0, nullptr, nullptr, nullptr, sm_scale, out,
                    reinterpret_cast<char*>(ws), 1, false, (hipStream_t)stream);
}

}  // extern "C"
