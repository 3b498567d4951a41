// Plan kernels: the centroid block scores, top-k block selection and the
// per-head budget (adakv/attention.py:149-247 with the numerics of the NumPy
// oracle: adakv/estimator.py:62-74, adakv/budget.py:28-86,
// adakv/selector.py:18-60).
//
// score_kernel   (score.hpp) instantiated here for centroid summaries; the
//                minmax instantiation lives in minmax.hip.
// select_kernel  one workgroup per (sequence, q-head).  Holds the head's scores
//                in registers, computes the normalised softmax entropy, picks
//                the top content blocks with a linear-bin radix select plus a
//                bitonic sort of the survivors and writes the block-table row
//                (forced blocks, then content by descending score).  No
//                inter-workgroup communication: the cross-head budget
//                normalisation (budget.py:83-84) is done by its consumer.
// budget_kernel  one workgroup per sequence: sel_lens from the weights (used
//                by the plan-only entry point; the fused decode derives the
//                counts itself).
#include <float.h>

#include <algorithm>

#include "common.hpp"
#include "internal.hpp"
#include "score.hpp"
#include "select.hpp"

namespace adakv {
namespace {

// ------------------------------------------------------------- selection ----
template <int NT, int IPT>
__global__ __launch_bounds__(NT) void select_kernel(SelectArgs a) {
  static_assert(IPT <= 64 && IPT % 4 == 0 && NT >= 256, "one mask word per thread");
  constexpr int NW = NT / kWave;
  using Mask = MaskT<IPT>;
  constexpr Mask kOne = 1;
  __shared__ SelectLds<NT> L;
  __shared__ float s_r[NW][3];

  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & (kWave - 1), w = tid / kWave;
  const int len = seq_len_of(a.seq_lens, a.uniform_len, b);
  const int nb = len > 0 ? ceil_div(len, a.bs) : 0;
  const Bounds bb = budget_bounds(nb, a.cfg);
  const int c_lo = bb.sink, c_hi = nb - bb.local;
  const int n_content = max(c_hi - c_lo, 0);
  const int KC = min(max(bb.kcap - bb.n_forced, 0), n_content);
  const bool adaptive = a.cfg.policy == ADAKV_POLICY_ADAPTIVE && nb > 1;
  select_init(L);

  // ---- forced prefix and padding of the block-table row ----
  int32_t* trow = a.table + ((int64_t)b * a.Hq + h) * a.T;
  const int local_lo = max(bb.sink, nb - bb.local);
  for (int j = tid; j < bb.n_forced; j += NT) trow[j] = j < bb.sink ? j : local_lo + (j - bb.sink);
  for (int j = bb.n_forced + KC + tid; j < a.T; j += NT) trow[j] = -1;

  // ---- the head's scores: thread t owns blocks [t*IPT, (t+1)*IPT) ----
  const float* srow = a.scores + ((int64_t)b * a.Hq + h) * a.sp;
  const int base = tid * IPT;
  float v[IPT];
  load_scores(srow, nb, v);

  // ---- softmax partials: the score kernel's records plus the rows it left out ----
  // (blocks recomputed by the decode-time append are scored on their own and
  // belong to no record; each counts as a one-row part here).  Sub-chunk
  // content maxima go to L.maxv: 4 per record, then one per left-out row.
  const int first_app = a.n_new > 0 ? max(len - a.n_new, 0) / a.bs : nb;
  const int rows_in_chunks = min(nb, first_app);
  const int n_ck = ceil_div(rows_in_chunks, a.chunk_rows);
  const float tf = (float)fmax(a.cfg.temperature, 1e-6);
  const bool unit = tf == 1.f;
  SoftPart pt = soft_empty();
  bool has = false;
  for (int c = tid; c < n_ck; c += NT) {
    const float4 r0 = *reinterpret_cast<const float4*>(a.parts + part_offset(b, a.Hq, h, a.parts_pitch, c, 0));
    const float4 r1 = *reinterpret_cast<const float4*>(a.parts + part_offset(b, a.Hq, h, a.parts_pitch, c, 1));
    pt = soft_merge(pt, SoftPart{r0.x, r0.y, r0.z});
    const float mx[4] = {r1.x, r1.y, r1.z, r1.w};   // the sub-chunks' largest content scores
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * c + i < NT) L.maxv[4 * c + i] = mx[i];
    has = true;
  }
  Mask content = 0;
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int idx = base + i;
    const bool is_content = idx >= c_lo && idx < c_hi;
    if (is_content) content |= kOne << i;
    if (idx >= rows_in_chunks && idx < nb) {
      const float z = unit ? v[i] : __fdiv_rn(v[i], tf);
      pt = soft_merge(pt, SoftPart{z, 1.f, 0.f});
      const int t = 4 * n_ck + idx - rows_in_chunks;
      if (t < NT) L.maxv[t] = is_content ? sanitize(v[i]) : -INFINITY;
      has = true;
    }
  }
  const int n_max = min(4 * n_ck + (nb - rows_in_chunks), NT);
  if (__ballot(has) != 0) pt = soft_group_merge<kWave>(pt);   // waves without partials skip the merge
  if (lane == 0) { s_r[w][0] = pt.m; s_r[w][1] = pt.S; s_r[w][2] = pt.T; }
  __syncthreads();

  if (KC > 0) {
    const int nf = bb.n_forced;
    if (w == 0) select_threshold(L, KC, n_max);
    __syncthreads();
    select_content<NT, IPT>(L, [&](int i) { return v[i]; }, content, base, KC, INFINITY,
                            [&](int r, int blk) { trow[nf + r] = blk; }, [](int) {});
  }
  // the head's entropy weight from the waves' partials (adakv/budget.py:33-37)
  if (adaptive && w == NW - 1) {
    SoftPart p = lane < NW ? SoftPart{s_r[lane][0], s_r[lane][1], s_r[lane][2]} : soft_empty();
    p = soft_group_merge<kWave>(p);
    if (lane == 0) a.wbuf[(int64_t)b * a.Hq + h] = entropy_weight(p, log((double)max(nb, 2)));
  }
}

// ------------------------------------------------------- nucleus weights ----
// One workgroup per (sequence, q-head): the nucleus weight of the head's whole
// score row (adakv/budget.py:38-41) into wbuf, for the consumers of the
// weights (budget kernel, decode, fused selection).
template <int NT, int IPT>
__global__ __launch_bounds__(NT) void nucleus_kernel(SelectArgs a) {
  __shared__ NucleusLds N;
  const int h = blockIdx.x, b = blockIdx.y;
  const int len = seq_len_of(a.seq_lens, a.uniform_len, b);
  const int nb = len > 0 ? ceil_div(len, a.bs) : 0;
  if (nb <= 1) return;                     // no weight is read: one block takes the k_min rule
  float v[IPT];
  load_scores(a.scores + ((int64_t)b * a.Hq + h) * a.sp, nb, v);
  const float tf = (float)fmax(a.cfg.temperature, 1e-6);
  const double wn = nucleus_weight<NT, IPT>(N, v, nb, tf, a.cfg.nucleus_p);
  if (threadIdx.x == 0) a.wbuf[(int64_t)b * a.Hq + h] = wn;
}

// -------------------------------------------------------------- budgets ----
__global__ __launch_bounds__(kNT) void budget_kernel(BudgetArgs a) {
  extern __shared__ double s_w[];
  __shared__ double s_sum;
  const int b = blockIdx.x;
  const int len = seq_len_of(a.seq_lens, a.uniform_len, b);
  const int nb = len > 0 ? ceil_div(len, a.bs) : 0;
  const Bounds bb = budget_bounds(nb, a.cfg);
  const bool adaptive = a.cfg.policy != ADAKV_POLICY_FIXED && nb > 1;   // weights in wbuf
  if (adaptive) {
    for (int h = threadIdx.x; h < a.Hq; h += kNT) s_w[h] = a.wbuf[(int64_t)b * a.Hq + h];
    __syncthreads();
    if (threadIdx.x == 0) s_sum = numpy_pairwise_sum<6>(s_w, a.Hq);
    __syncthreads();
  }
  for (int h = threadIdx.x; h < a.Hq; h += kNT)
    a.sel_lens[(int64_t)b * a.Hq + h] =
        head_count(bb, a.cfg.policy, adaptive ? s_w[h] : 0.0, adaptive ? s_sum : 0.0, a.Hq);
}

}  // namespace

int score_chunks_max(int max_blocks, int D) {
  // the smallest chunk is that of fp32 centroids: 16 rows per wave-wide load set
  const int cb = std::max(1, (kNT / kWave) * (kWave / std::max(1, D / 4)) * 4);
  return (max_blocks + cb - 1) / cb;
}

hipError_t launch_score(ScoreArgs& a, int cdt, int D, hipStream_t s) {
  if (a.minmax) return launch_score_minmax(a, cdt, D, s);
  return launch_score_kind<false>(a, cdt, D, s);
}

hipError_t launch_select(const SelectArgs& a, int max_blocks, hipStream_t s) {
  dim3 grid(a.Hq, a.B);
  if (max_blocks <= 256 * 4) hipLaunchKernelGGL((select_kernel<256, 4>), grid, dim3(256), 0, s, a);
  else if (max_blocks <= 1024 * 4) hipLaunchKernelGGL((select_kernel<1024, 4>), grid, dim3(1024), 0, s, a);
  else if (max_blocks <= 1024 * 8) hipLaunchKernelGGL((select_kernel<1024, 8>), grid, dim3(1024), 0, s, a);
  else if (max_blocks <= 512 * 32) hipLaunchKernelGGL((select_kernel<512, 32>), grid, dim3(512), 0, s, a);
  else if (max_blocks <= 512 * 64) hipLaunchKernelGGL((select_kernel<512, 64>), grid, dim3(512), 0, s, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_nucleus(const SelectArgs& a, int max_blocks, hipStream_t s) {
  dim3 grid(a.Hq, a.B);
  if (max_blocks <= 256 * 4) hipLaunchKernelGGL((nucleus_kernel<256, 4>), grid, dim3(256), 0, s, a);
  else if (max_blocks <= 1024 * 4) hipLaunchKernelGGL((nucleus_kernel<1024, 4>), grid, dim3(1024), 0, s, a);
  else if (max_blocks <= 1024 * 8) hipLaunchKernelGGL((nucleus_kernel<1024, 8>), grid, dim3(1024), 0, s, a);
  else if (max_blocks <= 1024 * 16) hipLaunchKernelGGL((nucleus_kernel<1024, 16>), grid, dim3(1024), 0, s, a);
  else if (max_blocks <= 1024 * 32) hipLaunchKernelGGL((nucleus_kernel<1024, 32>), grid, dim3(1024), 0, s, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_budget(const BudgetArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(budget_kernel, dim3(a.B), dim3(kNT), (size_t)a.Hq * sizeof(double), s, a);
  return hipGetLastError();
}

}  // namespace adakv
