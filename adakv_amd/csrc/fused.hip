// Fused selection + sparse decode of one AdaKV decode step, after the score
// kernel (adakv/attention.py:202-268: budget, selection and block-sparse
// attention of every q-head in one launch).
//
// One 512-thread workgroup per (q-head, sequence) (8 waves: the matrix-core
// decode needs more registers than a 16-wave workgroup leaves a wave):
//
// 1. Loads, issued in the order they are consumed: the softmax records the
//    score kernel left for every head of the sequence (one record per score
//    workgroup), this head's scores, its query, and the K/V tiles of its
//    forced sink and local blocks (known before any selection, so their HBM
//    latency hides under the selection).
// 2. Entropy weights of all the sequence's heads (adakv/budget.py:33-37): a
//    16-lane row merges one head's records.  Every workgroup of the sequence
//    evaluates the same weights in the same order, so each derives the same
//    sum of weights in NumPy's pairwise order and its own head's count
//    (adakv/budget.py:80-86) without any inter-workgroup hand-off.
// 3. The top k - n_forced content blocks of this head (select.hpp), written
//    to the block-table row and an LDS list.
// 4. Flash-decode over the head's k blocks on the matrix cores (attend.hpp):
//    16-token tiles spread over the decode waves, tile i on wave i % DW; the
//    waves' (m, l, acc) are merged through LDS.  The block count per head is
//    small (k_max), so one workgroup per head needs no split-K.
#include <float.h>

#include <algorithm>

#include "attend.hpp"
#include "common.hpp"
#include "internal.hpp"
#include "select.hpp"

namespace adakv {
namespace {

constexpr int kFusedThreads = 512;
constexpr int kLanesPerHead = 16;            // lanes merging one head's records
constexpr int kRecsPerLane = 4;              // records a lane loads up front

// Decode waves: all 8.
template <int D>
constexpr int fused_decode_waves() { return kFusedThreads / kWave; }

template <int D, int IPT>
union FusedBig {
  struct {
    SelectLds<kFusedThreads> sel;                                  // the selection
    alignas(16) float sc[kFusedThreads * IPT];                     // and this head's scores
  } x;
  uint32_t vt[fused_decode_waves<D>() * TileShape<D>::VT_WORDS];   // then the V tiles
};

template <int D, int IPT>
constexpr size_t fused_static_lds() {
  return sizeof(FusedBig<D, IPT>) + kSortCap * sizeof(int) + (2 + D) * fused_decode_waves<D>() * sizeof(float);
}

// Scores per thread for a max_blocks (0: not served).
inline int fused_ipt(int max_blocks) {
  return max_blocks <= kFusedThreads * 4 ? 4 : max_blocks <= kFusedThreads * 8 ? 8
       : max_blocks <= kFusedThreads * 16 ? 16 : 0;
}

// x / d, with s = log2(d) when d is a power of two (else -1).
__device__ __forceinline__ int div_p2(int x, int d, int s) { return s >= 0 ? (x >> s) : x / d; }

__device__ __forceinline__ double readlane_d(double x, int l) {
  const long long u = __double_as_longlong(x);
  const int lo = __builtin_amdgcn_readlane((int)(u & 0xffffffffll), l);
  const int hi = __builtin_amdgcn_readlane((int)(u >> 32), l);
  return __longlong_as_double(((long long)hi << 32) | (uint32_t)lo);
}

// NumPy's pairwise sum of a[0, n) for n <= 128 (the single-block case of
// numpy_pairwise_sum), by one wave: lane j < 8 is NumPy's accumulator j
// (a[j] + a[j + 8] + ... in order), then the fixed combination and the tail.
// Every lane receives the sum.
__device__ __forceinline__ double wave_pairwise_sum(const double* a, int n) {
  if (n < 8) {
    double r = 0.0;
    for (int i = 0; i < n; ++i) r += a[i];
    return r;
  }
  const int lane = threadIdx.x & (kWave - 1);
  const int m8 = n - (n % 8);
  double r = 0.0;
  if (lane < 8) {
    r = a[lane];
    for (int i = 8 + lane; i < m8; i += 8) r += a[i];
  }
  double x[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = readlane_d(r, j);
  double res = ((x[0] + x[1]) + (x[2] + x[3])) + ((x[4] + x[5]) + (x[6] + x[7]));
  for (int i = m8; i < n; ++i) res += a[i];
  return res;
}

template <int KVDT, int D, int IPT>
__global__ __launch_bounds__(kFusedThreads) void select_decode_kernel(FusedArgs fa) {
  constexpr int NT = kFusedThreads, NW = NT / kWave;
  constexpr int DW = fused_decode_waves<D>();
  constexpr int NT16 = TileShape<D>::NT16;
  constexpr int LPH = kLanesPerHead, HPW = kWave / LPH, RPL = kRecsPerLane;
  using Mask = MaskT<IPT>;
  constexpr Mask kOne = 1;
  __shared__ __align__(16) FusedBig<D, IPT> big;
  __shared__ int s_list[kSortCap];          // content blocks by rank
  __shared__ float s_m[DW], s_l[DW];
  __shared__ float s_acc[DW][D];            // the decode waves' accumulators for the merge
  extern __shared__ double s_w[];            // [Hq] budget weights of the sequence's heads

  const SelectArgs& a = fa.s;
  const DecodeArgs& d = fa.d;
  // XCD-aware placement: workgroups are dealt to the 8 XCDs in turn (linear id
  // mod 8), so linear id i takes position (i mod 8) * n/8 + i / 8 of the
  // (sequence, q-head) order: each XCD holds consecutive q-heads -- the heads
  // of a KV group, the sequences' records and their shared sink, local and
  // common blocks then meet in one L2.
  int h, b;
  {
    const int n = gridDim.x * gridDim.y, i = blockIdx.y * gridDim.x + blockIdx.x;
    const int pos = (n & 7) == 0 ? (i & 7) * (n >> 3) + (i >> 3) : i;
    h = pos % gridDim.x;
    b = pos / gridDim.x;
  }
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), w = tid / kWave;
  const int col = lane & 15, grp = lane >> 4;
  const int Hq = a.Hq;
  const int len = seq_len_of(a.seq_lens, a.uniform_len, b);
  const int nb = len > 0 ? div_p2(len + a.bs - 1, a.bs, a.bs_shift) : 0;
  const Bounds bb = budget_bounds(nb, a.cfg);
  const int nf = bb.n_forced;
  const int c_lo = bb.sink, c_hi = nb - bb.local;
  const int local_lo = max(bb.sink, nb - bb.local);
  const bool adaptive = a.cfg.policy == ADAKV_POLICY_ADAPTIVE && nb > 1;   // entropy weights from the records
  const bool nucleus = a.cfg.policy == ADAKV_POLICY_NUCLEUS && nb > 1;     // weights from the nucleus kernel
  int32_t* trow = a.table + ((int64_t)b * Hq + h) * a.T;
  const int64_t oo = (int64_t)b * d.osb + (int64_t)h * d.osh;
  if (nb == 0) {                             // empty sequence: no block, 0/0 as the reference kernel
    for (int j = tid; j < a.T; j += NT) trow[j] = -1;
    if (tid == 0 && d.sel_lens_out) d.sel_lens_out[(int64_t)b * Hq + h] = 0;
    for (int i = tid; i < D; i += NT) store_elt(d.out, d.odt, oo + i, __builtin_nanf(""));
    return;
  }
  select_init(big.x.sel);

  // ---- 1. loads ----
  // Every load here is unconditional, its index clamped in bounds (values not
  // wanted are discarded where they are consumed): a load under a branch makes
  // the compiler wait for it where the branches join.
  //
  // (a) the records of each 16-lane row's head (RPL per lane, the rest later
  //     if a head has more): all heads when the budget is adaptive (four per
  //     wave and pass), else only this head (for its content maxima), and the
  //     score of one row no record covers (the decode-time append).
  const int first_app = a.n_new > 0 ? div_p2(max(len - a.n_new, 0), a.bs, a.bs_shift) : nb;
  const int rows_in_chunks = min(nb, first_app);
  const int n_ck = (rows_in_chunks + a.chunk_rows - 1) >> a.chunk_shift;   // records
  const int n_extra = nb - rows_in_chunks;                                 // rows no record covers
  const float tf = (float)fmax(a.cfg.temperature, 1e-6);
  const int hl = lane % LPH;
  auto head_of = [&](int p) -> int {
    if (adaptive) return (p * NW + w) * HPW + lane / LPH;
    return (w == 0 && lane < LPH) ? h : -1;
  };
  // per-lane offsets stay 32-bit (the host bounds Hq * pitch)
  const float* parts_b = a.parts + (int64_t)b * Hq * a.parts_pitch * kPartFloats;
  const float* scores_b = a.scores + (int64_t)b * Hq * a.sp;
  auto rec = [&](int hh, int j) {
    return reinterpret_cast<const float4*>(parts_b + (hh * a.parts_pitch + min(j, max(n_ck - 1, 0))) * kPartFloats);
  };
  auto extra = [&](int hh, int e) { return scores_b + hh * a.sp + min(rows_in_chunks + e, nb - 1); };
  const int hh0 = head_of(0);
  const int hs0 = (hh0 >= 0 && hh0 < Hq) ? hh0 : h;
  float4 R0[RPL], R1[RPL];
#pragma unroll
  for (int u = 0; u < RPL; ++u) {
    R0[u] = rec(hs0, hl + LPH * u)[0];
    R1[u] = rec(hs0, hl + LPH * u)[1];
  }
  const float X0 = *extra(hs0, hl);
  __builtin_amdgcn_sched_barrier(0);
  // (b) this head's scores: thread t owns blocks [t*IPT, (t+1)*IPT); rows
  //     past nb (stale) are never content
  float v[IPT];
  {
    const float* srow = scores_b + h * a.sp;
#pragma unroll
    for (int i = 0; i < IPT; i += 4) {
      const float4 f = *reinterpret_cast<const float4*>(srow + min(tid * IPT + i, a.sp - 4));
      v[i] = f.x; v[i + 1] = f.y; v[i + 2] = f.z; v[i + 3] = f.w;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // (c) the query (same 16-bit type as K, 16-byte aligned rows), as the B
  //     operand of S^T: lane (col, grp) holds q[D/4*grp + 8*s .. +7] in
  //     every column (columns other than 0 are masked out of the softmax)
  uint4 qf[D / 32];
  {
    const uint16_t* qp = reinterpret_cast<const uint16_t*>(d.q) + (int64_t)b * d.qsb + (int64_t)h * d.qsh + (D / 4) * grp;
#pragma unroll
    for (int s2 = 0; s2 < D / 32; ++s2) qf[s2] = *reinterpret_cast<const uint4*>(qp + 8 * s2);
  }
  __builtin_amdgcn_sched_barrier(0);
  // (d) the decode's addressing: item i (16-token sub-tile i % n_sub of list
  //     entry i / n_sub) belongs to decode wave i % DW; the first n_forced
  //     entries are the sink blocks then the local blocks, as in the table row
  const int n_sub = (a.bs + 15) >> 4;
  const int nf_items = nf * n_sub;
  const int64_t head_off = ((int64_t)b * d.sb + (int64_t)(h / d.G) * d.sh + (D / 4) * grp) * 2;
  const char* kbase = reinterpret_cast<const char*>(d.k) + head_off;
  const char* vbase = reinterpret_cast<const char*>(d.v) + head_off;
  const int64_t row_bytes = d.ss * 2;
  auto item = [&](int j, int& t0, int& t_hi) {
    const int e = n_sub == 1 ? j : j / n_sub, sub = j - e * n_sub;
    const int blk = e < bb.sink ? e : (e < nf ? local_lo + (e - bb.sink) : s_list[e - nf]);
    t0 = blk * a.bs + sub * 16;
    t_hi = min(min(blk * a.bs + a.bs, len), t0 + 16);
  };
  // the forced tiles of the prefetch path (below): known before any selection
  const int wu = __builtin_amdgcn_readfirstlane(w);   // the wave index, provably uniform
  const bool pf_shape = n_sub == 1 && nf <= DW;
  const bool p_load = pf_shape && wu < nf;
  TileBuf<D> P;
  int p0 = 0, p1 = 1;
  if (p_load) {
    item(wu, p0, p1);
    tile_load<D>(kbase, vbase, row_bytes, p0, p1, P);
  }
  __builtin_amdgcn_sched_barrier(0);
  const double lognb = log((double)max(nb, 2));   // while the loads are in flight

  // ---- 2. entropy weights and this head's content maxima ----
  // Maxima of record j at 4j .. 4j+3, of row e no record covers at 4*n_ck + e.
  // one head per 16-lane row: merge its records (and rows no record covers)
  auto merge_head = [&](int hh, const float4 (&Q0)[RPL], const float4 (&Q1)[RPL], float X) {
    const bool on = hh >= 0 && hh < Hq;
    SoftPart pt = soft_empty();
    if (on) {
      const bool own = hh == h;
      auto take_rec = [&](int j, const float4& q0, const float4& q1) {
        pt = soft_merge(pt, SoftPart{q0.x, q0.y, q0.z});
        if (own) {
          const float mx[4] = {q0.w, q1.x, q1.y, q1.z};
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (4 * j + i < NT) big.x.sel.maxv[4 * j + i] = mx[i];
        }
      };
      auto take_row = [&](int e, float x) {
        pt = soft_merge(pt, SoftPart{tf == 1.f ? x : __fdiv_rn(x, tf), 1.f, 0.f});
        const int r = rows_in_chunks + e, t = 4 * n_ck + e;
        if (own && t < NT) big.x.sel.maxv[t] = (r >= c_lo && r < c_hi) ? sanitize(x) : -INFINITY;
      };
#pragma unroll
      for (int u = 0; u < RPL; ++u)
        if (hl + LPH * u < n_ck) take_rec(hl + LPH * u, Q0[u], Q1[u]);
      for (int j = hl + LPH * RPL; j < n_ck; j += LPH) take_rec(j, rec(hh, j)[0], rec(hh, j)[1]);   // long heads
      if (hl < n_extra) take_row(hl, X);
      for (int e = hl + LPH; e < n_extra; e += LPH) take_row(e, *extra(hh, e));
    }
    pt = soft_group_merge<LPH>(pt);
    if (adaptive && on && hl == 0) s_w[hh] = entropy_weight(pt, lognb);
  };
  // the first pass consumes the records loaded up front, in place
  merge_head(hh0, R0, R1, X0);
  if (nucleus)                               // written by the nucleus kernel before this launch
    for (int hh = tid; hh < Hq; hh += NT) s_w[hh] = a.wbuf[(int64_t)b * Hq + hh];
  const int passes = adaptive ? ceil_div(Hq, HPW * NW) : 1;
  for (int p = 1; p < passes; ++p) {         // more than 32 heads
    const int hh = head_of(p);
    const int hs = (hh >= 0 && hh < Hq) ? hh : h;
    float4 Q0[RPL], Q1[RPL];
#pragma unroll
    for (int u = 0; u < RPL; ++u) { Q0[u] = rec(hs, hl + LPH * u)[0]; Q1[u] = rec(hs, hl + LPH * u)[1]; }
    merge_head(hh, Q0, Q1, *extra(hs, hl));
  }
  // this head's scores to LDS (the selection reads them there, so they hold
  // no registers while the tiles are prefetched), this thread's content bits
  // and its largest sanitised content score
  const int base = tid * IPT;
  Mask content = 0;
  float vmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const bool is_c = base + i >= c_lo && base + i < c_hi;
    if (is_c) content |= kOne << i;
    vmax = fmaxf(vmax, is_c ? sanitize(v[i]) : -INFINITY);
  }
#pragma unroll
  for (int i = 0; i < IPT; i += 4)
    *reinterpret_cast<float4*>(&big.x.sc[base + i]) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
  lds_barrier();

  // ---- 3. the head's count and selection ----
  // every wave evaluates the sum of weights in NumPy's order
  const bool weighted = adaptive || nucleus;
  const double wsum = !weighted ? 0.0 : Hq <= 128 ? wave_pairwise_sum(s_w, Hq) : numpy_pairwise_sum<6>(s_w, Hq);
  const int k = min(head_count(bb, a.cfg.policy, weighted ? s_w[h] : 0.0, wsum, Hq), a.T);
  if (tid == 0) {
    if (d.sel_lens_out) d.sel_lens_out[(int64_t)b * Hq + h] = k;
    if (adaptive) a.wbuf[(int64_t)b * Hq + h] = s_w[h];
  }
  const int KC = max(k - nf, 0);
  for (int j = tid; j < nf; j += NT) trow[j] = j < bb.sink ? j : local_lo + (j - bb.sink);
  for (int j = k + tid; j < a.T; j += NT) trow[j] = -1;
  // Prefetch: with one tile per block, the forced blocks on their own waves
  // and at most DW candidates, wave w holds forced block w (w < nf, loaded in
  // the prologue) and loads candidate (w - nf) mod DW as soon as the
  // candidates are known, before they are ranked; after the rank it computes
  // the candidate if its rank is < KC (the decode does not depend on the
  // order of the blocks).  Only the waves that own a tile issue loads.
  bool prefetched = false;
  TileBuf<D> C;
  int c0 = 0, c1 = 1, cand = -1;
  if (KC > 0) {
    if (w == 0) select_threshold(big.x.sel, KC, min(4 * n_ck + n_extra, NT));
    lds_barrier();
    select_content<NT, IPT>(
        big.x.sel, [&](int i) { return big.x.sc[base + i]; }, content, base, KC, vmax,
        [&](int r, int blk) {
          s_list[r] = blk;
          trow[nf + r] = blk;
        },
        [&](int n_cand) {
          prefetched = pf_shape && n_cand <= DW;
          const int c = (wu - nf % DW + DW) % DW;
          if (prefetched && wu < DW && c < n_cand) {
            const int blk = key_index(big.x.sel.keys[c]);
            c0 = blk * a.bs;
            c1 = min(c0 + a.bs, len);
            tile_load<D>(kbase, vbase, row_bytes, c0, c1, C);
            cand = c;
          }
        });
  }
  const bool c_take = cand >= 0 && big.x.sel.rank[cand] < KC;   // read before the LDS is reused
  lds_barrier();                           // s_list complete; the selection's LDS becomes the V tiles

  // ---- 4. flash-decode over the k blocks ----
  TileState<D> st;
  tile_init(st);
  const int n_items = k * n_sub;
  if (w < DW) {
    uint32_t* vt = big.vt + w * TileShape<D>::VT_WORDS;
    const float scale = d.scale_log2;
    auto load = [&](int t0, int t_hi, TileBuf<D>& r) { tile_load<D>(kbase, vbase, row_bytes, t0, t_hi, r); };
    auto compute = [&](int t0, int t_hi, const TileBuf<D>& r) {
      tile_update<KVDT, D>(st, r, qf, vt, t0, t_hi, col == 0, scale);
    };
    const int mine = w < n_items ? (n_items - w + DW - 1) / DW : 0;   // items of this wave
    if (prefetched) {
      // forced tile (item w) and the wave's candidate, both loaded earlier
      __builtin_amdgcn_sched_barrier(0);
      if (p_load) compute(p0, p1, P);
      if (c_take) compute(c0, c1, C);
    } else if (mine > 0) {
      // items loaded now, at most two in flight, each load issued for an
      // item the wave computes
      TileBuf<D> A, B;
      int a0, a1, b0, b1;
      item(w, a0, a1);
      load(a0, a1, A);
      if (mine == 1) {
        __builtin_amdgcn_sched_barrier(0);
        compute(a0, a1, A);
      } else {
        item(w + DW, b0, b1);
        load(b0, b1, B);
        if (mine == 2) {
          __builtin_amdgcn_sched_barrier(0);
          compute(a0, a1, A);
          compute(b0, b1, B);
        } else {
          // A holds item j, B item j + DW
          int j = w;
          for (;;) {
            __builtin_amdgcn_sched_barrier(0);
            compute(a0, a1, A);
            const bool more = j + 2 * DW < n_items;
            if (more) {
              item(j + 2 * DW, a0, a1);
              load(a0, a1, A);
            }
            __builtin_amdgcn_sched_barrier(0);
            compute(b0, b1, B);
            if (!more) break;
            j += 2 * DW;
            if (j + DW >= n_items) {
              __builtin_amdgcn_sched_barrier(0);
              compute(a0, a1, A);
              break;
            }
            item(j + DW, b0, b1);
            load(b0, b1, B);
          }
        }
      }
    }
  }
  tile_finish(st);
  if (w < DW && lane == 0) {
    s_m[w] = st.m_h;
    s_l[w] = st.l_h;
  }
  if (w < DW && grp == 0) {
#pragma unroll
    for (int n = 0; n < NT16; ++n) s_acc[w][n * 16 + col] = st.acc[n][0];   // O[head 0][16n + col]
  }
  lds_barrier();
  for (int i = tid; i < D; i += NT) {
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < DW; ++ww) M = fmaxf(M, s_m[ww]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int ww = 0; ww < DW; ++ww) {
        const float f = s_m[ww] == -INFINITY ? 0.f : exp2f(s_m[ww] - M);
        L += s_l[ww] * f;
        O += s_acc[ww][i] * f;
      }
    }
    store_elt(d.out, d.odt, oo + i, O / L);   // no block at all: 0/0 as the reference kernel
  }
}

template <int KVDT, int D>
hipError_t launch_fd(const FusedArgs& a, int max_blocks, hipStream_t s) {
  const dim3 grid(a.s.Hq, a.s.B);
  const size_t dyn = (size_t)a.s.Hq * sizeof(double);
  switch (fused_ipt(max_blocks)) {
    case 4: hipLaunchKernelGGL((select_decode_kernel<KVDT, D, 4>), grid, dim3(kFusedThreads), dyn, s, a); break;
    case 8: hipLaunchKernelGGL((select_decode_kernel<KVDT, D, 8>), grid, dim3(kFusedThreads), dyn, s, a); break;
    case 16: hipLaunchKernelGGL((select_decode_kernel<KVDT, D, 16>), grid, dim3(kFusedThreads), dyn, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int KVDT>
hipError_t launch_fk(const FusedArgs& a, int D, int max_blocks, hipStream_t s) {
  switch (D) {
    case 32: return launch_fd<KVDT, 32>(a, max_blocks, s);
    case 64: return launch_fd<KVDT, 64>(a, max_blocks, s);
    case 128: return launch_fd<KVDT, 128>(a, max_blocks, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

// The fused kernel serves head_dim <= 128 and up to 16 scores per thread (the
// register budget of a 512-thread workgroup); other shapes take the
// three-kernel path.
bool select_decode_supported(int D, int max_blocks, int table_width, int Hq, int sp, int parts_pitch) {
  return D <= 128 && max_blocks <= kFusedThreads * 16 && table_width <= kSortCap &&
         (int64_t)Hq * sp < (1ll << 31) && (int64_t)Hq * parts_pitch * kPartFloats < (1ll << 31);
}

template <int D>
size_t fused_lds_d(int ipt) {
  switch (ipt) {
    case 4: return fused_static_lds<D, 4>();
    case 8: return fused_static_lds<D, 8>();
    case 16: return fused_static_lds<D, 16>();
    default: return (size_t)-1;
  }
}

size_t select_decode_lds(int D, int Hq, int max_blocks) {
  const int ipt = fused_ipt(max_blocks);
  size_t st = 0;
  switch (D) {
    case 32: st = fused_lds_d<32>(ipt); break;
    case 64: st = fused_lds_d<64>(ipt); break;
    case 128: st = fused_lds_d<128>(ipt); break;
    default: return (size_t)-1;
  }
  return st == (size_t)-1 ? st : st + (size_t)Hq * sizeof(double);
}

hipError_t launch_select_decode(const FusedArgs& a, int kvdt, int D, int max_blocks, hipStream_t s) {
  switch (kvdt) {
    case ADAKV_F16: return launch_fk<ADAKV_F16>(a, D, max_blocks, s);
    case ADAKV_BF16: return launch_fk<ADAKV_BF16>(a, D, max_blocks, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace adakv
