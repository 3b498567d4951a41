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

// Decode waves: all 8.
template <int D>
constexpr int fused_decode_waves() { return kFusedThreads / kWave; }

template <int D>
union FusedBig {
  SelectLds<kFusedThreads> sel;                                    // the selection
  uint32_t vt[fused_decode_waves<D>() * TileShape<D>::VT_WORDS];   // then the V tiles
  float acc[fused_decode_waves<D>()][D];                           // then the merge
};

template <int D>
constexpr size_t fused_static_lds() {
  return sizeof(FusedBig<D>) + kSortCap * sizeof(int) + 2 * fused_decode_waves<D>() * sizeof(float);
}

template <int KVDT, int D, int IPT>
__global__ __launch_bounds__(kFusedThreads) void select_decode_kernel(FusedArgs fa) {
  constexpr int NT = kFusedThreads, NW = NT / kWave;
  constexpr int DW = fused_decode_waves<D>();
  constexpr int NT16 = TileShape<D>::NT16;
  using Mask = MaskT<IPT>;
  constexpr Mask kOne = 1;
  __shared__ __align__(16) FusedBig<D> big;
  __shared__ int s_list[kSortCap];          // content blocks by rank
  __shared__ float s_m[DW], s_l[DW];
  extern __shared__ double s_w[];            // [Hq] entropy weights of the sequence's heads

  const SelectArgs& a = fa.s;
  const DecodeArgs& d = fa.d;
  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & (kWave - 1), w = tid / kWave;
  const int col = lane & 15, grp = lane >> 4;
  const int Hq = a.Hq;
  const int len = seq_len_of(a.seq_lens, a.uniform_len, b);
  const int nb = len > 0 ? ceil_div(len, a.bs) : 0;
  const Bounds bb = budget_bounds(nb, a.cfg);
  const int nf = bb.n_forced;
  const int c_lo = bb.sink, c_hi = nb - bb.local;
  const int local_lo = max(bb.sink, nb - bb.local);
  const bool adaptive = a.cfg.policy == ADAKV_POLICY_ADAPTIVE && nb > 1;
  int32_t* trow = a.table + ((int64_t)b * Hq + h) * a.T;
  const int64_t oo = (int64_t)b * d.osb + (int64_t)h * d.osh;
  if (nb == 0) {                             // empty sequence: no block, 0/0 as the reference kernel
    for (int j = tid; j < a.T; j += NT) trow[j] = -1;
    if (tid == 0 && d.sel_lens_out) d.sel_lens_out[(int64_t)b * Hq + h] = 0;
    for (int i = tid; i < D; i += NT) store_elt(d.out, d.odt, oo + i, __builtin_nanf(""));
    return;
  }
  select_init(big.sel);

  // ---- 1. loads ----
  // (a) the first record of each 16-lane row's head: all heads when the
  //     budget is adaptive (four per wave and pass), else only this head (for
  //     its content maxima).  Records j < n_ck come from the score workgroups,
  //     j >= n_ck are the rows no record covers (the decode-time append).
  const int first_app = a.n_new > 0 ? max(len - a.n_new, 0) / a.bs : nb;
  const int rows_in_chunks = min(nb, first_app);
  const int n_ck = ceil_div(rows_in_chunks, a.chunk_rows);
  const int n_virt = n_ck + (nb - rows_in_chunks);
  const float tf = (float)fmax(a.cfg.temperature, 1e-6);
  constexpr int LPH = kLanesPerHead, HPW = kWave / LPH;
  const int hl = lane % LPH;
  auto head_of = [&](int p) -> int {
    if (adaptive) return (p * NW + w) * HPW + lane / LPH;
    return (w == 0 && lane < LPH) ? h : -1;
  };
  auto fetch = [&](int hh, int j, float4& r0, float4& r1) {
    if (j < n_ck) {
      const float4* rec = reinterpret_cast<const float4*>(
          a.parts + (((int64_t)b * Hq + hh) * a.parts_pitch + j) * kPartFloats);
      r0 = rec[0];
      r1 = rec[1];
    } else {
      r0.x = a.scores[((int64_t)b * Hq + hh) * a.sp + rows_in_chunks + (j - n_ck)];
    }
  };
  const int hh0 = head_of(0);
  const bool on0 = hh0 >= 0 && hh0 < Hq && hl < n_virt;
  float4 r0 = make_float4(0.f, 0.f, 0.f, 0.f), r1 = r0;
  if (on0) fetch(hh0, hl, r0, r1);
  __builtin_amdgcn_sched_barrier(0);
  // (b) this head's scores: thread t owns blocks [t*IPT, (t+1)*IPT)
  float v[IPT];
  load_scores(a.scores + ((int64_t)b * Hq + h) * a.sp, nb, v);
  __builtin_amdgcn_sched_barrier(0);
  // (c) the query (B operand, head in column 0)
  uint4 qf[D / 32];
  load_q_frag<KVDT, D>(d.q, d.qdt, (int64_t)b * d.qsb + (int64_t)h * d.qsh, d.qsh, 1, qf);
  __builtin_amdgcn_sched_barrier(0);
  // (d) the forced tiles: item i (16-token sub-tile i % n_sub of list entry
  //     i / n_sub) belongs to decode wave i % DW; the first n_forced entries
  //     are the sink blocks then the local blocks, as in the table row
  const int n_sub = ceil_div(a.bs, 16);
  const int nf_items = nf * n_sub;
  const int64_t head_off = ((int64_t)b * d.sb + (int64_t)(h / d.G) * d.sh + (D / 4) * grp) * 2;
  const char* kbase = reinterpret_cast<const char*>(d.k) + head_off;
  const char* vbase = reinterpret_cast<const char*>(d.v) + head_off;
  const int64_t row_bytes = d.ss * 2;
  auto item = [&](int j, int& t0, int& t_hi) {
    const int e = j / n_sub;
    const int blk = e < bb.sink ? e : (e < nf ? local_lo + (e - bb.sink) : s_list[e - nf]);
    t0 = blk * a.bs + (j % n_sub) * 16;
    t_hi = min(min(blk * a.bs + a.bs, len), t0 + 16);
  };
  const bool pre = w < DW && w < nf_items;   // uniform over the wave
  TileBuf<D> P;
  int p0 = 0, p1 = 1;
  if (pre) {
    item(w, p0, p1);
    tile_load<D>(kbase, vbase, row_bytes, p0, p1, P);
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- 2. entropy weights and this head's content maxima ----
  auto consume = [&](int hh, int j, const float4& q0, const float4& q1, SoftPart& pt) {
    SoftPart x;
    if (j < n_ck) {
      x = SoftPart{q0.x, q0.y, q0.z};
      if (hh == h) {
        const float mx[4] = {q0.w, q1.x, q1.y, q1.z};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (4 * j + i < NT) big.sel.maxv[4 * j + i] = mx[i];
      }
    } else {
      const int r = rows_in_chunks + (j - n_ck);
      x = SoftPart{tf == 1.f ? q0.x : __fdiv_rn(q0.x, tf), 1.f, 0.f};
      const int t = 4 * n_ck + (j - n_ck);
      if (hh == h && t < NT) big.sel.maxv[t] = (r >= c_lo && r < c_hi) ? sanitize(q0.x) : -INFINITY;
    }
    pt = soft_merge(pt, x);
  };
  const int passes = adaptive ? ceil_div(Hq, HPW * NW) : 1;
  for (int p = 0; p < passes; ++p) {
    const int hh = head_of(p);
    const bool on = hh >= 0 && hh < Hq;
    SoftPart pt = soft_empty();
    if (p == 0) {
      if (on0) consume(hh, hl, r0, r1, pt);
    } else if (on && hl < n_virt) {
      float4 q0, q1;
      fetch(hh, hl, q0, q1);
      consume(hh, hl, q0, q1, pt);
    }
    for (int j = hl + LPH; on && j < n_virt; j += LPH) {   // heads with more records than lanes
      float4 q0, q1;
      fetch(hh, j, q0, q1);
      consume(hh, j, q0, q1, pt);
    }
    pt = soft_group_merge<LPH>(pt);
    if (adaptive && on && hl == 0) s_w[hh] = entropy_weight(pt, nb);
  }
  __syncthreads();

  // ---- 3. the head's count and selection ----
  // every thread evaluates the sum of weights in NumPy's order (LDS broadcasts)
  const double wsum = adaptive ? numpy_pairwise_sum<6>(s_w, Hq) : 0.0;
  const int k = min(head_count(bb, a.cfg.policy, adaptive ? s_w[h] : 0.0, wsum, Hq), a.T);
  if (tid == 0) {
    if (d.sel_lens_out) d.sel_lens_out[(int64_t)b * Hq + h] = k;
    if (adaptive) a.wbuf[(int64_t)b * Hq + h] = s_w[h];
  }
  const int KC = max(k - nf, 0);
  for (int j = tid; j < nf; j += NT) trow[j] = j < bb.sink ? j : local_lo + (j - bb.sink);
  for (int j = k + tid; j < a.T; j += NT) trow[j] = -1;
  if (KC > 0) {
    const int base = tid * IPT;
    Mask content = 0;
#pragma unroll
    for (int i = 0; i < IPT; ++i)
      if (base + i >= c_lo && base + i < c_hi) content |= kOne << i;
    const int n_max = min(4 * n_ck + (nb - rows_in_chunks), NT);
    select_content<NT, IPT>(big.sel, v, content, base, KC, n_max, [&](int r, int blk) {
      s_list[r] = blk;
      trow[nf + r] = blk;
    });
  }
  __syncthreads();                           // s_list complete; the selection's LDS becomes the V tiles

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
    if (mine > 0) {
      // item w is the prefetched forced tile when `pre`; later items are
      // loaded now, at most two in flight, each load issued for an item
      // the wave computes
      TileBuf<D> A, B;
      int a0, a1, b0, b1;
      if (pre) {
        A = P; a0 = p0; a1 = p1;
      } else {
        item(w, a0, a1);
        load(a0, a1, A);
      }
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
  __syncthreads();                           // the V tiles are dead: merge through the same LDS
  if (w < DW && grp == 0) {
#pragma unroll
    for (int n = 0; n < NT16; ++n) big.acc[w][n * 16 + col] = st.acc[n][0];   // O[head 0][16n + col]
  }
  __syncthreads();
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
        O += big.acc[ww][i] * f;
      }
    }
    store_elt(d.out, d.odt, oo + i, O / L);   // no block at all: 0/0 as the reference kernel
  }
}

template <int KVDT, int D>
hipError_t launch_fd(const FusedArgs& a, int max_blocks, hipStream_t s) {
  const dim3 grid(a.s.Hq, a.s.B);
  const size_t dyn = (size_t)a.s.Hq * sizeof(double);
  if (max_blocks <= kFusedThreads * 4)
    hipLaunchKernelGGL((select_decode_kernel<KVDT, D, 4>), grid, dim3(kFusedThreads), dyn, s, a);
  else if (max_blocks <= kFusedThreads * 8)
    hipLaunchKernelGGL((select_decode_kernel<KVDT, D, 8>), grid, dim3(kFusedThreads), dyn, s, a);
  else if (max_blocks <= kFusedThreads * 16)
    hipLaunchKernelGGL((select_decode_kernel<KVDT, D, 16>), grid, dim3(kFusedThreads), dyn, s, a);
  else
    return hipErrorInvalidValue;
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
bool select_decode_supported(int D, int max_blocks, int table_width) {
  return D <= 128 && max_blocks <= kFusedThreads * 16 && table_width <= kSortCap;
}

size_t select_decode_lds(int D, int Hq) {
  size_t st = 0;
  switch (D) {
    case 32: st = fused_static_lds<32>(); break;
    case 64: st = fused_static_lds<64>(); break;
    case 128: st = fused_static_lds<128>(); break;
    default: return (size_t)-1;
  }
  return st + (size_t)Hq * sizeof(double);
}

hipError_t launch_select_decode(const FusedArgs& a, int kvdt, int D, int max_blocks, hipStream_t s) {
  switch (kvdt) {
    case ADAKV_F16: return launch_fk<ADAKV_F16>(a, D, max_blocks, s);
    case ADAKV_BF16: return launch_fk<ADAKV_BF16>(a, D, max_blocks, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace adakv
