// Eviction baselines on the GPU: H2O and SnapKV freeze a retained block set
// at prefill from the prompt's own attention, and every later decode step
// attends that set plus the current sink and local blocks (adakv/baselines.py,
// adakv/baselines_rt.py; the decode itself is the table-driven sparse decode).
//
// importance_lse_kernel    per (q-head, 64 queries per wave): the row
//                          log-sum-exp (base 2) of the causal logits
//                          q_i . k_j * scale over keys j <= i.
// importance_colsum_kernel per (q-head, 64 keys per wave): the column sums
//                          sum_i exp2(s_ij - lse_i) over the queries
//                          i >= max(j, first_query).
//     Both stream S^T = K . Q^T through the matrix cores, 16x16 tiles over
//     head_dim (v_mfma_f32_16x16x32 for bf16/fp16, v_mfma_f32_16x16x4 for
//     fp32): the wave keeps four 16-row tiles of one operand in registers and
//     streams the other operand 16 rows at a time.  Nothing is atomic: each
//     importance entry is summed by one lane in query order, then across the
//     16 lanes of its row, so a rerun gives the same bits.
// pool_kernel              SnapKV's same-length max pool over key positions.
// retain_kernel            per head: block sums of the importance over real
//                          tokens (fp64, rounded to fp32), sink + local forced,
//                          the top content blocks by the shared radix select
//                          (ties: lower block first); mask bytes and, when
//                          asked, the retained blocks as an ascending table.
// union_table_kernel       per head: the ascending table of the union of a
//                          frozen table (or a mask) with the sink and local
//                          blocks of the current block count.
#include <float.h>
#include <math.h>

#include <algorithm>

#include "adakv_amd.h"
#include "common.hpp"
#include "internal.hpp"
#include "select.hpp"

namespace adakv {
namespace {

constexpr int kEvNT = 256;          // importance kernels: 4 independent waves
constexpr int kEvRows = 64;         // resident rows per wave (4 tiles of 16)
constexpr int kRetainNT = 1024;
constexpr int kRetainIPT = 16;
constexpr int kRetainMaxBlocks = kRetainNT * kRetainIPT;
constexpr int kUnionNT = 256;
constexpr int kUnionMaxBlocks = 65536;
constexpr int kMaxTokens = 1 << 20;

typedef float float4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

struct ImpArgs {
  const char* q;               // byte pointers
  const char* k;
  int64_t qsh, qss, ksh, kss;  // strides in bytes
  int Hq, G, L, q0;
  float c2;                    // sm_scale * log2(e)
  float* lse;                  // [Hq, L - q0], base-2 log-sum-exp
  float* imp;                  // [Hq, pitch]
  int pitch;
  int nsplit, klen;            // pass 1 key split: nsplit ranges of klen keys (a multiple of 16)
  float2* part;                // nsplit > 1: partial (max, sum) [Hq, nsplit, L - q0]
  int hpw;                     // q-heads per wave: 1, or G for a short query range (the wave
                               // reads its keys once and serves the whole group)
};

// Workgroup x index -> q-head.  Consecutive workgroups go to the 8 XCDs in
// turn, each with its own L2; with Hq % 8 == 0 this puts the q-heads
// [x*Hq/8, (x+1)*Hq/8) on XCD x, so the q-heads of a KV group (adjacent heads)
// share their keys through one L2.
__device__ __forceinline__ int head_of(int bx, int Hq) {
  return (Hq % 8 == 0) ? (bx % 8) * (Hq / 8) + bx / 8 : bx;
}

// First q-head of the wave's workgroup: the swizzled head, or the group's first.
__device__ __forceinline__ int first_head(const ImpArgs& a) {
  return a.hpw == 1 ? head_of(blockIdx.x, a.Hq) : (int)blockIdx.x * a.hpw;
}

__device__ __forceinline__ void softmax_merge(float& m, float& l, float m2, float l2) {
  const float mx = fmaxf(m, m2);
  if (mx == -INFINITY) return;
  l = (m == -INFINITY ? 0.f : l * __builtin_amdgcn_exp2f(m - mx)) +
      (m2 == -INFINITY ? 0.f : l2 * __builtin_amdgcn_exp2f(m2 - mx));
  m = mx;
}

// One lane's slice of a 16-row tile: lane (col, grp) holds row col, elements
// [STEP*s + SUB*grp, +SUB) of k-step s -- the A/B operand layout of the 16x16
// matrix-core instructions (for fp32, the four elements of a slice feed four
// 16x16x4 steps; a permutation of the dot product's terms shared by both
// operands).
template <int DT, int D>
struct Frag {
  static constexpr int kStep = DT == ADAKV_F32 ? 16 : 32;
  static constexpr int kSub = DT == ADAKV_F32 ? 4 : 8;
  static constexpr int kEl = DT == ADAKV_F32 ? 4 : 2;
  static constexpr int N = D / kStep;
  uint4 v[N];
  __device__ __forceinline__ void load(const char* row, int grp) {
#pragma unroll
    for (int s = 0; s < N; ++s) v[s] = load16(row + (int64_t)(kStep * s + kSub * grp) * kEl);
  }
};

template <int DT, int D>
__device__ __forceinline__ float4_t tile_dot(const Frag<DT, D>& a, const Frag<DT, D>& b) {
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < Frag<DT, D>::N; ++s) {
    if constexpr (DT == ADAKV_F32) {
      const uint32_t x[4] = {a.v[s].x, a.v[s].y, a.v[s].z, a.v[s].w};
      const uint32_t y[4] = {b.v[s].x, b.v[s].y, b.v[s].z, b.v[s].w};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(x[j]), __uint_as_float(y[j]), acc, 0, 0, 0);
    } else if constexpr (DT == ADAKV_BF16) {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a.v[s]),
                                                    __builtin_bit_cast(bf16x8_t, b.v[s]), acc, 0, 0, 0);
    } else {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a.v[s]),
                                                   __builtin_bit_cast(f16x8_t, b.v[s]), acc, 0, 0, 0);
    }
  }
  return acc;  // lane (col, grp): element i = tile row 4*grp + i, column col
}

// ---- pass 1: log-sum-exp of every query row --------------------------------
// Wave: queries [q0 + qw, +64) resident as B (columns), keys streamed as A
// rows 16 at a time over [0, last query] -- or, when the queries are too few
// to fill the GPU (SnapKV's window), over one of nsplit key ranges, whose
// partial (max, sum) importance_merge_kernel combines.  Lane (col, grp) keeps
// an online (max, sum) for query col of each resident tile over keys
// 4*grp + i of each step; the four lanes of a column merge at the end.
template <int DT, int D>
__global__ __launch_bounds__(kEvNT) void importance_lse_kernel(ImpArgs a) {
  const int h0 = first_head(a);
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int col = lane & 15, grp = lane >> 4;
  const int nq = a.L - a.q0;
  // The wave's four resident tiles are four consecutive (q-head, 16-query tile)
  // pairs of its q-heads (one head, or a KV group's heads for a short query
  // range); waves -> (pair group, key split), splits fastest, the pair groups
  // holding the last queries (the most keys) dispatched first.
  const int nqt = (nq + 15) / 16;
  const int npairs = a.hpw * nqt;
  const int ngroups = (npairs + 3) / 4;
  const int gw = (int)blockIdx.y * (kEvNT / kWave) + w;
  if (gw >= ngroups * a.nsplit) return;                   // uniform over the wave; no barriers below
  const int split = gw % a.nsplit;
  const int pg = ngroups - 1 - gw / a.nsplit;
  const char* kb = a.k + (int64_t)(h0 / a.G) * a.ksh;
  int hs[4], qrow[4];
  bool live[4];
  int qlast = 0;
  Frag<DT, D> qf[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int p = pg * 4 + t;
    live[t] = p < npairs;                                 // uniform over the wave
    hs[t] = h0 + (live[t] ? p / nqt : 0);
    qrow[t] = a.q0 + 16 * (live[t] ? p % nqt : 0);
    if (live[t]) qlast = max(qlast, min(qrow[t] + 15, a.L - 1));
    qf[t].load(a.q + (int64_t)hs[t] * a.qsh + (int64_t)min(qrow[t] + col, a.L - 1) * a.qss, grp);
  }
  const int jb = split * a.klen, je = min(jb + a.klen, qlast + 1);
  float m[4], l[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) { m[t] = -INFINITY; l[t] = 0.f; }
  // keys of the next step are loaded before this step's products
  Frag<DT, D> kf;
  if (jb < je) kf.load(kb + (int64_t)min(jb + col, a.L - 1) * a.kss, grp);
  for (int j0 = jb; j0 < je; j0 += 16) {
    Frag<DT, D> kn;
    if (j0 + 16 < je) kn.load(kb + (int64_t)min(j0 + 16 + col, a.L - 1) * a.kss, grp);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (!live[t]) continue;                             // uniform over the wave
      const float4_t s = tile_dot(kf, qf[t]);
      const int qi = qrow[t] + col;
      float z[4], mx = m[t];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        z[i] = (j0 + 4 * grp + i <= qi) ? s[i] * a.c2 : -INFINITY;
        mx = fmaxf(mx, z[i]);
      }
      if (mx != -INFINITY) {
        float acc = m[t] == -INFINITY ? 0.f : l[t] * __builtin_amdgcn_exp2f(m[t] - mx);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc += __builtin_amdgcn_exp2f(z[i] - mx);   // exp2(-inf) = 0
        l[t] = acc;
        m[t] = mx;
      }
    }
    kf = kn;
  }
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int o = 16; o <= 32; o <<= 1) softmax_merge(m[t], l[t], __shfl_xor(m[t], o), __shfl_xor(l[t], o));
    const int qo = qrow[t] - a.q0 + col;
    if (live[t] && grp == 0 && qo < nq) {
      if (a.nsplit == 1) a.lse[(int64_t)hs[t] * nq + qo] = m[t] + log2f(l[t]);
      else a.part[((int64_t)hs[t] * a.nsplit + split) * nq + qo] = make_float2(m[t], l[t]);
    }
  }
}

// Pass 1 with a key split: lse of each (q-head, query) from its partials, one
// wave per (q-head, query), the lanes striding over the splits.
__global__ __launch_bounds__(256) void importance_merge_kernel(ImpArgs a) {
  const int nq = a.L - a.q0;
  const int lane = threadIdx.x & (kWave - 1);
  const int qo = blockIdx.x * (256 / kWave) + threadIdx.x / kWave, h = blockIdx.y;
  if (qo >= nq) return;                                   // uniform over the wave
  float m = -INFINITY, l = 0.f;
  for (int s = lane; s < a.nsplit; s += kWave) {
    const float2 p = a.part[((int64_t)h * a.nsplit + s) * nq + qo];
    softmax_merge(m, l, p.x, p.y);
  }
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) softmax_merge(m, l, __shfl_xor(m, o), __shfl_xor(l, o));
  if (lane == 0) a.lse[(int64_t)h * nq + qo] = m + log2f(l);
}

// ---- pass 2: column sums ------------------------------------------------------
// Wave: keys [kw, +64) resident as A (rows), queries streamed as B columns 16
// at a time over [max(kw, q0), L).  Lane (col, grp) adds p = exp2(s - lse) of
// query col to its keys 4*grp + i of each tile; the 16 lanes of a row are
// summed at the end.
template <int DT, int D>
__global__ __launch_bounds__(kEvNT) void importance_colsum_kernel(ImpArgs a) {
  const int h0 = first_head(a);
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int col = lane & 15, grp = lane >> 4;
  const int nq = a.L - a.q0;
  const int kw = (blockIdx.y * (kEvNT / kWave) + w) * kEvRows;
  if (kw >= a.L) return;                                  // uniform over the wave; no barriers below
  const char* kb = a.k + (int64_t)(h0 / a.G) * a.ksh;
  Frag<DT, D> kf[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) kf[t].load(kb + (int64_t)min(kw + 16 * t + col, a.L - 1) * a.kss, grp);
  // (q-head, 16-query step) pairs in one loop -- the q-heads of the wave one
  // after another -- so that the next pair's queries and lse are in flight
  // while this pair's products run, across head boundaries too
  const int i_begin = max(kw, a.q0);                      // < L: kw < L and q0 < L
  auto q_row = [&](int hh, int i0) {
    return a.q + (int64_t)(h0 + hh) * a.qsh + (int64_t)min(i0 + col, a.L - 1) * a.qss;
  };
  auto lse_of = [&](int hh, int i0) {
    const int qi = i0 + col;
    return qi < a.L ? a.lse[(int64_t)(h0 + hh) * nq + qi - a.q0] : INFINITY;   // absent: exp2(-inf) = 0
  };
  float acc[4][4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[t][i] = 0.f;
  Frag<DT, D> qf;
  qf.load(q_row(0, i_begin), grp);
  float ls = lse_of(0, i_begin);
  for (int hh = 0, i0 = i_begin; hh < a.hpw;) {
    // the pair after this one: the next 16 queries, or the next head's first
    const bool last_of_head = i0 + 16 >= a.L;
    const int nh = last_of_head ? hh + 1 : hh, ni = last_of_head ? i_begin : i0 + 16;
    Frag<DT, D> qn;
    float ln = INFINITY;
    if (nh < a.hpw) {
      qn.load(q_row(nh, ni), grp);
      ln = lse_of(nh, ni);
    }
    const int qi = i0 + col;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float4_t s = tile_dot(kf[t], qf);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kj = kw + 16 * t + 4 * grp + i;
        acc[t][i] += (kj <= qi) ? __builtin_amdgcn_exp2f(s[i] * a.c2 - ls) : 0.f;
      }
    }
    if (last_of_head) {                                   // the head's sums out
      float* out = a.imp + (int64_t)(h0 + hh) * a.pitch;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        float r[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          r[i] = group_sum<16>(acc[t][i]);
          acc[t][i] = 0.f;
        }
        const int kj = kw + 16 * t + 4 * grp;
        if (col == 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (kj + i < a.L) out[kj + i] = r[i];
        }
      }
    }
    qf = qn;
    ls = ln;
    hh = nh;
    i0 = ni;
  }
}

// ---- SnapKV's pool --------------------------------------------------------------
__global__ __launch_bounds__(256) void pool_kernel(const float* in, float* out, int L, int pitch, int r) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= L) return;
  const float* row = in + (int64_t)blockIdx.y * pitch;
  float m = row[t];
  for (int u = max(t - r, 0); u <= min(t + r, L - 1); ++u) m = fmaxf(m, row[u]);
  out[(int64_t)blockIdx.y * pitch + t] = m;
}

// ---- ascending table of a bitmap ------------------------------------------------
// bits[0, ceil(n/32)) in LDS after a barrier; every thread of the workgroup calls.
template <int NT>
__device__ void table_from_bits(const uint32_t* bits, int n, int32_t* trow, int width, int32_t* len_out,
                                int* scratch) {
  const int words = (n + 31) / 32;
  const int per = (words + NT - 1) / NT;
  const int w0 = min((int)threadIdx.x * per, words), w1 = min(w0 + per, words);
  int cnt = 0;
  for (int i = w0; i < w1; ++i) cnt += __popc(bits[i]);
  int total;
  int o = block_excl_scan<NT>(cnt, scratch, &total);
  for (int i = w0; i < w1; ++i) {
    uint32_t x = bits[i];
    while (x) {
      const int b = __builtin_ctz(x);
      x &= x - 1;
      if (o < width) trow[o] = 32 * i + b;
      ++o;
    }
  }
  if (threadIdx.x == 0) *len_out = total;
}

__device__ __forceinline__ void set_bit(uint32_t* bits, int b) { atomicOr(&bits[b >> 5], 1u << (b & 31)); }

// ---- retained set ----------------------------------------------------------------
struct RetainArgs {
  const float* imp;
  int pitch, n_real, bs, budget, sink, local, c_min;
  uint8_t* mask;
  int mask_pitch;
  int32_t* table;              // nullptr: no table
  int width;
  int32_t* lens;
};

__global__ __launch_bounds__(kRetainNT) void retain_kernel(RetainArgs a) {
  constexpr int NT = kRetainNT, IPT = kRetainIPT;
  using Mask = MaskT<IPT>;
  constexpr Mask kOne = 1;
  __shared__ SelectLds<NT> L;
  __shared__ uint32_t bits[kRetainMaxBlocks / 32];
  __shared__ int scan[NT / kWave];
  const int h = blockIdx.x, tid = threadIdx.x;
  const int nb = (a.n_real + a.bs - 1) / a.bs;
  const int sink = min(a.sink, nb), local = min(a.local, nb);
  const int c_lo = sink, c_hi = max(nb - local, sink);
  const int n_forced = sink + (nb - max(nb - local, sink));
  const int k = min(max(a.budget, min(sink + local + a.c_min, nb)), nb);
  const int KC = min(max(k - n_forced, 0), c_hi - c_lo);
  select_init(L);
  for (int i = tid; i < (nb + 31) / 32; i += NT) bits[i] = 0;

  // block sums over real tokens: thread t owns blocks [t*IPT, (t+1)*IPT)
  const float* row = a.imp + (int64_t)h * a.pitch;
  const int base = tid * IPT;
  float v[IPT];
  Mask content = 0;
  float vmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int b = base + i;
    double s = 0.0;
    if (b < nb) {
      const int t1 = min((b + 1) * a.bs, a.n_real);
      for (int t = b * a.bs; t < t1; ++t) s += (double)row[t];
    }
    v[i] = (float)s;
    if (b >= c_lo && b < c_hi) {
      content |= kOne << i;
      vmax = fmaxf(vmax, sanitize(v[i]));
    }
  }
  L.maxv[tid] = vmax;
  __syncthreads();
  for (int b = tid; b < nb; b += NT)
    if (b < sink || b >= c_hi) set_bit(bits, b);
  if (KC > 0) {
    if (tid < kWave) select_threshold(L, KC, NT);
    __syncthreads();
    select_content<NT, IPT>(L, [&](int i) { return v[i]; }, content, base, KC, INFINITY,
                            [&](int, int blk) { set_bit(bits, blk); }, [](int) {});
  }
  __syncthreads();
  uint8_t* mrow = a.mask + (int64_t)h * a.mask_pitch;
  for (int b = tid; b < nb; b += NT) mrow[b] = (bits[b >> 5] >> (b & 31)) & 1u;
  if (a.table) table_from_bits<NT>(bits, nb, a.table + (int64_t)h * a.width, a.width, a.lens + h, scan);
}

// ---- union of a frozen set with the current sink and local blocks ---------------
struct UnionArgs {
  const int32_t* ftable;       // frozen rows [H, fwidth] (or nullptr)
  int fwidth;
  const int32_t* flens;
  const uint8_t* mask;         // or mask rows [H, mask_pitch] over [0, n_mask)
  int mask_pitch, n_mask;
  int n, sink, local;          // output block count and forced blocks
  int32_t* table;
  int width;
  int32_t* lens;
};

__global__ __launch_bounds__(kUnionNT) void union_table_kernel(UnionArgs a) {
  __shared__ uint32_t bits[kUnionMaxBlocks / 32];
  __shared__ int scan[kUnionNT / kWave];
  const int h = blockIdx.x, tid = threadIdx.x;
  for (int i = tid; i < (a.n + 31) / 32; i += kUnionNT) bits[i] = 0;
  __syncthreads();
  if (a.ftable) {
    const int32_t* f = a.ftable + (int64_t)h * a.fwidth;
    const int cnt = min(max(a.flens[h], 0), a.fwidth);
    for (int j = tid; j < cnt; j += kUnionNT) {
      const int b = f[j];
      if (b >= 0 && b < a.n) set_bit(bits, b);
    }
  }
  if (a.mask) {
    const uint8_t* m = a.mask + (int64_t)h * a.mask_pitch;
    for (int b = tid; b < min(a.n_mask, a.n); b += kUnionNT)
      if (m[b]) set_bit(bits, b);
  }
  const int sink = min(a.sink, a.n), lo = max(a.n - a.local, 0);
  for (int b = tid; b < a.n; b += kUnionNT)
    if (b < sink || b >= lo) set_bit(bits, b);
  __syncthreads();
  table_from_bits<kUnionNT>(bits, a.n, a.table + (int64_t)h * a.width, a.width, a.lens + h, scan);
}

// A short query range (at most 256 queries: SnapKV's window) is served by
// waves that each take a whole KV group: the keys of a wave are read once for
// its G q-heads.
constexpr int kGroupedQueries = 256;
int heads_per_wave(int G, int nq) { return nq <= kGroupedQueries ? G : 1; }

// Pass-1 key splits: none while the query waves fill the GPU (H2O); otherwise
// (few queries) enough splits for about 8192 waves, each over at least 256 keys.
int lse_pair_groups(int G, int nq) {
  return (heads_per_wave(G, nq) * ((nq + 15) / 16) + 3) / 4;
}

int lse_splits(int Hq, int G, int nq, int L) {
  const int64_t waves = (int64_t)(Hq / heads_per_wave(G, nq)) * lse_pair_groups(G, nq);
  if (waves >= 1024) return 1;
  return (int)std::max<int64_t>(1, std::min<int64_t>((8192 + waves - 1) / waves, (L + 255) / 256));
}

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

size_t importance_ws(int Hq, int G, int nq, int L) {
  const int ns = lse_splits(Hq, G, nq, L);
  const size_t lse = align256((size_t)Hq * nq * sizeof(float));
  return ns == 1 ? lse : lse + (size_t)Hq * ns * nq * sizeof(float2);
}

template <int DT>
hipError_t launch_importance_dt(ImpArgs a, int D, hipStream_t s) {
  constexpr int kRowsPerGroup = kEvNT / kWave * kEvRows;
  const int nq = a.L - a.q0;
  a.hpw = heads_per_wave(a.G, nq);
  a.nsplit = lse_splits(a.Hq, a.G, nq, a.L);
  a.klen = (a.L + a.nsplit - 1) / a.nsplit;
  a.klen = (a.klen + 15) / 16 * 16;
  a.part = reinterpret_cast<float2*>(reinterpret_cast<char*>(a.lse) + align256((size_t)a.Hq * nq * sizeof(float)));
  const int waves1 = lse_pair_groups(a.G, nq) * a.nsplit;
  const dim3 g1(a.Hq / a.hpw, (waves1 + kEvNT / kWave - 1) / (kEvNT / kWave));
  const dim3 g2(a.Hq / a.hpw, (a.L + kRowsPerGroup - 1) / kRowsPerGroup);
  if (D == 64) importance_lse_kernel<DT, 64><<<g1, kEvNT, 0, s>>>(a);
  else importance_lse_kernel<DT, 128><<<g1, kEvNT, 0, s>>>(a);
  if (a.nsplit > 1) importance_merge_kernel<<<dim3((nq + 3) / 4, a.Hq), 256, 0, s>>>(a);
  if (D == 64) importance_colsum_kernel<DT, 64><<<g2, kEvNT, 0, s>>>(a);
  else importance_colsum_kernel<DT, 128><<<g2, kEvNT, 0, s>>>(a);
  return hipGetLastError();
}

int status_of(hipError_t e) { return e == hipSuccess ? ADAKV_OK : ADAKV_ERR_LAUNCH; }
bool valid_dtype(int dt) { return dt == ADAKV_F32 || dt == ADAKV_F16 || dt == ADAKV_BF16; }
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_prompt(const adakv_prompt_t* p) {
  if (!p || !p->q || !p->k) return ADAKV_ERR_NULL;
  if (!valid_dtype(p->dtype)) return ADAKV_ERR_DTYPE;
  if (p->n_q_heads < 1 || p->n_kv_heads < 1 || p->n_q_heads % p->n_kv_heads) return ADAKV_ERR_SHAPE;
  if (p->n_tokens < 1) return ADAKV_ERR_SHAPE;
  if (p->n_tokens > kMaxTokens || p->n_q_heads > 65535) return ADAKV_ERR_UNSUPPORTED;
  if (p->head_dim != 64 && p->head_dim != 128) return ADAKV_ERR_UNSUPPORTED;
  const int e = p->dtype == ADAKV_F32 ? 4 : 8;             // elements per 16 bytes
  if (!aligned16(p->q) || !aligned16(p->k)) return ADAKV_ERR_VALUE;
  if (p->q_stride_h % e || p->q_stride_s % e || p->k_stride_h % e || p->k_stride_s % e) return ADAKV_ERR_VALUE;
  if (p->q_stride_h < 0 || p->q_stride_s < 0 || p->k_stride_h < 0 || p->k_stride_s < 0) return ADAKV_ERR_VALUE;
  return ADAKV_OK;
}

int check_sel(const adakv_selection_t* s) {
  if (!s || !s->block_table || !s->sel_lens) return ADAKV_ERR_NULL;
  if (s->table_width < 1) return ADAKV_ERR_SHAPE;
  return ADAKV_OK;
}

}  // namespace
}  // namespace adakv

using namespace adakv;

extern "C" {

size_t adakv_importance_workspace_bytes(const adakv_prompt_t* p, int32_t first_query) {
  if (check_prompt(p) != ADAKV_OK || first_query < 0 || first_query >= p->n_tokens) return 0;
  return importance_ws(p->n_q_heads, p->n_q_heads / p->n_kv_heads, p->n_tokens - first_query, p->n_tokens);
}

int adakv_key_importance(const adakv_prompt_t* p, int32_t first_query, float sm_scale, float* importance,
                         int32_t pitch, void* ws, size_t ws_bytes, void* stream) {
  int st;
  if ((st = check_prompt(p))) return st;
  if (!importance || !ws) return ADAKV_ERR_NULL;
  if (first_query < 0 || first_query >= p->n_tokens || !isfinite(sm_scale)) return ADAKV_ERR_VALUE;
  if (pitch < p->n_tokens) return ADAKV_ERR_SHAPE;
  if (ws_bytes < adakv_importance_workspace_bytes(p, first_query) || ((uintptr_t)ws & 255u))
    return ADAKV_ERR_WORKSPACE;
  const int el = p->dtype == ADAKV_F32 ? 4 : 2;
  ImpArgs a;
  a.q = reinterpret_cast<const char*>(p->q);
  a.k = reinterpret_cast<const char*>(p->k);
  a.qsh = p->q_stride_h * el; a.qss = p->q_stride_s * el;
  a.ksh = p->k_stride_h * el; a.kss = p->k_stride_s * el;
  a.Hq = p->n_q_heads; a.G = p->n_q_heads / p->n_kv_heads;
  a.L = p->n_tokens; a.q0 = first_query;
  a.c2 = (float)((double)sm_scale * 1.4426950408889634);
  a.lse = reinterpret_cast<float*>(ws);
  a.imp = importance; a.pitch = pitch;
  a.nsplit = 1; a.klen = p->n_tokens; a.part = nullptr; a.hpw = 1;   // set by the launcher
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  switch (p->dtype) {
    case ADAKV_F32: e = launch_importance_dt<ADAKV_F32>(a, p->head_dim, s); break;
    case ADAKV_F16: e = launch_importance_dt<ADAKV_F16>(a, p->head_dim, s); break;
    default: e = launch_importance_dt<ADAKV_BF16>(a, p->head_dim, s); break;
  }
  return status_of(e);
}

int adakv_importance_pool(const float* in, float* out, int32_t n_heads, int32_t n_tokens, int32_t pitch,
                          int32_t kernel, void* stream) {
  if (!in || !out) return ADAKV_ERR_NULL;
  if (n_heads < 1 || n_tokens < 1 || pitch < n_tokens) return ADAKV_ERR_SHAPE;
  if (n_heads > 65535 || n_tokens > kMaxTokens) return ADAKV_ERR_UNSUPPORTED;
  if (kernel < 1 || kernel % 2 == 0 || kernel > 1025) return ADAKV_ERR_VALUE;
  const float* in_end = in + (int64_t)(n_heads - 1) * pitch + n_tokens;
  const float* out_end = out + (int64_t)(n_heads - 1) * pitch + n_tokens;
  if (in < out_end && out < in_end) return ADAKV_ERR_VALUE;   // overlap
  pool_kernel<<<dim3((n_tokens + 255) / 256, n_heads), 256, 0, (hipStream_t)stream>>>(in, out, n_tokens, pitch,
                                                                                        kernel / 2);
  return status_of(hipGetLastError());
}

int adakv_retain_blocks(const float* importance, int32_t n_heads, int32_t pitch, int32_t n_real,
                        int32_t block_size, int32_t budget, int32_t n_sink_blocks, int32_t n_local_blocks,
                        int32_t c_min, uint8_t* mask, int32_t mask_pitch, const adakv_selection_t* sel,
                        void* stream) {
  if (!importance || !mask) return ADAKV_ERR_NULL;
  if (n_heads < 1 || n_real < 1 || block_size < 1 || pitch < n_real) return ADAKV_ERR_SHAPE;
  const int nb = (n_real + block_size - 1) / block_size;
  if (nb > kRetainMaxBlocks || n_heads > 65535) return ADAKV_ERR_UNSUPPORTED;
  if (mask_pitch < nb) return ADAKV_ERR_SHAPE;
  if (budget < 0 || n_sink_blocks < 0 || n_local_blocks < 0 || c_min < 0) return ADAKV_ERR_VALUE;
  RetainArgs a;
  a.imp = importance; a.pitch = pitch; a.n_real = n_real; a.bs = block_size;
  a.budget = budget; a.sink = n_sink_blocks; a.local = n_local_blocks; a.c_min = c_min;
  a.mask = mask; a.mask_pitch = mask_pitch;
  a.table = nullptr; a.width = 0; a.lens = nullptr;
  if (sel) {
    int st;
    if ((st = check_sel(sel))) return st;
    const int sink = std::min(n_sink_blocks, nb), local = std::min(n_local_blocks, nb);
    const int k = std::min(std::max(budget, std::min(sink + local + c_min, nb)), nb);
    if (sel->table_width < k) return ADAKV_ERR_SHAPE;
    a.table = sel->block_table; a.width = sel->table_width; a.lens = sel->sel_lens;
  }
  retain_kernel<<<n_heads, kRetainNT, 0, (hipStream_t)stream>>>(a);
  return status_of(hipGetLastError());
}

int adakv_frozen_table(const adakv_selection_t* frozen, int32_t n_heads, int32_t n_frozen_blocks, int32_t nb_now,
                       int32_t n_sink_blocks, int32_t n_local_blocks, const adakv_selection_t* out, void* stream) {
  int st;
  if ((st = check_sel(frozen)) || (st = check_sel(out))) return st;
  if (n_heads < 1 || n_frozen_blocks < 0 || nb_now < 1 || nb_now < n_frozen_blocks) return ADAKV_ERR_SHAPE;
  if (nb_now > kUnionMaxBlocks || n_heads > 65535) return ADAKV_ERR_UNSUPPORTED;
  if (n_sink_blocks < 0 || n_local_blocks < 0) return ADAKV_ERR_VALUE;
  const int64_t need = (int64_t)std::min(frozen->table_width, n_frozen_blocks) + std::min(n_sink_blocks, nb_now) +
                       std::min(n_local_blocks, nb_now);
  if (out->table_width < std::min<int64_t>(need, nb_now)) return ADAKV_ERR_SHAPE;
  UnionArgs a{};
  a.ftable = frozen->block_table; a.fwidth = frozen->table_width; a.flens = frozen->sel_lens;
  a.mask = nullptr; a.mask_pitch = 0; a.n_mask = 0;
  a.n = nb_now; a.sink = n_sink_blocks; a.local = n_local_blocks;
  a.table = out->block_table; a.width = out->table_width; a.lens = out->sel_lens;
  union_table_kernel<<<n_heads, kUnionNT, 0, (hipStream_t)stream>>>(a);
  return status_of(hipGetLastError());
}

int adakv_mask_table(const uint8_t* mask, int32_t n_heads, int32_t mask_pitch, int32_t n_mask_blocks,
                     int32_t nb_now, int32_t n_sink_blocks, int32_t n_local_blocks, const adakv_selection_t* out,
                     void* stream) {
  int st;
  if (!mask) return ADAKV_ERR_NULL;
  if ((st = check_sel(out))) return st;
  if (n_heads < 1 || n_mask_blocks < 1 || mask_pitch < n_mask_blocks || nb_now < n_mask_blocks)
    return ADAKV_ERR_SHAPE;
  if (nb_now > kUnionMaxBlocks || n_heads > 65535) return ADAKV_ERR_UNSUPPORTED;
  if (n_sink_blocks < 0 || n_local_blocks < 0) return ADAKV_ERR_VALUE;
  if (out->table_width < nb_now) return ADAKV_ERR_SHAPE;
  UnionArgs a{};
  a.ftable = nullptr; a.fwidth = 0; a.flens = nullptr;
  a.mask = mask; a.mask_pitch = mask_pitch; a.n_mask = n_mask_blocks;
  a.n = nb_now; a.sink = n_sink_blocks; a.local = n_local_blocks;
  a.table = out->block_table; a.width = out->table_width; a.lens = out->sel_lens;
  union_table_kernel<<<n_heads, kUnionNT, 0, (hipStream_t)stream>>>(a);
  return status_of(hipGetLastError());
}

}  // extern "C"
