// Plan kernels: centroid block scores, entropy weights, top-k block selection
// and the per-head budget (adakv/attention.py:149-247 with the numerics of the
// NumPy oracle: adakv/estimator.py:62-74, adakv/budget.py:28-86,
// adakv/selector.py:18-60).
//
// score_kernel   one workgroup per (sequence, KV head, chunk of CB blocks)
//                dotting every centroid row with the G query heads of the
//                group, plus one workgroup per appended block (the
//                decode-time centroid append), dispatched first, which
//                recomputes that block's centroid from K and scores it -- no
//                separate append launch.
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

namespace adakv {
namespace {

constexpr int kNT = 256;
constexpr int kSortCap = 512;

__device__ __forceinline__ float round_to(float x, int dt) {
  if (dt == ADAKV_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(x));
  if (dt == ADAKV_F16) return f16_bits_to_f32(f32_to_f16_bits(x));
  return x;
}

// NaN ranks last, infinities clamp to the finite range (they then tie with
// +/-FLT_MAX and are ordered by block index).
__device__ __forceinline__ float sanitize(float x) {
  if (x != x) return -FLT_MAX;
  return fminf(fmaxf(x, -FLT_MAX), FLT_MAX);
}

typedef float float4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

template <int DT>
__device__ __forceinline__ float4_t mfma_16x16x32(const uint4& a, const uint4& b, float4_t c) {
  if constexpr (DT == ADAKV_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
}
template <int DT>
__device__ __forceinline__ uint32_t pack2_typed(float lo, float hi) {
  if constexpr (DT == ADAKV_BF16) return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
  else return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
}

// ---------------------------------------------------------------- scores ----
// Decode-time append (adakv/estimator.py:62-74): block r gained tokens, so its
// centroid becomes the sequential fp32 mean of its real tokens (summed in
// token order, one correctly rounded division, one rounding to the centroid
// type); the new centroid is stored and scored against the G q-heads.  One
// workgroup per appended block; thread d owns column d: it loads that column
// of up to 16 token rows at once (every load instruction covers one row,
// coalesced) and adds them in token order in registers.
template <int CDT, int KDT, int D, int GMAX>
__device__ void append_block(const ScoreArgs& a, int b, int kvh, int r, int len, float (*s_red)[kNT / kWave]) {
  constexpr int TB = 16;                       // token rows loaded together
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int d = min(tid, D - 1);               // threads past D mirror the last column (unused)
  const int t0 = r * a.bs, t1 = min(t0 + a.bs, len);
  const int G = a.G;
  // the query column first: its loads overlap the key loads
  float qd[GMAX];
  with_dtype(a.qdt, [&](auto tag) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
      qd[g] = load_t<decltype(tag)::value>(a.q, (int64_t)b * a.qsb + (int64_t)(kvh * G + min(g, G - 1)) * a.qsh + d);
  });
  const int64_t kcol = (int64_t)b * a.ksb + (int64_t)kvh * a.ksh + d;
  float acc = 0.f;
  for (int p0 = t0; p0 < t1; p0 += TB) {
    float x[TB];
#pragma unroll
    for (int j = 0; j < TB; ++j) x[j] = load_t<KDT>(a.k, kcol + (int64_t)min(p0 + j, t1 - 1) * a.kss);
#pragma unroll
    for (int j = 0; j < TB; ++j)
      if (p0 + j < t1) acc = (p0 + j == t0) ? x[j] : acc + x[j];
  }
  const float m = __fdiv_rn(acc, (float)(t1 - t0));
  if (tid < D) store_elt(a.c, CDT, (((int64_t)b * a.Hkv + kvh) * a.max_blocks + r) * D + tid, m);
  const float c = tid < D ? round_to(m, CDT) : 0.f;
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g < G) {
      const float p = group_sum<kWave>(qd[g] * c);
      if (lane == 0) s_red[g][w] = p;
    }
  }
  __syncthreads();
  if (tid < G) {
    float sc = 0.f;
#pragma unroll
    for (int i = 0; i < kNT / kWave; ++i) sc += s_red[tid][i];
    a.scores[((int64_t)b * a.Hq + kvh * G + tid) * a.sp + r] = sc;
  }
}

// Softmax partial of a chunk for one head, written by one lane: see the
// PartRecord layout in internal.hpp.
__device__ __forceinline__ void write_part(const ScoreArgs& a, int b, int h, int chunk, float m, float S, float T,
                                           float lo, float hi) {
  float4* rec = reinterpret_cast<float4*>(a.parts + (((int64_t)b * a.Hq + h) * a.parts_pitch + chunk) * kPartFloats);
  rec[0] = make_float4(m, S, T, lo);
  rec[1] = make_float4(hi, 0.f, 0.f, 0.f);
}

// fp32 centroids: one workgroup per chunk of CB blocks; every centroid row is
// read once with 16-byte loads and dotted with the G queries (fp32 FMA, then a
// DPP butterfly over the lanes sharing the row); one partial per chunk.
template <int CDT, int D, int GMAX>
__device__ void score_chunk_valu(const ScoreArgs& a, int b, int kvh, int unit, int nb, int nrows,
                                 float (*s_q)[D], float* s_sc_flat) {
  constexpr int EPV = Elt<CDT>::kPerVec;
  constexpr int EB = Elt<CDT>::kBytes;
  constexpr int LPR = D / EPV;              // lanes per centroid row
  constexpr int RPL = kWave / LPR;          // rows per wave-wide load
  constexpr int NLD = 4;                    // loads in flight per lane
  constexpr int RPW = RPL * NLD;            // rows per wave
  constexpr int CB = (kNT / kWave) * RPW;   // rows (blocks) per workgroup
  auto s_sc = reinterpret_cast<float (*)[CB]>(s_sc_flat);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int G = a.G;
  const int row0 = unit * CB;
  const int seg = lane % LPR, rsub = lane / LPR;
  const int64_t cbase_el = (((int64_t)b * a.Hkv + kvh) * a.max_blocks) * D;
  const char* cbase = reinterpret_cast<const char*>(a.c) + cbase_el * EB;
  uint4 cv[NLD];
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    const int r = min(row0 + w * RPW + i * RPL + rsub, nrows - 1);   // in bounds; extra rows unused
    cv[i] = load16(cbase + ((int64_t)r * D + seg * EPV) * EB);
  }
  stage_q<kNT, GMAX, D>(s_q, a.q, a.qdt, (int64_t)b * a.qsb + (int64_t)kvh * G * a.qsh, a.qsh, G, 1.f);
  __syncthreads();
  float qv[GMAX][EPV];
#pragma unroll
  for (int g = 0; g < GMAX; ++g)
#pragma unroll
    for (int e = 0; e < EPV; ++e) qv[g][e] = g < G ? s_q[g][seg * EPV + e] : 0.f;
#pragma unroll
  for (int i = 0; i < NLD; ++i) {
    float x[EPV];
    unpack<CDT>(cv[i], x);
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      if (g < G) {
        float p = qv[g][0] * x[0];
#pragma unroll
        for (int e = 1; e < EPV; ++e) p = fmaf(qv[g][e], x[e], p);
        p = group_sum<LPR>(p);
        if (seg == 0) s_sc[g][w * RPW + i * RPL + rsub] = p;
      }
    }
  }
  __syncthreads();
  for (int idx = tid; idx < G * CB; idx += kNT) {
    const int g = idx / CB, r = idx % CB;
    if (row0 + r < nrows)
      a.scores[((int64_t)b * a.Hq + kvh * G + g) * a.sp + row0 + r] = s_sc[g][r];
  }
  if (a.parts == nullptr) return;
  // softmax partial of this chunk, one wave per q-head (adakv/budget.py:33-37 is
  // then finished from the partials by the selection)
  constexpr int RL = (CB + kWave - 1) / kWave;   // rows per lane
  const Bounds bb = budget_bounds(nb, a.cfg);
  const int c_lo = bb.sink, c_hi = nb - bb.local;
  const float tf = (float)fmax(a.cfg.temperature, 1e-6);
  for (int g = w; g < G; g += kNT / kWave) {
    float z[RL];
    float m = -INFINITY, lo = FLT_MAX, hi = -FLT_MAX;
#pragma unroll
    for (int k = 0; k < RL; ++k) {
      const int r = lane + k * kWave;
      const bool ok = r < CB && row0 + r < nrows;
      const float x = ok ? s_sc[g][r] : 0.f;
      z[k] = ok ? (tf == 1.f ? x : __fdiv_rn(x, tf)) : -INFINITY;
      m = fmaxf(m, z[k]);
      if (ok && row0 + r >= c_lo && row0 + r < c_hi) {
        const float xs = sanitize(x);
        lo = fminf(lo, xs);
        hi = fmaxf(hi, xs);
      }
    }
    m = wave_allreduce(m, OpMax());
    float S = 0.f, T = 0.f;
    if (m != -INFINITY) {
#pragma unroll
      for (int k = 0; k < RL; ++k) {
        if (z[k] != -INFINITY) {
          const float e = __expf(z[k] - m);
          S += e;
          T = fmaf(e, z[k] - m, T);
        }
      }
    }
    S = wave_allreduce(S, OpAdd());
    T = wave_allreduce(T, OpAdd());
    lo = wave_allreduce(lo, OpMin());
    hi = wave_allreduce(hi, OpMax());
    if (lane == 0) write_part(a, b, kvh * G + g, unit, m, S, T, lo, hi);
  }
}

// bf16 / fp16 centroids on the matrix cores: S = C . Q^T with
// v_mfma_f32_16x16x32 -- a wave holds 4 tiles of 16 centroid rows in the
// A-operand layout (lane l: row l%16, a contiguous D/2-byte slice of it, all
// loads issued at once), the group's q-heads, zero-padded to 16, form the B
// operand.  Result lane (col, grp) holds the scores of rows 4*grp .. +3 of a
// tile for head col: written as 16-byte stores, and reduced over the wave's
// 64 rows into that head's softmax partial (one partial per wave).
template <int CDT, int D, int GMAX>
__device__ void score_chunk_mfma(const ScoreArgs& a, int b, int kvh, int unit, int nb, int nrows) {
  static_assert(D % 32 == 0 && GMAX <= 16, "16x16 tiles over head_dim");
  constexpr int KS = D / 32;                // k-steps (16-byte loads per lane per tile)
  constexpr int TPW = 4;                    // tiles per wave
  constexpr int RPW = 16 * TPW;             // rows per wave = rows per partial
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int col = lane & 15, grp = lane >> 4;
  const int G = a.G;
  const int wrow0 = unit * (kNT / kWave) * RPW + w * RPW;
  if (wrow0 >= nrows) return;
  // A fragments: lane (col, grp) reads row wrow0 + 16t + col, elements [D/4*grp, D/4*(grp+1))
  const char* cbase = reinterpret_cast<const char*>(a.c) +
                      ((((int64_t)b * a.Hkv + kvh) * a.max_blocks) * D + (D / 4) * grp) * 2;
  uint4 cf[TPW][KS];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int r = min(wrow0 + 16 * t + col, nrows - 1);     // in bounds; extra rows masked below
#pragma unroll
    for (int s = 0; s < KS; ++s) cf[t][s] = load16(cbase + (int64_t)r * D * 2 + 16 * s);
  }
  // B fragments: lane (col, grp) holds q[head col][D/4*grp + 8s .. +7]
  uint4 qf[KS];
  with_dtype(a.qdt, [&](auto tag) {
    constexpr int QDT = decltype(tag)::value;
    const int64_t qo = (int64_t)b * a.qsb + (int64_t)(kvh * G + min(col, G - 1)) * a.qsh + (D / 4) * grp;
    float x[KS][8];
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int u = 0; u < 8; ++u) x[s][u] = load_t<QDT>(a.q, qo + 8 * s + u);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      uint32_t wv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) wv[u] = col < G ? pack2_typed<CDT>(x[s][2 * u], x[s][2 * u + 1]) : 0u;
      qf[s] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
    }
  });
  float sc[TPW][4];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = mfma_16x16x32<CDT>(cf[t][s], qf[s], acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[t][i] = acc[i];
  }
  // scores: rows 4*grp + i of each tile, head col
  if (col < G) {
    float* srow = a.scores + ((int64_t)b * a.Hq + kvh * G + col) * a.sp;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int r = wrow0 + 16 * t + 4 * grp;
      if (r + 3 < nrows) {
        *reinterpret_cast<float4*>(srow + r) = make_float4(sc[t][0], sc[t][1], sc[t][2], sc[t][3]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (r + i < nrows) srow[r + i] = sc[t][i];
      }
    }
  }
  if (a.parts == nullptr) return;
  // softmax partial of the wave's rows for head col (lanes col, col+16, col+32, col+48)
  const Bounds bb = budget_bounds(nb, a.cfg);
  const int c_lo = bb.sink, c_hi = nb - bb.local;
  const float tf = (float)fmax(a.cfg.temperature, 1e-6);
  // branch-free: content and validity are selects, empty rows contribute exp(-inf) = 0
  float m = -INFINITY, lo = FLT_MAX, hi = -FLT_MAX;
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = wrow0 + 16 * t + 4 * grp + i;
      const bool cont = (r >= c_lo) & (r < c_hi) & (r < nrows);
      const float xs = sanitize(sc[t][i]);
      lo = fminf(lo, cont ? xs : FLT_MAX);
      hi = fmaxf(hi, cont ? xs : -FLT_MAX);
    }
  }
  if (tf != 1.f) {   // temperature: the correctly rounded division only when it is needed (uniform)
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[t][i] = __fdiv_rn(sc[t][i], tf);
  }
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[t][i] = (wrow0 + 16 * t + 4 * grp + i < nrows) ? sc[t][i] : -INFINITY;
      m = fmaxf(m, sc[t][i]);
    }
  LanePair pr = swap16(m);
  m = fmaxf(pr.a, pr.b);
  pr = swap32(m);
  m = fmaxf(pr.a, pr.b);
  const float mm = m == -INFINITY ? 0.f : m;
  float S = 0.f, T = 0.f;
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float dz = sc[t][i] - mm;
      const float e = __expf(dz);
      S += e;
      T = fmaf(e, fmaxf(dz, -FLT_MAX), T);
    }
  pr = swap16(S); S = pr.a + pr.b; pr = swap32(S); S = pr.a + pr.b;
  pr = swap16(T); T = pr.a + pr.b; pr = swap32(T); T = pr.a + pr.b;
  pr = swap16(lo); lo = fminf(pr.a, pr.b); pr = swap32(lo); lo = fminf(pr.a, pr.b);
  pr = swap16(hi); hi = fmaxf(pr.a, pr.b); pr = swap32(hi); hi = fmaxf(pr.a, pr.b);
  if (grp == 0 && col < G) write_part(a, b, kvh * G + col, wrow0 / RPW, m, S, T, lo, hi);
}

// Scores of every block of every (sequence, KV head) against its G q-heads.
// 1-D grid: first n_app workgroups per (sequence, KV head) for the appended
// blocks (dispatched first: their dependent K loads are the longest chain),
// then n_chunks workgroups per (sequence, KV head).
template <int CDT, int D, int GMAX>
__global__ __launch_bounds__(kNT) void score_kernel(ScoreArgs a) {
  constexpr bool kMfma = CDT != ADAKV_F32;
  constexpr int CBV = (kNT / kWave) * (kWave / (D / Elt<CDT>::kPerVec)) * 4;   // VALU rows per workgroup
  __shared__ float s_q[GMAX][D];
  __shared__ float s_sc[kMfma ? 1 : GMAX * CBV];
  __shared__ float s_red[GMAX][kNT / kWave];

  int id = blockIdx.x;
  const bool app = id < a.n_app * a.Hkv * a.B;
  int unit, kvh, b;
  if (app) {
    unit = id % a.n_app; id /= a.n_app;
  } else {
    id -= a.n_app * a.Hkv * a.B;
    unit = id % a.n_chunks; id /= a.n_chunks;
  }
  kvh = id % a.Hkv;
  b = id / a.Hkv;
  const int len = seq_len_of(a.seq_lens, a.uniform_len, b);
  const int nb = len > 0 ? ceil_div(len, a.bs) : 0;
  const int first_app = a.n_new > 0 ? max(len - a.n_new, 0) / a.bs : nb;
  const int G = a.G;

  if (app) {
    const int r = first_app + unit;
    if (r >= nb) return;
    with_dtype(a.kdt, [&](auto tag) { append_block<CDT, decltype(tag)::value, D, GMAX>(a, b, kvh, r, len, s_red); });
    return;
  }
  const int nrows = min(nb, first_app);     // appended blocks are scored by their own workgroups
  if constexpr (kMfma) {
    score_chunk_mfma<CDT, D, GMAX>(a, b, kvh, unit, nb, nrows);
  } else {
    if (unit * CBV >= nrows) return;
    score_chunk_valu<CDT, D, GMAX>(a, b, kvh, unit, nb, nrows, s_q, s_sc);
  }
}

// ------------------------------------------------------------- selection ----
// Order-preserving map of a (sanitised) float to uint32 plus the block index,
// so that larger score, then smaller index, gives the larger key.
__device__ __forceinline__ uint64_t sel_key(float x, int idx) {
  uint32_t u = __float_as_uint(x);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint32_t)(0xffffffffu - (uint32_t)idx);
}
__device__ __forceinline__ int key_index(uint64_t k) {
  return (int)(0xffffffffu - (uint32_t)(k & 0xffffffffu));
}

// Bitonic sort of s_keys[0, n) into descending order; n a power of two <= kSortCap.
template <int NT>
__device__ void bitonic_desc(uint64_t* s_keys, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += NT) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = s_keys[i], y = s_keys[ixj];
          const bool desc = (i & k) == 0;
          if (desc ? (x < y) : (x > y)) {
            s_keys[i] = y;
            s_keys[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ int next_pow2(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

template <int IPT>
using MaskT = typename std::conditional<(IPT > 32), uint64_t, uint32_t>::type;

template <typename M>
__device__ __forceinline__ int popcnt(M m) {
  if constexpr (sizeof(M) == 8) return __popcll(m); else return __popc(m);
}

// Softmax partial (see PartRecord layout) and its merge: the larger max wins,
// the other side's sums are rescaled by exp(m' - M); T picks up (m' - M) * S'.
struct Part {
  float m, S, T, lo, hi;
};
__device__ __forceinline__ Part part_empty() { return Part{-INFINITY, 0.f, 0.f, FLT_MAX, -FLT_MAX}; }
__device__ __forceinline__ Part part_merge(const Part& x, const Part& y) {
  Part r;
  r.m = fmaxf(x.m, y.m);
  r.lo = fminf(x.lo, y.lo);
  r.hi = fmaxf(x.hi, y.hi);
  if (r.m == -INFINITY) { r.S = 0.f; r.T = 0.f; return r; }
  const float dx = x.m - r.m, dy = y.m - r.m;
  const float fx = x.m == -INFINITY ? 0.f : __expf(dx), fy = y.m == -INFINITY ? 0.f : __expf(dy);
  r.S = x.S * fx + y.S * fy;
  r.T = (x.m == -INFINITY ? 0.f : fx * fmaf(dx, x.S, x.T)) + (y.m == -INFINITY ? 0.f : fy * fmaf(dy, y.S, y.T));
  return r;
}
template <int CTRL>
__device__ __forceinline__ Part part_dpp(const Part& p) {
  return Part{dpp_mov<CTRL>(p.m), dpp_mov<CTRL>(p.S), dpp_mov<CTRL>(p.T), dpp_mov<CTRL>(p.lo), dpp_mov<CTRL>(p.hi)};
}
// Merge over the 64 lanes; every lane receives the result.
__device__ __forceinline__ Part part_wave_merge(Part p) {
  p = part_merge(p, part_dpp<0xB1>(p));
  p = part_merge(p, part_dpp<0x4E>(p));
  p = part_merge(p, part_dpp<0x141>(p));
  p = part_merge(p, part_dpp<0x140>(p));
  {
    const LanePair a = swap16(p.m), b = swap16(p.S), c = swap16(p.T), d = swap16(p.lo), e = swap16(p.hi);
    p = part_merge(Part{a.a, b.a, c.a, d.a, e.a}, Part{a.b, b.b, c.b, d.b, e.b});
  }
  {
    const LanePair a = swap32(p.m), b = swap32(p.S), c = swap32(p.T), d = swap32(p.lo), e = swap32(p.hi);
    p = part_merge(Part{a.a, b.a, c.a, d.a, e.a}, Part{a.b, b.b, c.b, d.b, e.b});
  }
  return p;
}

// Normalised entropy weight of head h (adakv/budget.py:33-37), by one wave
// from the per-wave softmax partials: sum p log p = T / S - log S.
template <int NW>
__device__ __forceinline__ void write_weight(const SelectArgs& a, int b, int h, int nb, bool adaptive,
                                             const float (*s_r)[5]) {
  if (!adaptive) return;
  const int lane = threadIdx.x & (kWave - 1);
  const bool ok = lane < NW;
  const float m = ok ? s_r[lane][0] : -INFINITY;
  const float M = wave_allreduce(m, OpMax());
  float S = 0.f, T = 0.f;
  if (m != -INFINITY) {
    const float d = m - M, f = __expf(d);
    S = s_r[lane][1] * f;
    T = f * fmaf(d, s_r[lane][1], s_r[lane][2]);
  }
  S = wave_allreduce(S, OpAdd());
  T = wave_allreduce(T, OpAdd());
  if (lane == 0) {
    const float hs = T / S - __logf(S);
    a.wbuf[(int64_t)b * a.Hq + h] = (double)(-hs) / log((double)max(nb, 2)) + 1e-6;
  }
}

// One wave: the digit d of a 256-bin histogram (bins indexed by digit, larger
// digit = larger key) that holds the need-th largest key; out[0] = d, out[1] =
// keys in larger digits.  out[1] = -1 when the histogram holds fewer than need keys.
__device__ __forceinline__ void radix_digit(const int* hist, int need, int* out) {
  const int lane = threadIdx.x & (kWave - 1);
  int c4[4], s4 = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) { c4[j] = hist[255 - (4 * lane + j)]; s4 += c4[j]; }
  const int inc = wave_incl_scan(s4);
  const int tot = __builtin_amdgcn_readlane(inc, kWave - 1);
  int before = inc - s4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (before < need && need <= before + c4[j]) { out[0] = 255 - (4 * lane + j); out[1] = before; }
    before += c4[j];
  }
  if (lane == 0 && (tot < need || need <= 0)) { out[0] = 0; out[1] = -1; }
}

template <int NT, int IPT>
__global__ __launch_bounds__(NT) void select_kernel(SelectArgs a) {
  static_assert(IPT <= 64 && IPT % 4 == 0 && NT >= 256, "one mask word per thread");
  constexpr int NW = NT / kWave;
  using Mask = MaskT<IPT>;
  constexpr Mask kOne = 1;
  __shared__ __align__(16) uint64_t s_keys[kSortCap];
  __shared__ int s_hist[256];
  __shared__ float s_r[NW][5];
  __shared__ int s_rank[kSortCap];
  __shared__ __align__(16) float s_max[NT];   // chunk content maxima (+ appended rows)
  __shared__ float s_tau;
  __shared__ int s_rh[512];             // two radix histograms for the threshold
  __shared__ float s_f[NW];
  __shared__ int s_i[NW];
  __shared__ int s_bc[4];
  __shared__ int s_n;

  const int h = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & (kWave - 1), w = tid / kWave;
  const int len = seq_len_of(a.seq_lens, a.uniform_len, b);
  const int nb = len > 0 ? ceil_div(len, a.bs) : 0;
  const Bounds bb = budget_bounds(nb, a.cfg);
  const int c_lo = bb.sink, c_hi = nb - bb.local;
  const int n_content = max(c_hi - c_lo, 0);
  const int KC = min(max(bb.kcap - bb.n_forced, 0), n_content);
  const bool adaptive = a.cfg.policy == ADAKV_POLICY_ADAPTIVE && nb > 1;
  if (tid == 0) { s_n = 0; s_tau = -FLT_MAX; }
  for (int i = tid; i < kSortCap; i += NT) s_rank[i] = 0;
  for (int i = tid; i < 512; i += NT) s_rh[i] = 0;

  // ---- forced prefix and padding of the block-table row ----
  int32_t* trow = a.table + ((int64_t)b * a.Hq + h) * a.T;
  const int local_lo = max(bb.sink, nb - bb.local);
  for (int j = tid; j < bb.n_forced; j += NT) trow[j] = j < bb.sink ? j : local_lo + (j - bb.sink);
  for (int j = bb.n_forced + KC + tid; j < a.T; j += NT) trow[j] = -1;

  // ---- the head's scores: thread t owns blocks [t*IPT, (t+1)*IPT) ----
  const float* srow = a.scores + ((int64_t)b * a.Hq + h) * a.sp;
  const int base = tid * IPT;
  float v[IPT];
#pragma unroll
  for (int i = 0; i < IPT; i += 4) {
    if (base + i + 3 < nb) {
      const float4 f = *reinterpret_cast<const float4*>(srow + base + i);
      v[i] = f.x; v[i + 1] = f.y; v[i + 2] = f.z; v[i + 3] = f.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) v[i + j] = (base + i + j < nb) ? srow[base + i + j] : 0.f;
    }
  }

  // ---- softmax partials: the score kernel's chunks plus the rows it left out ----
  // (blocks recomputed by the decode-time append are scored on their own and
  // belong to no chunk; each counts as a one-row chunk here).  A wave first
  // takes the max, rescales its lanes' sums to it once, then adds.
  const int first_app = a.n_new > 0 ? max(len - a.n_new, 0) / a.bs : nb;
  const int rows_in_chunks = min(nb, first_app);
  const int n_chunks = ceil_div(rows_in_chunks, a.chunk_rows);
  const float tf = (float)fmax(a.cfg.temperature, 1e-6);
  const bool unit = tf == 1.f;
  Part pt = part_empty();
  bool has = false;
  for (int c = tid; c < n_chunks; c += NT) {
    const float4* rec = reinterpret_cast<const float4*>(a.parts + (((int64_t)b * a.Hq + h) * a.parts_pitch + c) *
                                                                  kPartFloats);
    const float4 r0 = rec[0], r1 = rec[1];
    pt = part_merge(pt, Part{r0.x, r0.y, r0.z, r0.w, r1.x});
    // content maximum of the chunk (none: -inf); chunks past NT are not counted
    if (c < NT) s_max[c] = (r1.x == -FLT_MAX && r0.w == FLT_MAX) ? -INFINITY : r1.x;
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
      const float xs = sanitize(v[i]);
      pt = part_merge(pt, Part{z, 1.f, 0.f, is_content ? xs : FLT_MAX, is_content ? xs : -FLT_MAX});
      const int t = n_chunks + idx - rows_in_chunks;
      if (t < NT) s_max[t] = is_content ? xs : -INFINITY;
      has = true;
    }
  }
  const int n_max = min(n_chunks + (nb - rows_in_chunks), NT);
  if (tid >= n_max && tid < ((n_max + 3) & ~3)) s_max[tid] = -INFINITY;
  if (__ballot(has) != 0) {                    // waves without partials skip the reductions
    const float M = wave_allreduce(pt.m, OpMax());
    float S = 0.f, T = 0.f;
    if (pt.m != -INFINITY) {
      const float d = pt.m - M, f = __expf(d);
      S = pt.S * f;
      T = f * fmaf(d, pt.S, pt.T);
    }
    pt = Part{M, wave_allreduce(S, OpAdd()), wave_allreduce(T, OpAdd()), wave_allreduce(pt.lo, OpMin()),
              wave_allreduce(pt.hi, OpMax())};
  }
  if (lane == 0) { s_r[w][0] = pt.m; s_r[w][1] = pt.S; s_r[w][2] = pt.T; s_r[w][3] = pt.lo; s_r[w][4] = pt.hi; }
  __syncthreads();
  if (KC <= 0) {
    if (w == NW - 1) write_weight<NW>(a, b, h, nb, adaptive, s_r);
    return;
  }

  // ---- selection threshold tau from the chunk content maxima ----
  // Two radix passes over the order-preserving keys of the maxima (top byte,
  // then the next byte within the bin that holds the KC-th largest) give the
  // 16-bit key prefix of the KC-th largest maximum; tau is the smallest float
  // with that prefix.  At least KC content scores (those maxima) are >= tau,
  // so every one of the top KC is; missing maxima only lower tau.
  {
    const bool has_max = tid < n_max && s_max[tid] != -INFINITY;
    const uint32_t key = has_max ? (uint32_t)(sel_key(s_max[tid], 0) >> 32) : 0u;
    if (has_max) atomicAdd(&s_rh[key >> 24], 1);
    __syncthreads();
    if (w == 0) radix_digit(s_rh, KC, s_bc);          // s_bc[0] = digit, s_bc[1] = count above
    __syncthreads();
    const uint32_t b1 = (uint32_t)s_bc[0];
    const int above1 = s_bc[1];
    if (has_max && (key >> 24) == b1) atomicAdd(&s_rh[256 + ((key >> 16) & 0xffu)], 1);
    __syncthreads();
    if (w == 0) {
      radix_digit(s_rh + 256, KC - above1, s_bc + 2);
      if (lane == 0) {
        const uint32_t tk = (b1 << 24) | ((uint32_t)s_bc[2] << 16);
        const uint32_t u = (tk & 0x80000000u) ? (tk & 0x7fffffffu) : ~tk;
        s_tau = (above1 < 0 || s_bc[3] < 0) ? -FLT_MAX : fmaxf(__uint_as_float(u), -FLT_MAX);
      }
    }
  }
  __syncthreads();

  // ---- candidates: content scores >= tau, one LDS atomic per wave ----
  const float tau = s_tau;
  Mask cm = 0;
  if (tau == -FLT_MAX) {                       // the bottom of the range: compare sanitised scores
#pragma unroll
    for (int i = 0; i < IPT; ++i) cm |= (sanitize(v[i]) >= tau) ? (kOne << i) : Mask(0);
  } else {
#pragma unroll
    for (int i = 0; i < IPT; ++i) cm |= (v[i] >= tau) ? (kOne << i) : Mask(0);
  }
  cm &= content;
  {
    const int c = popcnt(cm);
    const int inc = wave_incl_scan(c);
    const int wtot = __builtin_amdgcn_readlane(inc, kWave - 1);
    if (wtot) {
      int o0 = 0;
      if (lane == kWave - 1) o0 = atomicAdd(&s_n, wtot);
      int o = __builtin_amdgcn_readlane(o0, kWave - 1) + inc - c;
#pragma unroll
      for (int i = 0; i < IPT; ++i) {
        const bool bit = (cm >> i) & kOne;
        if (__ballot(bit)) {                   // most element positions hold no candidate in the wave
          if (bit && o < kSortCap) s_keys[o] = sel_key(sanitize(v[i]), base + i);
          o += bit ? 1 : 0;
        }
      }
    }
  }
  __syncthreads();
  const int n_cand = s_n;
  if (n_cand <= kSortCap) {
    // rank every candidate against all others, the pairs spread over the workgroup
    if (tid == 0 && (n_cand & 1)) s_keys[n_cand] = 0;   // pad to pairs: key 0 ranks below every key
    __syncthreads();
    const int n2 = (n_cand + 1) & ~1;
    const int npad = next_pow2(max(n_cand, 1));
    const int parts = max(NT / npad, 1), jlen = (ceil_div(n2, parts) + 1) & ~1;
    const int i = tid % npad, j0 = (tid / npad) * jlen, j1 = min(n2, j0 + jlen);
    if (i < n_cand && tid / npad < parts) {
      const uint64_t ki = s_keys[i];
      int r = 0;
#pragma unroll 4
      for (int j = j0; j < j1; j += 2) {
        const ulonglong2 y = *reinterpret_cast<const ulonglong2*>(&s_keys[j]);
        r += (y.x > ki) + (y.y > ki);
      }
      if (r) atomicAdd(&s_rank[i], r);
    }
    __syncthreads();
    for (int e = tid; e < n_cand; e += NT)
      if (s_rank[e] < KC) trow[bb.n_forced + s_rank[e]] = key_index(s_keys[e]);
    if (w == NW - 1) write_weight<NW>(a, b, h, nb, adaptive, s_r);
    return;
  }
  if (w == NW - 1) write_weight<NW>(a, b, h, nb, adaptive, s_r);
#pragma unroll
  for (int i = 0; i < IPT; ++i)
    if ((content >> i) & kOne) v[i] = sanitize(v[i]);

  // ---- fallback: the boundary bin holds too many blocks; refine exactly ----
  Mask cand = content, sel = 0;
  int need = KC, nsel = 0;
  bool sort_union = false;
  for (;;) {
    const int cnt = block_reduce<NT>(popcnt(cand), s_i, OpAdd());
    if (need <= 0) { cand = 0; break; }
    if (need >= cnt) { sel |= cand; cand = 0; nsel += cnt; need = 0; break; }
    if (nsel + cnt <= kSortCap) { sort_union = true; break; }
    if (cnt <= kSortCap) {
      int tot;
      const int off = block_excl_scan<NT>(popcnt(cand), s_i, &tot);
      int o = off;
#pragma unroll
      for (int i = 0; i < IPT; ++i)
        if ((cand >> i) & kOne) s_keys[o++] = sel_key(v[i], base + i);
      const int n = next_pow2(tot);
      for (int i = tot + tid; i < n; i += NT) s_keys[i] = 0;
      __syncthreads();
      bitonic_desc<NT>(s_keys, n);
      const uint64_t kth = s_keys[need - 1];
#pragma unroll
      for (int i = 0; i < IPT; ++i)
        if (((cand >> i) & kOne) && sel_key(v[i], base + i) >= kth) sel |= kOne << i;
      nsel += need; need = 0; cand = 0;
      __syncthreads();
      break;
    }
    float lo2 = FLT_MAX, hi2 = -FLT_MAX;
#pragma unroll
    for (int i = 0; i < IPT; ++i)
      if ((cand >> i) & kOne) { lo2 = fminf(lo2, v[i]); hi2 = fmaxf(hi2, v[i]); }
    lo2 = block_reduce<NT>(lo2, s_f, OpMin());
    hi2 = block_reduce<NT>(hi2, s_f, OpMax());
    if (lo2 == hi2) {
      // all candidates tie: take the lowest block indices
      int tot;
      const int off = block_excl_scan<NT>(popcnt(cand), s_i, &tot);
      int r = off;
#pragma unroll
      for (int i = 0; i < IPT; ++i)
        if ((cand >> i) & kOne) { if (r < need) sel |= kOne << i; ++r; }
      nsel += need; need = 0; cand = 0;
      break;
    }
    // 256 linear bins in double precision: vhi2 and vlo2 always land in
    // different bins, so the candidate set shrinks on every pass
    const double inv = 256.0 / ((double)hi2 - (double)lo2);
    auto bin2 = [&](float x) { return (int)fmin(255.0, floor(((double)hi2 - (double)x) * inv)); };
    for (int i = tid; i < 256; i += NT) s_hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < IPT; ++i)
      if ((cand >> i) & kOne) atomicAdd(&s_hist[bin2(v[i])], 1);
    __syncthreads();
    if (tid < kWave) {
      int c4[4], s4 = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) { c4[j] = s_hist[4 * tid + j]; s4 += c4[j]; }
      int before = wave_incl_scan(s4) - s4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (before < need && need <= before + c4[j]) { s_bc[2] = 4 * tid + j; s_bc[3] = before; }
        before += c4[j];
      }
    }
    __syncthreads();
    const int bs2 = s_bc[2], above = s_bc[3];
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
      if ((cand >> i) & kOne) {
        const int bi = bin2(v[i]);
        if (bi < bs2) { sel |= kOne << i; cand &= ~(kOne << i); }
        else if (bi > bs2) cand &= ~(kOne << i);
      }
    }
    nsel += above;
    need -= above;
    __syncthreads();
  }
  const Mask outm = sort_union ? (sel | cand) : sel;
  int tot;
  const int off = block_excl_scan<NT>(popcnt(outm), s_i, &tot);
  if (sort_union || KC <= kSortCap) {
    int o = off;
#pragma unroll
    for (int i = 0; i < IPT; ++i)
      if ((outm >> i) & kOne) s_keys[o++] = sel_key(v[i], base + i);
    const int n = next_pow2(tot);
    for (int i = tot + tid; i < n; i += NT) s_keys[i] = 0;
    __syncthreads();
    bitonic_desc<NT>(s_keys, n);
    for (int j = tid; j < KC; j += NT) trow[bb.n_forced + j] = key_index(s_keys[j]);
  } else {
    // more than kSortCap content blocks: listed in block order
    int o = off;
#pragma unroll
    for (int i = 0; i < IPT; ++i)
      if ((outm >> i) & kOne) trow[bb.n_forced + o++] = base + i;
  }
}

// -------------------------------------------------------------- budgets ----
__global__ __launch_bounds__(kNT) void budget_kernel(BudgetArgs a) {
  extern __shared__ double s_w[];
  __shared__ double s_sum;
  const int b = blockIdx.x;
  const int len = seq_len_of(a.seq_lens, a.uniform_len, b);
  const int nb = len > 0 ? ceil_div(len, a.bs) : 0;
  const Bounds bb = budget_bounds(nb, a.cfg);
  const bool adaptive = a.cfg.policy == ADAKV_POLICY_ADAPTIVE && nb > 1;
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

template <int CDT, int D>
hipError_t launch_score_d(ScoreArgs& a, hipStream_t s) {
  if constexpr (CDT == ADAKV_F32) {
    constexpr int CB = (kNT / kWave) * (kWave / (D / 4)) * 4;   // rows per workgroup = rows per partial
    a.chunk_rows = CB;
    a.n_chunks = (a.max_blocks + CB - 1) / CB;
  } else {
    a.chunk_rows = 64;                                          // rows per wave = rows per partial
    a.n_chunks = (a.max_blocks + 4 * 64 - 1) / (4 * 64);        // 4 waves per workgroup
  }
  // blocks holding the newest n_new tokens: at most ceil(n_new / bs) + 1
  a.n_app = a.n_new > 0 ? std::min((a.n_new + a.bs - 1) / a.bs + 1, a.max_blocks) : 0;
  dim3 grid((unsigned)((int64_t)(a.n_app + a.n_chunks) * a.Hkv * a.B));
  if (a.G <= 1) hipLaunchKernelGGL((score_kernel<CDT, D, 1>), grid, dim3(kNT), 0, s, a);
  else if (a.G <= 2) hipLaunchKernelGGL((score_kernel<CDT, D, 2>), grid, dim3(kNT), 0, s, a);
  else if (a.G <= 4) hipLaunchKernelGGL((score_kernel<CDT, D, 4>), grid, dim3(kNT), 0, s, a);
  else hipLaunchKernelGGL((score_kernel<CDT, D, 8>), grid, dim3(kNT), 0, s, a);
  return hipGetLastError();
}

template <int CDT>
hipError_t launch_score_c(ScoreArgs& a, int D, hipStream_t s) {
  switch (D) {
    case 32: return launch_score_d<CDT, 32>(a, s);
    case 64: return launch_score_d<CDT, 64>(a, s);
    case 128: return launch_score_d<CDT, 128>(a, s);
    case 256: return launch_score_d<CDT, 256>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int score_chunks_max(int max_blocks, int D) {
  // the smallest chunk is that of fp32 centroids: 16 rows per wave-wide load set
  const int cb = std::max(1, (kNT / kWave) * (kWave / std::max(1, D / 4)) * 4);
  return (max_blocks + cb - 1) / cb;
}

hipError_t launch_score(ScoreArgs& a, int cdt, int D, hipStream_t s) {
  switch (cdt) {
    case ADAKV_F32: return launch_score_c<ADAKV_F32>(a, D, s);
    case ADAKV_F16: return launch_score_c<ADAKV_F16>(a, D, s);
    case ADAKV_BF16: return launch_score_c<ADAKV_BF16>(a, D, s);
    default: return hipErrorInvalidValue;
  }
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

hipError_t launch_budget(const BudgetArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(budget_kernel, dim3(a.B), dim3(kNT), (size_t)a.Hq * sizeof(double), s, a);
  return hipGetLastError();
}

}  // namespace adakv
