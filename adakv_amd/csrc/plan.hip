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
#include "select.hpp"

namespace adakv {
namespace {

constexpr int kNT = 256;
constexpr int kScoreTiles = 4;   // 16-row centroid tiles per wave of the matrix-core scan

__device__ __forceinline__ float round_to(float x, int dt) {
  if (dt == ADAKV_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(x));
  if (dt == ADAKV_F16) return f16_bits_to_f32(f32_to_f16_bits(x));
  return x;
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

// Softmax partial of a score workgroup's rows for one head, written by one
// lane: m, S, T and the content maxima of the 4 sub-chunks (select.hpp).
__device__ __forceinline__ void write_part(const ScoreArgs& a, int b, int h, int slot, float m, float S, float T,
                                           float hi0, float hi1, float hi2, float hi3) {
  float4* rec = reinterpret_cast<float4*>(a.parts + (((int64_t)b * a.Hq + h) * a.parts_pitch + slot) * kPartFloats);
  rec[0] = make_float4(m, S, T, hi0);
  rec[1] = make_float4(hi1, hi2, hi3, 0.f);
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
  // then finished from the partials by the selection); the chunk is one
  // sub-chunk for the content maxima
  constexpr int RL = (CB + kWave - 1) / kWave;   // rows per lane
  const Bounds bb = budget_bounds(nb, a.cfg);
  const int c_lo = bb.sink, c_hi = nb - bb.local;
  const float tf = (float)fmax(a.cfg.temperature, 1e-6);
  for (int g = w; g < G; g += kNT / kWave) {
    float z[RL];
    float m = -INFINITY, hi = -INFINITY;
#pragma unroll
    for (int k = 0; k < RL; ++k) {
      const int r = lane + k * kWave;
      const bool ok = r < CB && row0 + r < nrows;
      const float x = ok ? s_sc[g][r] : 0.f;
      z[k] = ok ? (tf == 1.f ? x : __fdiv_rn(x, tf)) : -INFINITY;
      m = fmaxf(m, z[k]);
      if (ok && row0 + r >= c_lo && row0 + r < c_hi) hi = fmaxf(hi, sanitize(x));
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
    hi = wave_allreduce(hi, OpMax());
    if (lane == 0) write_part(a, b, kvh * G + g, unit, m, S, T, hi, -INFINITY, -INFINITY, -INFINITY);
  }
}

// bf16 / fp16 centroids on the matrix cores: S = C . Q^T with
// v_mfma_f32_16x16x32 -- a wave holds 4 tiles of 16 centroid rows in the
// A-operand layout (lane l: row l%16, a contiguous D/2-byte slice of it, all
// loads issued at once), the group's q-heads, zero-padded to 16, form the B
// operand.  Result lane (col, grp) holds the scores of rows 4*grp .. +3 of a
// tile for head col: written as 16-byte stores, and reduced over the wave's
// 64 rows (one sub-chunk) into that head's softmax partial; the 4 waves'
// partials are merged through LDS into the workgroup's record.
template <int CDT, int D, int GMAX>
__device__ void score_chunk_mfma(const ScoreArgs& a, int b, int kvh, int unit, int nb, int nrows,
                                 float (*s_pm)[GMAX][4]) {
  static_assert(D % 32 == 0 && GMAX <= 16, "16x16 tiles over head_dim");
  constexpr int KS = D / 32;                // k-steps (16-byte loads per lane per tile)
  constexpr int TPW = kScoreTiles;          // tiles per wave
  constexpr int RPW = 16 * TPW;             // rows per wave = rows per sub-chunk
  constexpr int NWV = kNT / kWave;
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int col = lane & 15, grp = lane >> 4;
  const int G = a.G;
  const int wrow0 = unit * NWV * RPW + w * RPW;
  if (unit * NWV * RPW >= nrows) return;    // uniform over the workgroup
  const bool wave_on = wrow0 < nrows;       // uniform over the wave
  float m = -INFINITY, S = 0.f, T = 0.f, hi = -INFINITY;
  if (wave_on) {
    // B fragments: lane (col, grp) holds q[head col][32s + 8grp .. +7] (columns
    // col >= G repeat the last head; their scores are never stored).  With q of
    // the centroid type and 16-byte aligned rows they are plain 16-byte loads,
    // issued first; otherwise typed loads after the centroid loads.
    uint4 qf[KS];
    const int64_t qo = (int64_t)b * a.qsb + (int64_t)(kvh * G + min(col, G - 1)) * a.qsh + 8 * grp;
    if (a.q_vec) {
      const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q) + qo;
#pragma unroll
      for (int s = 0; s < KS; ++s) qf[s] = *reinterpret_cast<const uint4*>(qp + 32 * s);
    }
    // A fragments: lane (col, grp) reads row wrow0 + 16t + col, elements
    // [32s + 8grp, 32s + 8grp + 8) at k-step s, so that the 4 lanes of a row
    // read one whole 64-byte segment per load instruction
    const char* cbase = reinterpret_cast<const char*>(a.c) +
                        ((((int64_t)b * a.Hkv + kvh) * a.max_blocks) * D + 8 * grp) * 2;
    uint4 cf[TPW][KS];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int r = min(wrow0 + 16 * t + col, nrows - 1);     // in bounds; extra rows masked below
#pragma unroll
      for (int s = 0; s < KS; ++s) cf[t][s] = load16(cbase + (int64_t)r * D * 2 + 64 * s);
    }
    if (!a.q_vec) {
      with_dtype(a.qdt, [&](auto tag) {
        constexpr int QDT = decltype(tag)::value;
        float x[KS][8];
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int u = 0; u < 8; ++u) x[s][u] = load_t<QDT>(a.q, qo + 32 * s + u);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          uint32_t wv[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) wv[u] = pack2_typed<CDT>(x[s][2 * u], x[s][2 * u + 1]);
          qf[s] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
        }
      });
    }
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
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = wrow0 + 16 * t + 4 * grp + i;
        const bool cont = (r >= c_lo) & (r < c_hi) & (r < nrows);
        hi = fmaxf(hi, cont ? sanitize(sc[t][i]) : -INFINITY);
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
    pr = swap16(hi); hi = fmaxf(pr.a, pr.b); pr = swap32(hi); hi = fmaxf(pr.a, pr.b);
  }
  if (a.parts == nullptr) return;           // uniform
  if (grp == 0 && col < G) {
    s_pm[w][col][0] = m; s_pm[w][col][1] = S; s_pm[w][col][2] = T; s_pm[w][col][3] = hi;
  }
  __syncthreads();
  if (w == 0 && lane < G) {
    // the workgroup's record: the 4 sub-chunk partials rescaled to their common max
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NWV; ++ww) M = fmaxf(M, s_pm[ww][lane][0]);
    float SS = 0.f, TT = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int ww = 0; ww < NWV; ++ww) {
        const float mw = s_pm[ww][lane][0];
        if (mw != -INFINITY) {
          const float d = mw - M, f = __expf(d);
          SS += s_pm[ww][lane][1] * f;
          TT += f * fmaf(d, s_pm[ww][lane][1], s_pm[ww][lane][2]);
        }
      }
    }
    write_part(a, b, kvh * G + lane, unit, M, SS, TT, s_pm[0][lane][3], s_pm[1][lane][3], s_pm[2][lane][3],
               s_pm[3][lane][3]);
  }
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
  __shared__ float s_pm[kNT / kWave][GMAX][4];

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
    score_chunk_mfma<CDT, D, GMAX>(a, b, kvh, unit, nb, nrows, s_pm);
  } else {
    if (unit * CBV >= nrows) return;
    score_chunk_valu<CDT, D, GMAX>(a, b, kvh, unit, nb, nrows, s_q, s_sc);
  }
}

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
    const float4* rec = reinterpret_cast<const float4*>(a.parts + (((int64_t)b * a.Hq + h) * a.parts_pitch + c) *
                                                                  kPartFloats);
    const float4 r0 = rec[0], r1 = rec[1];
    pt = soft_merge(pt, SoftPart{r0.x, r0.y, r0.z});
    const float mx[4] = {r0.w, r1.x, r1.y, r1.z};
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
    a.chunk_rows = 4 * 16 * kScoreTiles;                        // 4 waves of 16-row tiles per record
    a.n_chunks = (a.max_blocks + a.chunk_rows - 1) / a.chunk_rows;
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
