// Block-score kernel (adakv/estimator.py:62-79, adakv/attention.py:185-198),
// a template over the summary kind: instantiated for centroids in plan.hip and
// for minmax rows in minmax.hip (two translation units, built in parallel).
//
// score_kernel   one workgroup per (sequence, KV head, chunk of blocks)
//                dotting every summary row with the G query heads of the
//                group, plus one workgroup per appended block (the
//                decode-time summary append), dispatched first, which
//                recomputes that block's summary from K and scores it -- no
//                separate append launch.  Each chunk workgroup also writes
//                the softmax record of its rows per q-head, which the
//                selection kernels merge into the head's entropy weight.
//
// A minmax row [max | min] of length 2*head_dim scored against
// [max(q, 0) | min(q, 0)] is the Quest bound of adakv/estimator.py:76-79 as a
// dot product of length 2*head_dim: the same scan at twice the row length.
#pragma once

#include <float.h>

#include "common.hpp"
#include "internal.hpp"
#include "select.hpp"

namespace adakv {
namespace {

constexpr int kNT = 256;
constexpr int kScoreTiles = 4;   // 16-row summary tiles per wave of the matrix-core scan (at most)
constexpr int kScoreFill = 256;  // workgroups the scan aims for (one per CU) before it shortens its waves

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
// summary is recomputed from its real tokens, stored, and scored against the G
// q-heads.  A centroid is the sequential fp32 mean (summed in token order, one
// correctly rounded division, one rounding to the centroid type); a minmax
// row (MM) holds the per-dimension max of the keys in columns [0, D/2) and
// their min in [D/2, D), scored against max(q, 0) and min(q, 0)
// (adakv/estimator.py:76-79).  One workgroup per appended block; thread d owns
// column d: it loads that column of up to 16 token rows at once (every load
// instruction covers one row, coalesced) and reduces them in token order in
// registers.
template <int CDT, int KDT, int D, int GMAX, bool MM>
__device__ __forceinline__ void append_block(const ScoreArgs& a, int b, int kvh, int r, int len, float (*s_red)[kNT / kWave]) {
  constexpr int TB = 16;                       // token rows loaded together
  constexpr int DH = MM ? D / 2 : D;           // head_dim
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int d = min(tid, D - 1);               // threads past D mirror the last column (unused)
  const int dk = MM ? d % DH : d;              // the key / query column it reduces
  const bool upper = !MM || d < DH;            // max (or sum) column; else a min column
  const int t0 = r * a.bs, t1 = min(t0 + a.bs, len);
  const int G = a.G;
  // the query column first: its loads overlap the key loads
  float qd[GMAX];
  with_dtype(a.qdt, [&](auto tag) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g)
      qd[g] = load_t<decltype(tag)::value>(a.q, (int64_t)b * a.qsb + (int64_t)(kvh * G + min(g, G - 1)) * a.qsh + dk);
  });
  if constexpr (MM) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g) qd[g] = upper ? fmaxf(qd[g], 0.f) : fminf(qd[g], 0.f);
  }
  const int64_t kcol = (int64_t)b * a.ksb + (int64_t)kvh * a.ksh + dk;
  float acc = 0.f;
  for (int p0 = t0; p0 < t1; p0 += TB) {
    float x[TB];
#pragma unroll
    for (int j = 0; j < TB; ++j) x[j] = load_t<KDT>(a.k, kcol + (int64_t)min(p0 + j, t1 - 1) * a.kss);
#pragma unroll
    for (int j = 0; j < TB; ++j) {
      if (p0 + j < t1) {
        if constexpr (MM) acc = (p0 + j == t0) ? x[j] : (upper ? fmaxf(acc, x[j]) : fminf(acc, x[j]));
        else acc = (p0 + j == t0) ? x[j] : acc + x[j];
      }
    }
  }
  const float m = MM ? acc : __fdiv_rn(acc, (float)(t1 - t0));
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

// Record of a score workgroup's rows for one head, written by one lane: the
// softmax partial m, S, T and the top two content blocks of each of the 4
// sub-chunks with a bound of the rest (layout in select.hpp).
__device__ __forceinline__ void write_part(const ScoreArgs& a, int b, int h, int slot, float m, float S, float T,
                                           const Top2 (&t)[4]) {
  auto rec = [&](int g) { return reinterpret_cast<float4*>(a.parts + part_offset(b, a.Hq, h, a.parts_pitch, slot, g)); };
  auto pk = [](const Top2& x) { return __uint_as_float(((uint32_t)x.r1 & 0xffffu) | ((uint32_t)x.r2 << 16)); };
  *rec(0) = make_float4(m, S, T, 0.f);
  *rec(1) = make_float4(t[0].v1, t[1].v1, t[2].v1, t[3].v1);
  *rec(2) = make_float4(t[0].v2, t[1].v2, t[2].v2, t[3].v2);
  *rec(3) = make_float4(t[0].v3, t[1].v3, t[2].v3, t[3].v3);
  *rec(4) = make_float4(pk(t[0]), pk(t[1]), pk(t[2]), pk(t[3]));
}

// fp32 centroids: one workgroup per chunk of CB blocks; every centroid row is
// read once with 16-byte loads and dotted with the G queries (fp32 FMA, then a
// DPP butterfly over the lanes sharing the row); one partial per chunk.
template <int CDT, int D, int GMAX, bool MM>
__device__ __forceinline__ void score_chunk_valu(const ScoreArgs& a, int b, int kvh, int unit, int nb, int nrows,
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
  stage_q<kNT, GMAX, D, MM>(s_q, a.q, a.qdt, (int64_t)b * a.qsb + (int64_t)kvh * G * a.qsh, a.qsh, G, 1.f);
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
    float m = -INFINITY;
    Top2 tp = top2_empty();
#pragma unroll
    for (int k = 0; k < RL; ++k) {
      const int r = lane + k * kWave;
      const bool ok = r < CB && row0 + r < nrows;
      const float x = ok ? s_sc[g][r] : 0.f;
      z[k] = ok ? (tf == 1.f ? x : __fdiv_rn(x, tf)) : -INFINITY;
      m = fmaxf(m, z[k]);
      top2_push(tp, (ok && row0 + r >= c_lo && row0 + r < c_hi) ? sanitize(x) : -INFINITY, row0 + r);
    }
    tp = top2_wave(tp);
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
    const Top2 t4[4] = {tp, top2_empty(), top2_empty(), top2_empty()};   // the chunk is one sub-chunk
    if (lane == 0) write_part(a, b, kvh * G + g, unit, m, S, T, t4);
  }
}

// bf16 / fp16 centroids on the matrix cores: S = C . Q^T with
// v_mfma_f32_16x16x32 -- a wave holds TPW tiles of 16 centroid rows in the
// A-operand layout (lane l: row l%16, a contiguous D/2-byte slice of it, all
// loads issued at once), the group's q-heads, zero-padded to 16, form the B
// operand.  Result lane (col, grp) holds the scores of rows 4*grp .. +3 of a
// tile for head col: written as 16-byte stores, and reduced over the wave's
// 16 * TPW rows (one sub-chunk) into that head's softmax partial; the 4 waves'
// partials are merged through LDS into the workgroup's record.
template <int CDT, int D, int GMAX, bool MM, int TPW>
__device__ __forceinline__ void score_chunk_mfma(const ScoreArgs& a, int b, int kvh, int unit, int nb, int nrows,
                                 float (*s_pm)[GMAX][4], Top2 (*s_tp)[GMAX]) {
  static_assert(D % 32 == 0 && GMAX <= 16, "16x16 tiles over head_dim");
  constexpr int KS = D / 32;                // k-steps (16-byte loads per lane per tile)
  constexpr int QS = MM ? KS / 2 : KS;      // distinct q slices (a minmax row repeats q: max(q,0), min(q,0))
  // TPW: tiles per wave
  constexpr int RPW = 16 * TPW;             // rows per wave = rows per sub-chunk
  constexpr int NWV = kNT / kWave;
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int col = lane & 15, grp = lane >> 4;
  const int G = a.G;
  const int wrow0 = unit * NWV * RPW + w * RPW;
  if (unit * NWV * RPW >= nrows) return;    // uniform over the workgroup
  const bool wave_on = wrow0 < nrows;       // uniform over the wave
  float m = -INFINITY, S = 0.f, T = 0.f;
  Top2 tp = top2_empty();
  if (wave_on) {
    // B fragments: lane (col, grp) holds q[head col][32s + 8grp .. +7] (columns
    // col >= G repeat the last head; their scores are never stored); for a
    // minmax row, step s < QS takes max(q, 0) of slice s and step s >= QS
    // min(q, 0) of slice s - QS.  With q of the summary type and 16-byte
    // aligned rows they are plain 16-byte loads, issued first (the sign split
    // is a mask of the raw bits); otherwise typed loads after the summary loads.
    uint4 qf[KS];
    const int64_t qo = (int64_t)b * a.qsb + (int64_t)(kvh * G + min(col, G - 1)) * a.qsh + 8 * grp;
    if (a.q_vec) {
      const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q) + qo;
#pragma unroll
      for (int s = 0; s < QS; ++s) qf[s] = *reinterpret_cast<const uint4*>(qp + 32 * s);
    }
    // A fragments: lane (col, grp) reads row wrow0 + 16t + col, elements
    // [32s + 8grp, 32s + 8grp + 8) at k-step s, so that the 4 lanes of a row
    // read one whole 64-byte segment per load instruction
    const char* cbase = reinterpret_cast<const char*>(a.c) +
                        ((((int64_t)b * a.Hkv + kvh) * a.max_blocks) * D + 8 * grp) * 2;
    uint4 cf[TPW][KS];
    auto issue = [&](auto ld) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int r = min(wrow0 + 16 * t + col, nrows - 1);     // in bounds; extra rows masked below
#pragma unroll
        for (int s = 0; s < KS; ++s) cf[t][s] = ld(cbase + (int64_t)r * D * 2 + 64 * s);
      }
    };
    if (a.stream_loads) issue([](const char* p) { return load16_stream(p); });
    else issue([](const char* p) { return load16(p); });
    if (!a.q_vec) {
      with_dtype(a.qdt, [&](auto tag) {
        constexpr int QDT = decltype(tag)::value;
        float x[QS][8];
#pragma unroll
        for (int s = 0; s < QS; ++s)
#pragma unroll
          for (int u = 0; u < 8; ++u) x[s][u] = load_t<QDT>(a.q, qo + 32 * s + u);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          float y[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const float v = x[s % QS][u];
            y[u] = !MM ? v : s < QS ? fmaxf(v, 0.f) : fminf(v, 0.f);
          }
          uint32_t wv[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) wv[u] = pack2_typed<CDT>(y[2 * u], y[2 * u + 1]);
          qf[s] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
        }
      });
    } else if constexpr (MM) {
      // raw 16-bit halves: sign bit set -> the half belongs to min(q, 0), else to max(q, 0)
#pragma unroll
      for (int s = KS - 1; s >= 0; --s) {
        const uint4 r = qf[s % QS];
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
        uint32_t o[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t neg = ((w[u] >> 15) & 0x00010001u) * 0xFFFFu;
          o[u] = s < QS ? (w[u] & ~neg) : (w[u] & neg);
        }
        qf[s] = make_uint4(o[0], o[1], o[2], o[3]);
      }
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
    // Uniform over the wave: every row of the wave is a content row and holds
    // a score.  Then the content maximum is sanitize() of the plain maximum
    // (sanitize is monotone and maps NaN to its lowest value, which fmaxf
    // skips), and at temperature 1 it is also the softmax maximum: no per-row
    // selects.  Waves at the sink / local edges or past the scored rows take
    // the masked path.
    const bool full = wrow0 >= c_lo && wrow0 + RPW <= min(c_hi, nrows);
    float mx = -INFINITY;
    // the exact top two content rows of the sub-chunk for head col: this
    // lane's rows in increasing order, then the 4 lanes of the column
    if (full) {
#pragma unroll
      for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          mx = fmaxf(mx, sc[t][i]);
          top2_push(tp, sanitize(sc[t][i]), wrow0 + 16 * t + 4 * grp + i);
        }
    } else {
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = wrow0 + 16 * t + 4 * grp + i;
          const bool cont = (r >= c_lo) & (r < c_hi) & (r < nrows);
          top2_push(tp, cont ? sanitize(sc[t][i]) : -INFINITY, r);
        }
      }
    }
    tp = top2_merge_lanes<16>(tp);
    tp = top2_merge_lanes<32>(tp);
    if (tf != 1.f) {   // temperature: the correctly rounded division only when it is needed (uniform)
#pragma unroll
      for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[t][i] = __fdiv_rn(sc[t][i], tf);
    }
    if (full && tf == 1.f) {
      m = mx;
    } else {
#pragma unroll
      for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sc[t][i] = (wrow0 + 16 * t + 4 * grp + i < nrows) ? sc[t][i] : -INFINITY;
          m = fmaxf(m, sc[t][i]);
        }
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
  }
  if (a.parts == nullptr) return;           // uniform
  if (grp == 0 && col < G) {
    s_pm[w][col][0] = m; s_pm[w][col][1] = S; s_pm[w][col][2] = T;
    s_tp[w][col] = tp;
  }
  __syncthreads();
  if (w == 0 && lane < G) {
    // the workgroup's record: the 4 sub-chunk partials rescaled to their common
    // max.  Every wave's partial is read first and combined without branches
    // (a branch per partial serialised the LDS round trips); an empty partial
    // (m = -inf, S = T = 0) adds exactly zero.
    float4 pm[NWV];
#pragma unroll
    for (int ww = 0; ww < NWV; ++ww) pm[ww] = *reinterpret_cast<const float4*>(&s_pm[ww][lane][0]);
    const Top2 t4[4] = {s_tp[0][lane], s_tp[1][lane], s_tp[2][lane], s_tp[3][lane]};
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NWV; ++ww) M = fmaxf(M, pm[ww].x);
    float SS = 0.f, TT = 0.f;
#pragma unroll
    for (int ww = 0; ww < NWV; ++ww) {
      const bool on = pm[ww].x != -INFINITY;
      const float d = on ? pm[ww].x - M : 0.f, f = on ? __expf(d) : 0.f;
      SS += pm[ww].y * f;
      TT += f * fmaf(d, pm[ww].y, pm[ww].z);
    }
    write_part(a, b, kvh * G + lane, unit, M, SS, TT, t4);
  }
}

// Scores of every block of every (sequence, KV head) against its G q-heads.
// 1-D grid: first n_app workgroups per (sequence, KV head) for the appended
// blocks (dispatched first: their dependent K loads are the longest chain),
// then n_chunks workgroups per (sequence, KV head).
template <int CDT, int D, int GMAX, bool MM, int TPW>
__global__ __launch_bounds__(kNT) void score_kernel(ScoreArgs a) {
  warm_kernargs<sizeof(ScoreArgs) + 8>();
  constexpr bool kMfma = CDT != ADAKV_F32;
  constexpr int CBV = (kNT / kWave) * (kWave / (D / Elt<CDT>::kPerVec)) * 4;   // VALU rows per workgroup
  __shared__ float s_q[GMAX][D];
  __shared__ float s_sc[kMfma ? 1 : GMAX * CBV];
  __shared__ float s_red[GMAX][kNT / kWave];
  __shared__ __align__(16) float s_pm[kNT / kWave][GMAX][4];
  __shared__ Top2 s_tp[kNT / kWave][GMAX];

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
  // Sequence b's chunks are rotated by 8b: workgroups are dealt to XCDs (id
  // mod 8) and then to an XCD's CUs in turn, so without it a CU would hold
  // the same chunk indices of every sequence, and in a ragged batch (the high
  // chunks of short sequences empty) the CUs of the high chunks would idle.
  if (!app) unit = (unit + 8 * b) % a.n_chunks;
  // uniform values kept in scalar registers (divisions expanded on the vector
  // unit and a length loaded from memory would otherwise move every bound and
  // address derived from them to the vector unit)
  unit = __builtin_amdgcn_readfirstlane(unit);
  kvh = __builtin_amdgcn_readfirstlane(kvh);
  b = __builtin_amdgcn_readfirstlane(b);
  const int len = __builtin_amdgcn_readfirstlane(seq_len_of(a.seq_lens, a.uniform_len, b));
  const int nb = len > 0 ? ceil_div(len, a.bs) : 0;
  const int first_app = a.n_new > 0 ? max(len - a.n_new, 0) / a.bs : nb;
  const int G = a.G;

  if (app) {
    const int r = first_app + unit;
    if (r >= nb) return;
    with_dtype(a.kdt, [&](auto tag) { append_block<CDT, decltype(tag)::value, D, GMAX, MM>(a, b, kvh, r, len, s_red); });
    return;
  }
  const int nrows = min(nb, first_app);     // appended blocks are scored by their own workgroups
  if constexpr (kMfma) {
    score_chunk_mfma<CDT, D, GMAX, MM, TPW>(a, b, kvh, unit, nb, nrows, s_pm, s_tp);
  } else {
    if (unit * CBV >= nrows) return;
    score_chunk_valu<CDT, D, GMAX, MM>(a, b, kvh, unit, nb, nrows, s_q, s_sc);
  }
}

template <int CDT, int D, bool MM, int TPW>
void launch_score_g(const ScoreArgs& a, dim3 grid, hipStream_t s) {
  if (a.G <= 1) hipLaunchKernelGGL((score_kernel<CDT, D, 1, MM, TPW>), grid, dim3(kNT), 0, s, a);
  else if (a.G <= 2) hipLaunchKernelGGL((score_kernel<CDT, D, 2, MM, TPW>), grid, dim3(kNT), 0, s, a);
  else if (a.G <= 4) hipLaunchKernelGGL((score_kernel<CDT, D, 4, MM, TPW>), grid, dim3(kNT), 0, s, a);
  else if (a.G <= 8) hipLaunchKernelGGL((score_kernel<CDT, D, 8, MM, TPW>), grid, dim3(kNT), 0, s, a);
  else hipLaunchKernelGGL((score_kernel<CDT, D, 16, MM, TPW>), grid, dim3(kNT), 0, s, a);
}

// Tiles per wave of the matrix-core scan: kScoreTiles, halved while the grid
// would hold fewer than kScoreFill workgroups (short contexts: more, shorter
// waves, and finer sub-chunk maxima for the selection's threshold), as long as
// the records still fit their pitch.
// Rows any sequence can have: every length is clamped to uniform_len on the
// device, so a summary buffer allocated for more blocks is not scanned past it.
inline int score_rows(const ScoreArgs& a) {
  return std::min(a.max_blocks, (a.uniform_len + a.bs - 1) / a.bs);
}

inline int score_tiles(const ScoreArgs& a) {
  const int rows = score_rows(a);
  auto chunks = [&](int tpw) { return (rows + 64 * tpw - 1) / (64 * tpw); };
  int tpw = kScoreTiles;
  while (tpw > 1 && (int64_t)chunks(tpw) * a.Hkv * a.B < kScoreFill &&
         (a.parts == nullptr || chunks(tpw / 2) <= a.parts_pitch))
    tpw /= 2;
  return tpw;
}

template <int CDT, int D, bool MM>
hipError_t launch_score_d(ScoreArgs& a, hipStream_t s) {
  int tpw = kScoreTiles;
  if constexpr (CDT == ADAKV_F32) {
    constexpr int CB = (kNT / kWave) * (kWave / (D / 4)) * 4;   // rows per workgroup = rows per partial
    a.chunk_rows = CB;
  } else {
    tpw = score_tiles(a);
    a.chunk_rows = 4 * 16 * tpw;                                // 4 waves of 16-row tiles per record
  }
  a.n_chunks = (score_rows(a) + a.chunk_rows - 1) / a.chunk_rows;
  // Non-temporal summary loads while the scan is at most two workgroups per
  // CU (its whole read in flight at once); cached loads for larger grids.
  // Measured: 128K, batch 1 (256 workgroups) 19.97 -> 19.3 us per step; an
  // 8-sequence ragged batch (2048) 39.7 -> 42 us with non-temporal loads.
  a.stream_loads = (int64_t)a.n_chunks * a.Hkv * a.B <= 2 * kScoreFill;
  // blocks holding the newest n_new tokens: at most ceil(n_new / bs) + 1
  a.n_app = a.n_new > 0 ? std::min((a.n_new + a.bs - 1) / a.bs + 1, a.max_blocks) : 0;
  dim3 grid((unsigned)((int64_t)(a.n_app + a.n_chunks) * a.Hkv * a.B));
  if constexpr (CDT == ADAKV_F32) {
    launch_score_g<CDT, D, MM, kScoreTiles>(a, grid, s);
  } else {
    if (tpw == 1) launch_score_g<CDT, D, MM, 1>(a, grid, s);
    else if (tpw == 2) launch_score_g<CDT, D, MM, 2>(a, grid, s);
    else launch_score_g<CDT, D, MM, kScoreTiles>(a, grid, s);
  }
  return hipGetLastError();
}

// D: the summary row length (head_dim; 2 * head_dim for a minmax row).
template <int CDT, bool MM>
hipError_t launch_score_c(ScoreArgs& a, int D, hipStream_t s) {
  switch (D) {
    case 32: if constexpr (!MM) return launch_score_d<CDT, 32, MM>(a, s); else return hipErrorInvalidValue;
    case 64: return launch_score_d<CDT, 64, MM>(a, s);
    case 128: return launch_score_d<CDT, 128, MM>(a, s);
    case 256: return launch_score_d<CDT, 256, MM>(a, s);
    default: return hipErrorInvalidValue;
  }
}

template <bool MM>
hipError_t launch_score_kind(ScoreArgs& a, int cdt, int D, hipStream_t s) {
  switch (cdt) {
    case ADAKV_F32: return launch_score_c<ADAKV_F32, MM>(a, D, s);
    case ADAKV_F16: return launch_score_c<ADAKV_F16, MM>(a, D, s);
    case ADAKV_BF16: return launch_score_c<ADAKV_BF16, MM>(a, D, s);
    default: return hipErrorInvalidValue;
  }
}


}  // namespace
}  // namespace adakv
