// Top-k content selection of one head inside one workgroup, shared by the
// plan-only selection kernel and the fused selection + decode kernel
// (adakv/selector.py:18-60: content blocks by descending score, ties by the
// lower block index), and the mergeable softmax partials the entropy weights
// are built from (adakv/budget.py:31-37).
#pragma once

#include <float.h>

#include <type_traits>

#include "common.hpp"

namespace adakv {

constexpr int kSortCap = 512;       // candidates ranked exactly by all-pairs comparison
constexpr int kSmallKC = 16;        // up to this many, the threshold is found by repeated wave maxima

// NaN ranks last, infinities clamp to the finite range (they then tie with
// +/-FLT_MAX and are ordered by block index).
__device__ __forceinline__ float sanitize(float x) {
  if (x != x) return -FLT_MAX;
  return fminf(fmaxf(x, -FLT_MAX), FLT_MAX);
}

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

// Bitonic sort of keys[0, n) into descending order; n a power of two <= kSortCap.
template <int NT>
__device__ void bitonic_desc(uint64_t* keys, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += NT) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = keys[i], y = keys[ixj];
          const bool desc = (i & k) == 0;
          if (desc ? (x < y) : (x > y)) {
            keys[i] = y;
            keys[ixj] = x;
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

// ---- softmax partials ------------------------------------------------------
// Partial of a set of a head's scores z = score / temperature: m = max z,
// S = sum exp(z - m), T = sum exp(z - m) * (z - m).  Two partials merge by
// rescaling both to the larger max: T picks up (m' - M) * S'.  Then
// sum p log p = T / S - log S over the whole set.
//
// Record written by the score kernel per (sequence, q-head, score workgroup),
// kPartFloats = 20 floats in five 16-byte groups (stored group-major, at
// part_offset()):
//   [0..3]   m, S, T of the workgroup's rows, one unused float;
//   [4..7]   the largest sanitised content score of each of its 4 sub-chunks
//            (the rows of one wave; -inf: no content block);
//   [8..11]  the second largest of each sub-chunk (-inf: fewer than two);
//   [12..15] the third largest of each sub-chunk (-inf: fewer than three),
//            which bounds every content score of the sub-chunk but the two;
//   [16..19] the blocks holding the two, (first | second << 16) per
//            sub-chunk (0xffff: none).
// The two are exact in the selector's order (larger score, then lower block).
struct SoftPart {
  float m, S, T;
};
__device__ __forceinline__ SoftPart soft_empty() { return SoftPart{-INFINITY, 0.f, 0.f}; }
__device__ __forceinline__ SoftPart soft_merge(const SoftPart& x, const SoftPart& y) {
  const float M = fmaxf(x.m, y.m);
  if (M == -INFINITY) return soft_empty();
  const float dx = x.m - M, dy = y.m - M;
  const float fx = x.m == -INFINITY ? 0.f : __expf(dx), fy = y.m == -INFINITY ? 0.f : __expf(dy);
  return SoftPart{M, x.S * fx + y.S * fy,
                  (x.m == -INFINITY ? 0.f : fx * fmaf(dx, x.S, x.T)) + (y.m == -INFINITY ? 0.f : fy * fmaf(dy, y.S, y.T))};
}

// Merge over aligned groups of N lanes (N a power of two <= 64): the max
// first, then every lane rescales its sums to it once and the sums are added.
template <int N>
__device__ __forceinline__ SoftPart soft_group_merge(SoftPart p) {
  static_assert(N >= 1 && N <= 64 && (N & (N - 1)) == 0, "aligned power-of-two lane groups");
  if constexpr (N == 1) return p;
  float M = p.m;
  if constexpr (N >= 2) M = fmaxf(M, dpp_mov<0xB1>(M));
  if constexpr (N >= 4) M = fmaxf(M, dpp_mov<0x4E>(M));
  if constexpr (N >= 8) M = fmaxf(M, dpp_mov<0x141>(M));
  if constexpr (N >= 16) M = fmaxf(M, dpp_mov<0x140>(M));
  if constexpr (N >= 32) { const LanePair q = swap16(M); M = fmaxf(q.a, q.b); }
  if constexpr (N == 64) { const LanePair q = swap32(M); M = fmaxf(q.a, q.b); }
  float S = 0.f, T = 0.f;
  if (p.m != -INFINITY) {
    const float d = p.m - M, f = __expf(d);
    S = p.S * f;
    T = f * fmaf(d, p.S, p.T);
  }
  return SoftPart{M, group_sum<N>(S), group_sum<N>(T)};
}

// ---- the exact top two of a set of (score, block) entries --------------------
// Order of the selector (adakv/selector.py:44-52): larger score first, then the
// lower block.  Empty entries are (-inf, 0xffff).  v3 bounds every entry of
// the set outside the top two (the third largest score; -inf: none).
struct Top2 {
  float v1, v2, v3;
  int r1, r2;
};
__device__ __forceinline__ Top2 top2_empty() { return Top2{-INFINITY, -INFINITY, -INFINITY, 0xffff, 0xffff}; }
__device__ __forceinline__ bool entry_before(float va, int ra, float vb, int rb) {
  return va > vb || (va == vb && ra < rb);
}
// Adds entry (x, r); r is above every block added before, so an equal score
// added later ranks after the earlier one.
__device__ __forceinline__ void top2_push(Top2& t, float x, int r) {
  const bool c1 = x > t.v1, c2 = x > t.v2;   // c1 implies c2
  t.v3 = c2 ? t.v2 : fmaxf(t.v3, x);
  t.v2 = c1 ? t.v1 : (c2 ? x : t.v2);
  t.r2 = c1 ? t.r1 : (c2 ? r : t.r2);
  t.v1 = c1 ? x : t.v1;
  t.r1 = c1 ? r : t.r1;
}
// The top two (and bound) of the union of two disjoint sets, each given by its
// own (symmetric in its arguments).
__device__ __forceinline__ Top2 top2_merge(const Top2& a, const Top2& b) {
  const bool aw = entry_before(a.v1, a.r1, b.v1, b.r1);
  const float lv = aw ? b.v1 : a.v1, sv = aw ? a.v2 : b.v2;   // loser's first, winner's second
  const int lr = aw ? b.r1 : a.r1, sr = aw ? a.r2 : b.r2;
  const bool lw = entry_before(lv, lr, sv, sr);
  // outside the new top two: the other of (lv, sv), the loser's second, both bounds
  const float rest = fmaxf(fmaxf(lw ? sv : lv, aw ? b.v2 : a.v2), fmaxf(a.v3, b.v3));
  return Top2{aw ? a.v1 : b.v1, lw ? lv : sv, rest, aw ? a.r1 : b.r1, lw ? lr : sr};
}
// Merge with the lane across a 16-lane row (swap16) or wave half (swap32).
template <int XOR>
__device__ __forceinline__ Top2 top2_merge_lanes(const Top2& t) {
  static_assert(XOR == 16 || XOR == 32, "row or half-wave partners");
  auto sw = [](float x) { return XOR == 16 ? swap16(x) : swap32(x); };
  const LanePair v1 = sw(t.v1), v2 = sw(t.v2), v3 = sw(t.v3), r1 = sw(__int_as_float(t.r1)),
                 r2 = sw(__int_as_float(t.r2));
  return top2_merge(Top2{v1.a, v2.a, v3.a, __float_as_int(r1.a), __float_as_int(r2.a)},
                    Top2{v1.b, v2.b, v3.b, __float_as_int(r1.b), __float_as_int(r2.b)});
}
// Merge with a DPP partner within 16 lanes (quad_perm / mirror controls, which
// pair lanes symmetrically).
template <int CTRL>
__device__ __forceinline__ Top2 top2_merge_dpp(const Top2& t) {
  const Top2 o{dpp_mov<CTRL>(t.v1), dpp_mov<CTRL>(t.v2), dpp_mov<CTRL>(t.v3),
               __float_as_int(dpp_mov<CTRL>(__int_as_float(t.r1))), __float_as_int(dpp_mov<CTRL>(__int_as_float(t.r2)))};
  return top2_merge(t, o);
}
// Over the whole wave (every lane receives the result).
__device__ __forceinline__ Top2 top2_wave(Top2 t) {
  t = top2_merge_dpp<0xB1>(t);
  t = top2_merge_dpp<0x4E>(t);
  t = top2_merge_dpp<0x141>(t);
  t = top2_merge_dpp<0x140>(t);
  t = top2_merge_lanes<16>(t);
  return top2_merge_lanes<32>(t);
}

// Normalised entropy weight (adakv/budget.py:33-37) from the merged partial of
// all of a head's scores: -sum p log p / log(max(nb, 2)) + 1e-6, in fp64 after
// the division as NumPy promotes it; lognb = log((double)max(nb, 2)).
__device__ __forceinline__ double entropy_weight(const SoftPart& p, double lognb) {
  const float hs = p.T / p.S - __logf(p.S);
  return (double)(-hs) / lognb + 1e-6;
}

// ---- the nucleus weight (adakv/budget.py:38-41) -----------------------------
// w = 1 + #{k : c_k < P}, where c_k is the sum of the k largest block
// probabilities p = softmax(scores / T) and P the nucleus mass (compared in
// fp32, as NumPy compares its fp32 cumulative sums with a Python float).
// Equivalently w = K*, the fewest top blocks whose mass reaches P (nb + 1 when
// no prefix does).  K* is found without sorting, by a radix search over
// dist = bits(p_max) - bits(p) (non-negative floats order as their bit
// patterns, so ascending dist is descending p): each pass histograms the MASS
// of the remaining candidates per digit of dist and walks the digits upward
// until the mass before plus the bucket's reaches P.
//
// * Pass 1 bins dist >> 19 (1/16-octave steps of p below its maximum), the
//   last bin collecting everything from 255/16 octaves down; that bin is not
//   accumulated but derived from the totals, so a peaked head's long tail
//   costs no atomics.  Passes 2-4 take bits 18..11, 10..3 and 2..0 of dist
//   within the chosen bin.  Should the crossing fall in the last bin, four
//   more passes search all 31 bits of dist among the tail's elements.
// * Masses are exact integers (p * 2^60, truncated), so the passes agree with
//   each other whatever the order of the atomic additions.
// * When the passes end, the crossing value p* is known exactly, with
//   a = #{p > p*} and M their mass; the crossing is the i-th copy of p*,
//   i = ceil((P - M) / p*), and K* = a + i.
struct NucleusLds {
  unsigned long long mass[2][256];   // pass k histograms into buffer k & 1 while the other is cleared
  int cnt[2][256];
  float fred[16];
  double dred[16];
  unsigned long long qred[16];
  unsigned long long m_above;
  int n_above, n_at, done;
  uint32_t prefix;
};

// Exclusive prefix sum over the wave of 64-bit integers: DPP row shifts on
// both halves within each 16-lane row, then the row totals by readlane (as
// wave_incl_scan).  Integer sums: exact in any order.  (A __shfl_up scan
// goes through ds_bpermute, one LDS round trip per step and half.)
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_row_shr_u64(unsigned long long v) {
  const uint32_t lo = (uint32_t)dpp_row_shr<CTRL>((int)(uint32_t)v);
  const uint32_t hi = (uint32_t)dpp_row_shr<CTRL>((int)(uint32_t)(v >> 32));
  return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long wave_excl_scan_u64(unsigned long long x) {
  const int lane = threadIdx.x & (kWave - 1);
  unsigned long long inc = x;
  inc += dpp_row_shr_u64<0x111>(inc);
  inc += dpp_row_shr_u64<0x112>(inc);
  inc += dpp_row_shr_u64<0x114>(inc);
  inc += dpp_row_shr_u64<0x118>(inc);
  auto lane_u64 = [&](int l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)inc, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(inc >> 32), l);
    return ((unsigned long long)hi << 32) | lo;
  };
  const unsigned long long r0 = lane_u64(15), r1 = lane_u64(31), r2 = lane_u64(47);
  const int row = lane >> 4;
  inc += (row >= 1 ? r0 : 0ull) + (row >= 2 ? r1 : 0ull) + (row >= 3 ? r2 : 0ull);
  return inc - x;
}

// One pass (the k-th): candidates are the elements with cand(i), of mass
// mq(i) and digit digit(i) in [0, 256).  With tail_bin, bin 255 is not
// accumulated: it holds the rest of m_tot / n_tot.  Returns false (uniformly)
// when the mass never reaches Pq.  On return N.prefix holds the chosen digit
// appended to `prefix`.  Histogram buffer k & 1 must be clear on entry; the
// other buffer is cleared while wave 0 scans this one, for the next pass.
template <int NT, int IPT, typename Mass, typename Cand, typename Digit>
__device__ __forceinline__ bool nucleus_pass(NucleusLds& N, int k, Mass mq, Cand cand, Digit digit,
                                             unsigned long long Pq, uint32_t prefix, int bits, bool tail_bin,
                                             unsigned long long m_tot, int n_tot) {
  static_assert(NT >= 2 * kWave, "wave 0 scans while the others clear");
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  unsigned long long* hmass = N.mass[k & 1];
  int* hcnt = N.cnt[k & 1];
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    if (cand(i)) {
      const int d = digit(i);
      if (!(tail_bin && d == 255)) {
        atomicAdd(&hmass[d], mq(i));
        atomicAdd(&hcnt[d], 1);
      }
    }
  }
  lds_barrier();
  if (w != 0) {
    for (int j = tid - kWave; j < 256; j += NT - kWave) { N.mass[(k + 1) & 1][j] = 0ull; N.cnt[(k + 1) & 1][j] = 0; }
  } else {
    // lane l holds digits 4l .. 4l+3: lane order is digit order
    unsigned long long bm[4], lm = 0ull;
    int bc[4], lc = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bm[j] = hmass[4 * lane + j];
      bc[j] = hcnt[4 * lane + j];
      lm += bm[j];
      lc += bc[j];
    }
    if (tail_bin) {
      const unsigned long long m_rest = m_tot - wave_sum(lm);
      const int n_rest = n_tot - wave_sum(lc);
      if (lane == kWave - 1) { bm[3] = m_rest; bc[3] = n_rest; lm += m_rest; lc += n_rest; }
    }
    unsigned long long R = N.m_above + wave_excl_scan_u64(lm);
    int C = N.n_above + wave_incl_scan(lc) - lc;
    int hit = -1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (hit < 0) {
        if (bc[j] > 0 && R + bm[j] >= Pq) {
          hit = j;
        } else {
          R += bm[j];
          C += bc[j];
        }
      }
    }
    const uint64_t hits = __ballot(hit >= 0);
    if (hits != 0 && lane == __builtin_ctzll(hits)) {
      N.prefix = (prefix << bits) | (uint32_t)(4 * lane + hit);
      N.m_above = R;
      N.n_above = C;
      N.n_at = bc[hit];
    }
    if (lane == 0) N.done = hits ? 0 : 1;
  }
  lds_barrier();
  return N.done == 0;
}

// z: the head's scores (overwritten), thread t owning blocks [t*IPT,
// (t+1)*IPT); nb > 1.  Every thread receives the weight.  Per element only
// dist is kept (its mass is recomputed from it), so large IPT stays within
// the register file.
template <int NT, int IPT>
__device__ double nucleus_weight(NucleusLds& N, float (&z)[IPT], int nb, float tf, float nucleus_p) {
  constexpr int NW = NT / kWave;
  static_assert(NW <= 16, "per-wave partials");
  constexpr double kScale = 1152921504606846976.0;   // 2^60
  constexpr uint32_t kNone = 0xffffffffu;             // dist of blocks >= nb (real dists are < 2^31)
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int base = tid * IPT;
  // z = s / T (in place) and its maximum
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    z[i] = base + i < nb ? (tf == 1.f ? z[i] : __fdiv_rn(z[i], tf)) : -INFINITY;
    mx = fmaxf(mx, z[i]);
  }
  mx = wave_allreduce(mx, OpMax());
  if (lane == 0) N.fred[w] = mx;
  lds_barrier();
  mx = N.fred[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) mx = fmaxf(mx, N.fred[i]);
  // p = exp(z - max) / sum, the sum taken in fp64 and rounded once to fp32
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    z[i] = z[i] == -INFINITY ? 0.f : expf(z[i] - mx);     // z now holds e = exp(z - max)
    s += (double)z[i];
  }
  s = wave_sum(s);
  if (lane == 0) N.dred[w] = s;
  lds_barrier();
  s = 0.0;
#pragma unroll
  for (int i = 0; i < NW; ++i) s += N.dred[i];
  const float s32 = (float)s;
  const uint32_t kmax = __float_as_uint(__fdiv_rn(1.f, s32));      // p of the largest score: exp(0) / sum
  uint32_t dist[IPT];
#pragma unroll
  for (int i = 0; i < IPT; ++i) dist[i] = base + i < nb ? kmax - __float_as_uint(__fdiv_rn(z[i], s32)) : kNone;
  auto mass_of = [&](int i) -> unsigned long long {
    return (unsigned long long)((double)__uint_as_float(kmax - dist[i]) * kScale);
  };
  // with few elements per thread their masses stay in registers, else each
  // pass recomputes them from dist
  constexpr bool kKeep = IPT <= 8;
  unsigned long long mkeep[kKeep ? IPT : 1];
  if constexpr (kKeep) {
#pragma unroll
    for (int i = 0; i < IPT; ++i) mkeep[i] = dist[i] != kNone ? mass_of(i) : 0ull;
  }
  auto mq = [&](int i) -> unsigned long long {
    if constexpr (kKeep) return mkeep[i];
    else return mass_of(i);
  };
  unsigned long long mloc = 0ull;
#pragma unroll
  for (int i = 0; i < IPT; ++i) mloc += dist[i] != kNone ? mq(i) : 0ull;
  mloc = wave_sum(mloc);
  if (lane == 0) N.qred[w] = mloc;
  if (tid == 0) { N.m_above = 0ull; N.n_above = 0; }
  for (int j = tid; j < 256; j += NT) { N.mass[0][j] = 0ull; N.cnt[0][j] = 0; }   // the first pass's histograms
  lds_barrier();
  unsigned long long m_tot = 0ull;
#pragma unroll
  for (int i = 0; i < NW; ++i) m_tot += N.qred[i];
  const double P = fmin(fmax((double)nucleus_p, 0.0), 2.0);
  const unsigned long long Pq = (unsigned long long)(P * kScale);
  auto valid = [&](int i) { return dist[i] != kNone; };
  // pass 1: 1/16-octave bins below the maximum, the tail in bin 255
  if (!nucleus_pass<NT, IPT>(N, 0, mq, valid, [&](int i) { return (int)min(dist[i] >> 19, 255u); }, Pq, 0u, 8,
                             true, m_tot, nb))
    return (double)(nb + 1);                 // the whole mass stays below P
  uint32_t pre = N.prefix;
  uint32_t dstar;
  if (pre < 255u) {
    // bits 18..11, 10..3, 2..0 of dist within the bin
    constexpr int kShift[3] = {11, 3, 0}, kBits[3] = {8, 8, 3};
#pragma unroll 1
    for (int ps = 0; ps < 3; ++ps) {
      const int sh = kShift[ps], nbits = kBits[ps];
      nucleus_pass<NT, IPT>(N, 1 + ps, mq, [&](int i) { return valid(i) && (dist[i] >> (sh + nbits)) == pre; },
                            [&](int i) { return (int)((dist[i] >> sh) & ((1u << nbits) - 1u)); }, Pq, pre,
                            nbits, false, 0ull, 0);
      pre = N.prefix;
    }
    dstar = pre;
  } else {
    // the crossing lies in the tail: all 31 bits of dist among its elements
    constexpr uint32_t kTail = 255u << 19;
    pre = 0u;
#pragma unroll 1
    for (int sh = 24; sh >= 0; sh -= 8) {
      const int nbits = sh == 24 ? 7 : 8;
      nucleus_pass<NT, IPT>(N, (24 - sh) / 8 + 1, mq,
                            [&](int i) {
                              return valid(i) && dist[i] >= kTail && (sh == 24 || (dist[i] >> (sh + 8)) == pre);
                            },
                            [&](int i) { return (int)((dist[i] >> sh) & ((1u << nbits) - 1u)); }, Pq, pre,
                            nbits, false, 0ull, 0);
      pre = N.prefix;
    }
    dstar = pre;
  }
  const unsigned long long pstar = (unsigned long long)((double)__uint_as_float(kmax - dstar) * kScale);
  const unsigned long long need = Pq - N.m_above;     // > 0: the mass before the crossing stays below P
  int i = pstar > 0 ? (int)((need + pstar - 1) / pstar) : N.n_at;
  i = min(max(i, 1), N.n_at);
  return (double)(N.n_above + i);
}

// ---- the selection ---------------------------------------------------------
template <int NT>
struct SelectLds {
  alignas(16) uint64_t keys[kSortCap];
  int hist[256];
  int rank[kSortCap];
  alignas(16) float maxv[NT];   // content maxima of sub-chunks (upper bounds for the threshold)
  int rh[512];                  // two radix histograms for the threshold
  float f[NT / kWave];
  int i[NT / kWave];
  int bc[4];
  float tau;
  int n;
};

// Clears what the selection expects to start at zero; before the first barrier.
template <int NT>
__device__ __forceinline__ void select_init(SelectLds<NT>& L) {
  const int tid = threadIdx.x;
  if (tid == 0) { L.n = 0; L.tau = -FLT_MAX; }
  for (int i = tid; i < kSortCap; i += NT) L.rank[i] = 0;
  for (int i = tid; i < 512; i += NT) L.rh[i] = 0;
}

// The head's scores: thread t owns blocks [t*IPT, (t+1)*IPT); blocks >= nb read 0.
template <int IPT>
__device__ __forceinline__ void load_scores(const float* srow, int nb, float (&v)[IPT]) {
  const int base = threadIdx.x * IPT;
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

// Selection of the KC largest content scores of a head, by (score desc,
// block asc), with NaN ranked last and infinities clamped (sanitize), in two
// steps.
//
// select_threshold, by one wave (no workgroup barrier inside): a threshold
// tau from L.maxv[0, n_max) (n_max <= NT), the content maxima of disjoint
// sub-chunks (or -inf), written before a barrier.  Two radix passes over the
// order-preserving keys of the maxima (top byte, then the next byte within
// the bin that holds the KC-th largest) give the 16-bit key prefix of the
// KC-th largest maximum; tau is the smallest float with that prefix (for
// KC <= kSmallKC, tau is that maximum itself).  Those KC maxima are KC
// distinct content scores >= tau, so every one of the top KC is >= tau;
// maxima left out only lower tau.  L is select_init'ed.
template <int NT>
__device__ void select_threshold(SelectLds<NT>& L, int KC, int n_max) {
  const int lane = threadIdx.x & (kWave - 1);
  if (KC <= kSmallKC) {
    // small KC: the exact KC-th largest maximum, by KC rounds of a wave max
    // that removes one occurrence each (so equal maxima count separately)
    constexpr int PER = NT / kWave;
    float mv[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) mv[i] = lane + kWave * i < n_max ? L.maxv[lane + kWave * i] : -INFINITY;
    float kth = -INFINITY;
    int found = 0;
    for (int r = 0; r < KC; ++r) {
      float lm = mv[0];
#pragma unroll
      for (int i = 1; i < PER; ++i) lm = fmaxf(lm, mv[i]);
      const float wm = wave_allreduce(lm, OpMax());
      if (wm == -INFINITY) break;                         // fewer than KC maxima
      const uint64_t holders = __ballot(lm == wm);
      if (lane == (int)__builtin_ctzll(holders)) {
        bool done = false;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const bool hit = !done && mv[i] == wm;
          mv[i] = hit ? -INFINITY : mv[i];
          done = done || hit;
        }
      }
      kth = wm;
      ++found;
    }
    if (lane == 0) L.tau = found == KC ? fmaxf(kth, -FLT_MAX) : -FLT_MAX;
    return;
  }
  for (int i = lane; i < n_max; i += kWave) {
    const float mv = L.maxv[i];
    if (mv != -INFINITY) atomicAdd(&L.rh[(uint32_t)(sel_key(mv, 0) >> 32) >> 24], 1);
  }
  __builtin_amdgcn_wave_barrier();             // a wave's LDS operations complete in order
  radix_digit(L.rh, KC, L.bc);                 // bc[0] = digit, bc[1] = count above
  __builtin_amdgcn_wave_barrier();
  const uint32_t b1 = (uint32_t)L.bc[0];
  const int above1 = L.bc[1];
  for (int i = lane; i < n_max; i += kWave) {
    const float mv = L.maxv[i];
    const uint32_t key = (uint32_t)(sel_key(mv, 0) >> 32);
    if (mv != -INFINITY && (key >> 24) == b1) atomicAdd(&L.rh[256 + ((key >> 16) & 0xffu)], 1);
  }
  __builtin_amdgcn_wave_barrier();
  radix_digit(L.rh + 256, KC - above1, L.bc + 2);
  __builtin_amdgcn_wave_barrier();
  if (lane == 0) {
    const uint32_t tk = (b1 << 24) | ((uint32_t)L.bc[2] << 16);
    const uint32_t u = (tk & 0x80000000u) ? (tk & 0x7fffffffu) : ~tk;
    L.tau = (above1 < 0 || L.bc[3] < 0) ? -FLT_MAX : fmaxf(__uint_as_float(u), -FLT_MAX);
  }
}

// select_content, by all NT threads after a barrier that follows
// select_threshold: get(i) is the score of block base + i (i < IPT, a
// constant in unrolled loops) of thread t, `content` its content bits; vmax >= the largest sanitised
// content score among them (a thread with vmax < tau holds no candidate and
// skips the comparisons).  on_cand(n_cand) runs right after the candidates
// are compacted in L.keys (before they are ranked), by every thread.  The candidates (content scores
// >= tau) are compacted -- only threads holding one take part -- and, when at
// most kSortCap survive, ranked exactly by all-pairs comparison; otherwise
// linear-bin radix passes refine the boundary and a bitonic sort orders the
// survivors.  Calls emit(r, block) for every rank r < KC (KC >= 1).
template <int NT, int IPT, typename Get, typename Emit, typename OnCand>
__device__ void select_content(SelectLds<NT>& L, Get&& get, MaskT<IPT> content, int base, int KC,
                               float vmax, Emit&& emit, OnCand&& on_cand) {
  using Mask = MaskT<IPT>;
  constexpr Mask kOne = 1;
  const int tid = threadIdx.x;
  const float tau = L.tau;
  Mask cm = 0;
  if (vmax >= tau) {
    if (tau == -FLT_MAX) {                     // the bottom of the range: compare sanitised scores
#pragma unroll
      for (int i = 0; i < IPT; ++i) cm |= (sanitize(get(i)) >= tau) ? (kOne << i) : Mask(0);
    } else {
#pragma unroll
      for (int i = 0; i < IPT; ++i) cm |= (get(i) >= tau) ? (kOne << i) : Mask(0);
    }
    cm &= content;
  }
  if (cm) {                                    // few threads hold a candidate
    int o = atomicAdd(&L.n, popcnt(cm));
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
      if ((cm >> i) & kOne) {
        if (o < kSortCap) L.keys[o] = sel_key(sanitize(get(i)), base + i);
        ++o;
      }
    }
  }
  lds_barrier();
  const int n_cand = L.n;
  on_cand(n_cand);
  if (n_cand <= kSortCap) {
    // rank every candidate against all others, the pairs spread over the workgroup
    if (tid == 0 && (n_cand & 1)) L.keys[n_cand] = 0;   // pad to pairs: key 0 ranks below every key
    lds_barrier();
    const int n2 = (n_cand + 1) & ~1;
    const int npad = next_pow2(max(n_cand, 1));
    if (npad <= NT) {
      // NT / npad threads per candidate, each over a slice of the others
      const int parts = NT / npad, jlen = (ceil_div(n2, parts) + 1) & ~1;
      const int i = tid % npad, j0 = (tid / npad) * jlen, j1 = min(n2, j0 + jlen);
      if (i < n_cand) {
        const uint64_t ki = L.keys[i];
        int r = 0;
#pragma unroll 4
        for (int j = j0; j < j1; j += 2) {
          const ulonglong2 y = *reinterpret_cast<const ulonglong2*>(&L.keys[j]);
          r += (y.x > ki) + (y.y > ki);
        }
        if (r) atomicAdd(&L.rank[i], r);
      }
    } else {
      // more candidates than threads: each thread ranks several against all
      for (int i = tid; i < n_cand; i += NT) {
        const uint64_t ki = L.keys[i];
        int r = 0;
        for (int j = 0; j < n2; j += 2) {
          const ulonglong2 y = *reinterpret_cast<const ulonglong2*>(&L.keys[j]);
          r += (y.x > ki) + (y.y > ki);
        }
        L.rank[i] = r;
      }
    }
    lds_barrier();
    for (int e = tid; e < n_cand; e += NT)
      if (L.rank[e] < KC) emit(L.rank[e], key_index(L.keys[e]));
    return;
  }
  auto sv = [&](int i) { return sanitize(get(i)); };     // the fallback ranks sanitised scores

  // ---- fallback: the boundary bin holds too many blocks; refine exactly ----
  Mask cand = content, sel = 0;
  int need = KC, nsel = 0;
  bool sort_union = false;
  for (;;) {
    const int cnt = block_reduce<NT>(popcnt(cand), L.i, OpAdd());
    if (need <= 0) { cand = 0; break; }
    if (need >= cnt) { sel |= cand; cand = 0; nsel += cnt; need = 0; break; }
    if (nsel + cnt <= kSortCap) { sort_union = true; break; }
    if (cnt <= kSortCap) {
      int tot;
      const int off = block_excl_scan<NT>(popcnt(cand), L.i, &tot);
      int o = off;
#pragma unroll
      for (int i = 0; i < IPT; ++i)
        if ((cand >> i) & kOne) L.keys[o++] = sel_key(sv(i), base + i);
      const int n = next_pow2(tot);
      for (int i = tot + tid; i < n; i += NT) L.keys[i] = 0;
      __syncthreads();
      bitonic_desc<NT>(L.keys, n);
      const uint64_t kth = L.keys[need - 1];
#pragma unroll
      for (int i = 0; i < IPT; ++i)
        if (((cand >> i) & kOne) && sel_key(sv(i), base + i) >= kth) sel |= kOne << i;
      nsel += need; need = 0; cand = 0;
      __syncthreads();
      break;
    }
    float lo2 = FLT_MAX, hi2 = -FLT_MAX;
#pragma unroll
    for (int i = 0; i < IPT; ++i)
      if ((cand >> i) & kOne) { lo2 = fminf(lo2, sv(i)); hi2 = fmaxf(hi2, sv(i)); }
    lo2 = block_reduce<NT>(lo2, L.f, OpMin());
    hi2 = block_reduce<NT>(hi2, L.f, OpMax());
    if (lo2 == hi2) {
      // all candidates tie: take the lowest block indices
      int tot;
      const int off = block_excl_scan<NT>(popcnt(cand), L.i, &tot);
      int r = off;
#pragma unroll
      for (int i = 0; i < IPT; ++i)
        if ((cand >> i) & kOne) { if (r < need) sel |= kOne << i; ++r; }
      nsel += need; need = 0; cand = 0;
      break;
    }
    // 256 linear bins in double precision: hi2 and lo2 always land in
    // different bins, so the candidate set shrinks on every pass
    const double inv = 256.0 / ((double)hi2 - (double)lo2);
    auto bin2 = [&](float x) { return (int)fmin(255.0, floor(((double)hi2 - (double)x) * inv)); };
    for (int i = tid; i < 256; i += NT) L.hist[i] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < IPT; ++i)
      if ((cand >> i) & kOne) atomicAdd(&L.hist[bin2(sv(i))], 1);
    __syncthreads();
    if (tid < kWave) {
      int c4[4], s4 = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) { c4[j] = L.hist[4 * tid + j]; s4 += c4[j]; }
      int before = wave_incl_scan(s4) - s4;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (before < need && need <= before + c4[j]) { L.bc[2] = 4 * tid + j; L.bc[3] = before; }
        before += c4[j];
      }
    }
    __syncthreads();
    const int bs2 = L.bc[2], above = L.bc[3];
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
      if ((cand >> i) & kOne) {
        const int bi = bin2(sv(i));
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
  const int off = block_excl_scan<NT>(popcnt(outm), L.i, &tot);
  if (sort_union || KC <= kSortCap) {
    int o = off;
#pragma unroll
    for (int i = 0; i < IPT; ++i)
      if ((outm >> i) & kOne) L.keys[o++] = sel_key(sv(i), base + i);
    const int n = next_pow2(tot);
    for (int i = tot + tid; i < n; i += NT) L.keys[i] = 0;
    __syncthreads();
    bitonic_desc<NT>(L.keys, n);
    for (int j = tid; j < KC; j += NT) emit(j, key_index(L.keys[j]));
  } else {
    // more than kSortCap content blocks: listed in block order
    int o = off;
#pragma unroll
    for (int i = 0; i < IPT; ++i)
      if ((outm >> i) & kOne) emit(o++, base + i);
  }
}

}  // namespace adakv
