// Fused budget + selection + sparse decode of one AdaKV decode step, after the
// score kernel (adakv/attention.py:202-268: budget, selection and block-sparse
// attention of every q-head in one launch).
//
// One workgroup of NT threads (4 or 8 waves) per (q-head, sequence).  The step
// is a short chain of phases with few workgroup barriers:
//
// 0. Loads, issued before anything is computed: the softmax records the score
//    kernel left for every head of the sequence (LPH lanes per head), this
//    head's scores (thread t owns blocks [t*IPT, (t+1)*IPT)), the query, and
//    the K/V tiles of the head's forced sink and local blocks, which are known
//    before any selection.
// 1. Every head's entropy weight (adakv/budget.py:33-37) from its merged
//    records; this thread's content maximum (an upper bound of its scores).
//    Barrier.
// 2. Every wave, redundantly (no barrier): the sum of weights in NumPy's
//    pairwise order and this head's count (adakv/budget.py:80-86), KC = count
//    - forced, and a threshold tau <= the KC-th largest thread maximum: that
//    maximum itself for KC <= 16 (repeated wave maxima), a 16-bit key prefix
//    of it above (two radix passes by one wave, one barrier).  The KC maxima
//    above tau are KC distinct content scores, so the top KC are all >= tau.
// 3. Candidates (content scores >= tau), compacted per wave by ballot, so their
//    order is the same on every run.  Barrier.  Every wave ranks all
//    candidates exactly (score desc, block asc; adakv/selector.py:18-60) in
//    registers: candidate lane c holds its rank, and the block of rank r is a
//    ballot away.  More candidates than two per lane (ties), or KC > 64, take
//    the general selection instead: an exact radix select over all content
//    scores.
// 4. Flash-decode over the head's k blocks on the matrix cores (attend.hpp):
//    16-token item j on wave j % NW, the forced items from the registers they
//    were loaded into in phase 0.  The waves' (m, l, acc) merge through LDS.
//
// Registers stay at or below 256 per wave: a build of this kernel at 329
// (with the general selection unrolled over a thread's scores) started 2.7 us
// later after the score kernel than one at 247 (measured with wall-clock
// stamps), so the general selection is written as plain loops.
#include <float.h>

#include <algorithm>

#include "attend.hpp"
#include "common.hpp"
#include "internal.hpp"
#include "select.hpp"

namespace adakv {
namespace {

constexpr int kFastKC = 16;         // KC up to this: tau by repeated wave maxima
constexpr int kRadixKC = 64;        // KC up to this: tau by two radix passes (else the general selection)
constexpr int kCandLanes = 2;       // candidates per lane on the fast path
constexpr int kRecsUpFront = 8;     // records per lane loaded in phase 0
constexpr int kPoolWave = 3;        // the wave that ranks the candidate pool in phase 1
constexpr int kWeightLanes = kPoolWave * 64;   // waves 0..2 compute the heads' weights

template <int NT, int D>
struct StepLds {
  float maxv[NT];                                             // thread content maxima
  uint64_t cand[NT / kWave][kCandLanes * kWave];              // candidate keys, per wave
  int wn[NT / kWave];                                         // candidates per wave (-1: too many)
  int hist[512];                                              // radix histograms
  int rd[4];                                                  // radix digit and count above
  int sc[NT / kWave];                                         // scan scratch
  float tau;
  alignas(16) uint64_t pool_pk[kWave];                        // the pool wave's ranked candidates
  int pool_rank[kWave];                                       //   and their ranks
  int pool_n;                                                 //   count (-1: more than a wave)
  float pool_bound;                                           //   bound of every entry outside it
  alignas(16) uint64_t keys[kSortCap];                        // general selection: selected keys
  int list[kSortCap];                                         // content blocks by rank (general path)
  alignas(16) uint16_t q[D];                                  // the query (16-bit, K's type)
  uint32_t vt[(NT / kWave) * TileShape<D>::VT_WORDS];         // the waves' V tiles
  float m[NT / kWave], l[NT / kWave];
  float acc[NT / kWave][D];
};

// Lanes merging one head's records: the largest power of two with
// Hq * LPH <= NT, at most 16 (2 for Hq = 64, 4 for Hq = 32 over 192 lanes).
template <int NT>
__device__ __forceinline__ int lanes_per_head(int Hq) {
  int l = 16;
  while (l > 1 && l * Hq > NT) l >>= 1;
  return l;
}

// x / d, with s = log2(d) when d is a power of two (else -1).
__device__ __forceinline__ int div_p2(int x, int d, int s) { return s >= 0 ? (x >> s) : x / d; }

// x / d and x % d for x >= 0 and a uniform d > 0: a shift or mask when d is a
// power of two (the usual case: q-heads, GQA group, lanes per head, 16-token
// tiles per block), the expanded integer division otherwise.
__device__ __forceinline__ int div_u(int x, int d) { return (d & (d - 1)) == 0 ? (x >> __builtin_ctz(d)) : x / d; }
__device__ __forceinline__ int mod_u(int x, int d) { return (d & (d - 1)) == 0 ? (x & (d - 1)) : x % d; }

__device__ __forceinline__ double readlane_d(double x, int l) {
  const long long u = __double_as_longlong(x);
  const int lo = __builtin_amdgcn_readlane((int)(u & 0xffffffffll), l);
  const int hi = __builtin_amdgcn_readlane((int)(u >> 32), l);
  return __longlong_as_double(((long long)hi << 32) | (uint32_t)lo);
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t x, int l) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(x >> 32), l);
  return ((uint64_t)hi << 32) | lo;
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

// The KC-th largest of mv[0, n) (LDS, n <= NT), by one wave and without any
// barrier: KC rounds of a wave maximum, each removing one occurrence (equal
// values count separately).  -FLT_MAX when fewer than KC values are finite
// maxima (> -inf); every lane receives it.
template <int NT>
__device__ __forceinline__ float kth_largest(const float* mv, int n, int KC) {
  constexpr int PER = NT / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  float x[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) x[i] = lane + kWave * i < n ? mv[lane + kWave * i] : -INFINITY;
  float kth = -INFINITY;
  int found = 0;
  for (int r = 0; r < KC; ++r) {
    float lm = x[0];
#pragma unroll
    for (int i = 1; i < PER; ++i) lm = fmaxf(lm, x[i]);
    const float wm = wave_allreduce(lm, OpMax());
    if (wm == -INFINITY) break;
    const uint64_t holders = __ballot(lm == wm);
    if (lane == (int)__builtin_ctzll(holders)) {
      bool done = false;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const bool hit = !done && x[i] == wm;
        x[i] = hit ? -INFINITY : x[i];
        done = done || hit;
      }
    }
    kth = wm;
    ++found;
  }
  return found == KC ? fmaxf(kth, -FLT_MAX) : -FLT_MAX;
}

// A lower bound of the KC-th largest of mv[0, N), by one wave (its own LDS
// histograms, no workgroup barrier): the order-preserving keys of the values
// share a common leading prefix (the bits where the largest and smallest key
// agree); two radix passes over the two bytes just below it (the first, then
// the next within the bin that holds the KC-th largest) fix the prefix of the
// KC-th largest through those 16 bits; the bound is the smallest float with
// that prefix.  (Digits taken below the shared prefix spread the atomics over
// the bins: the top byte, shared by nearly every value, put all of them on
// one or two addresses.)  -FLT_MAX when fewer than KC values are finite (> -inf).
template <int N>
__device__ __forceinline__ float kth_largest_radix(const float* mv, int KC, int* hist, int* rd) {
  static_assert(N % kWave == 0, "whole waves of values");
  constexpr int PER = N / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t key[PER];
  bool ok[PER];
  uint32_t kmax = 0u, kmin = 0xffffffffu;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const float x = mv[lane + kWave * i];
    ok[i] = x != -INFINITY;
    key[i] = (uint32_t)(sel_key(x, 0) >> 32);
    kmax = ok[i] ? max(kmax, key[i]) : kmax;
    kmin = ok[i] ? min(kmin, key[i]) : kmin;
  }
  kmax = wave_allreduce_b32(kmax, [](uint32_t x, uint32_t y) { return max(x, y); });
  kmin = wave_allreduce_b32(kmin, [](uint32_t x, uint32_t y) { return min(x, y); });
  for (int i = lane; i < 512; i += kWave) hist[i] = 0;
  __builtin_amdgcn_wave_barrier();             // a wave's LDS operations complete in order
  // shared leading bits (24 at most, so that the first digit fits below them)
  const int cp = kmax == kmin ? 24 : min(__builtin_clz(kmax ^ kmin), 24);
  const int sh1 = 24 - cp;                     // first digit: bits [sh1, sh1 + 8)
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (ok[i]) atomicAdd(&hist[(key[i] >> sh1) & 0xffu], 1);
  __builtin_amdgcn_wave_barrier();
  radix_digit(hist, KC, rd);                   // rd[0] = digit, rd[1] = count above
  __builtin_amdgcn_wave_barrier();
  const uint32_t d1 = (uint32_t)rd[0];
  const int above1 = rd[1];
  const uint32_t top = sh1 + 8 >= 32 ? 0u : (kmax >> (sh1 + 8)) << (sh1 + 8);   // the shared prefix
  uint32_t tk = top | (d1 << sh1);
  bool short2 = false;
  if (sh1 >= 8) {                              // second digit: bits [sh1 - 8, sh1)
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (ok[i] && ((key[i] >> sh1) & 0xffu) == d1) atomicAdd(&hist[256 + ((key[i] >> (sh1 - 8)) & 0xffu)], 1);
    __builtin_amdgcn_wave_barrier();
    radix_digit(hist + 256, KC - above1, rd + 2);
    __builtin_amdgcn_wave_barrier();
    tk |= (uint32_t)rd[2] << (sh1 - 8);
    short2 = rd[3] < 0;
  }
  const uint32_t u = (tk & 0x80000000u) ? (tk & 0x7fffffffu) : ~tk;
  return (above1 < 0 || short2) ? -FLT_MAX : fmaxf(__uint_as_float(u), -FLT_MAX);
}

// The general selection (rare: ties leave more candidates than the fast path
// holds, or KC > 64), by all NT threads: the exact top KC content blocks by an
// MSB-first radix select over the 32-bit keys of the sanitised scores,
// re-read from memory (four 8-bit passes), the blocks at the boundary key
// taken lowest block first; the KC selected (score, block) keys are sorted
// descending and emit(r, block) is called for every rank r < KC.  Plain loops
// keep the path small.  KC <= kSortCap and KC <= the number of content blocks.
template <int NT, int IPT, int D, typename Emit>
__device__ void select_general(StepLds<NT, D>& L, const float* srow, int sp, int c_lo, int c_hi, int base, int KC,
                               Emit&& emit) {
  const int tid = threadIdx.x;
  auto score = [&](int i) { return sanitize(srow[min(base + i, sp - 1)]); };
  auto is_c = [&](int i) { return base + i >= c_lo && base + i < c_hi; };
  auto key32 = [&](int i) { return (uint32_t)(sel_key(score(i), 0) >> 32); };
  uint32_t prefix = 0;
  int need = KC;
#pragma unroll 1
  for (int pass = 0; pass < 4; ++pass) {
    const int sh = 24 - 8 * pass;
    for (int j = tid; j < 256; j += NT) L.hist[j] = 0;
    lds_barrier();
#pragma unroll 1
    for (int i = 0; i < IPT; ++i) {
      if (!is_c(i)) continue;
      const uint32_t k = key32(i);
      if (pass == 0 || (k >> (sh + 8)) == prefix) atomicAdd(&L.hist[(k >> sh) & 255u], 1);
    }
    lds_barrier();
    if (tid < kWave) radix_digit(L.hist, need, L.rd);
    lds_barrier();
    prefix = (prefix << 8) | (uint32_t)L.rd[0];
    need -= L.rd[1];
  }
  // prefix is the boundary key: every block above it and the lowest-index
  // `need` of the blocks equal to it
  int n_eq = 0;
#pragma unroll 1
  for (int i = 0; i < IPT; ++i) n_eq += (is_c(i) && key32(i) == prefix) ? 1 : 0;
  int tot;
  const int eq_before = block_excl_scan<NT>(n_eq, L.sc, &tot);
  int n_sel = 0;
  {
    int e = eq_before;
#pragma unroll 1
    for (int i = 0; i < IPT; ++i) {
      if (!is_c(i)) continue;
      const uint32_t k = key32(i);
      if (k > prefix) ++n_sel;
      else if (k == prefix) n_sel += (e++ < need) ? 1 : 0;
    }
  }
  int o = block_excl_scan<NT>(n_sel, L.sc, &tot);   // tot == KC
  {
    int e = eq_before;
#pragma unroll 1
    for (int i = 0; i < IPT; ++i) {
      if (!is_c(i)) continue;
      const uint32_t k = key32(i);
      const bool take = k > prefix || (k == prefix && e++ < need);
      if (take && o < kSortCap) L.keys[o++] = sel_key(score(i), base + i);
    }
  }
  const int n = next_pow2(max(tot, 1));
  for (int i = tot + tid; i < n; i += NT) L.keys[i] = 0;
  __syncthreads();
  bitonic_desc<NT>(L.keys, n);
  for (int r = tid; r < KC; r += NT) emit(r, key_index(L.keys[r]));
}

// The KC-th largest of one value per lane (x), by repeated wave maxima that
// remove one occurrence each; -FLT_MAX when fewer than KC values are finite
// (> -inf).  Every lane receives it.  x is never NaN (pool entries are
// sanitized scores or -inf), so the rounds compare order-preserving unsigned
// keys: an integer maximum fuses with its DPP move and needs none of the NaN
// canonicalisation of a float maximum, and each round's maximum is read into
// a scalar register so the loop runs on scalar control.  (The keys order -0
// below +0 where floats compare them equal; the returned value compares
// equal either way.)
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  auto mx = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  x = mx(x, __float_as_uint(dpp_mov<0xB1>(__uint_as_float(x))));
  x = mx(x, __float_as_uint(dpp_mov<0x4E>(__uint_as_float(x))));
  x = mx(x, __float_as_uint(dpp_mov<0x141>(__uint_as_float(x))));
  x = mx(x, __float_as_uint(dpp_mov<0x140>(__uint_as_float(x))));
  LanePair p = swap16(__uint_as_float(x));
  x = mx(__float_as_uint(p.a), __float_as_uint(p.b));
  p = swap32(__uint_as_float(x));
  return mx(__float_as_uint(p.a), __float_as_uint(p.b));
}
__device__ __forceinline__ float kth_of_lanes(float x, int KC) {
  const int lane = threadIdx.x & (kWave - 1);
  constexpr uint32_t kNegInf = 0x007fffffu;     // the key of -inf; 0 marks a removed lane
  const uint32_t ux = __float_as_uint(x);
  uint32_t key = (ux & 0x80000000u) ? ~ux : (ux | 0x80000000u);
  uint32_t kth = kNegInf;
  int found = 0;
  for (int r = 0; r < KC; ++r) {
    const uint32_t wm = __builtin_amdgcn_readfirstlane(wave_max_u32(key));
    if (wm <= kNegInf) break;
    const uint64_t holders = __ballot(key == wm);
    if (lane == (int)__builtin_ctzll(holders)) key = 0u;
    kth = wm;
    ++found;
  }
  if (found != KC) return -FLT_MAX;
  return fmaxf(__uint_as_float((kth & 0x80000000u) ? (kth & 0x7fffffffu) : ~kth), -FLT_MAX);
}

__device__ __forceinline__ int wave_min_int(int x) {
  auto mn = [](int a, int b) { return a < b ? a : b; };
  x = mn(x, __float_as_int(dpp_mov<0xB1>(__int_as_float(x))));
  x = mn(x, __float_as_int(dpp_mov<0x4E>(__int_as_float(x))));
  x = mn(x, __float_as_int(dpp_mov<0x141>(__int_as_float(x))));
  x = mn(x, __float_as_int(dpp_mov<0x140>(__int_as_float(x))));
  LanePair p = swap16(__int_as_float(x));
  x = mn(__float_as_int(p.a), __float_as_int(p.b));
  p = swap32(__int_as_float(x));
  return mn(__float_as_int(p.a), __float_as_int(p.b));
}

template <int KVDT, int D, int NT, int IPT>
__global__ __launch_bounds__(NT) void select_decode_kernel(FusedArgs fa) {
  warm_kernargs<sizeof(FusedArgs) + 8>();
  constexpr int NW = NT / kWave;
  constexpr int NT16 = TileShape<D>::NT16;
  using Mask = MaskT<IPT>;
  constexpr Mask kOne = 1;
  constexpr int kPool = 9;                   // candidate entries per lane: 4 sub-chunks x 2, one appended row
  __shared__ __align__(16) StepLds<NT, D> L;
  extern __shared__ double s_w[];            // [Hq] budget weights of the sequence's heads

  const SelectArgs& a = fa.s;
  const DecodeArgs& d = fa.d;
  // XCD-aware placement: workgroups are dealt to the 8 XCDs in turn (linear id
  // mod 8), so linear id i takes position (i mod 8) * n/8 + i / 8 of the
  // (sequence, q-head) order: each XCD holds consecutive q-heads -- the heads
  // of a KV group, whose sink, local and shared blocks then meet in one L2.
  int h, b;
  {
    const int n = gridDim.x * gridDim.y, i = blockIdx.y * gridDim.x + blockIdx.x;
    const int pos = (n & 7) == 0 ? (i & 7) * (n >> 3) + (i >> 3) : i;
    // (uniform values kept in scalar registers: a length loaded from memory
    // or a division expanded on the vector unit would otherwise drag every
    // bound and address derived from it onto the vector unit)
    h = __builtin_amdgcn_readfirstlane(mod_u(pos, gridDim.x));
    b = __builtin_amdgcn_readfirstlane(div_u(pos, gridDim.x));
  }
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wu = __builtin_amdgcn_readfirstlane(tid / kWave);   // the wave index, provably uniform
  const int col = lane & 15, grp = lane >> 4;
  const int Hq = a.Hq;
  const int len = __builtin_amdgcn_readfirstlane(seq_len_of(a.seq_lens, a.uniform_len, b));
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

  // ---- 0. loads, each with its index clamped in bounds ----
  // (a) the softmax partials of this lane's head: head tid / LPH, records hl, hl + LPH, ...
  const int first_app = a.n_new > 0 ? div_p2(max(len - a.n_new, 0), a.bs, a.bs_shift) : nb;
  const int rows_in_chunks = min(nb, first_app);
  const int n_ck = (rows_in_chunks + a.chunk_rows - 1) >> a.chunk_shift;   // records per head
  const int n_extra = nb - rows_in_chunks;                                 // rows no record covers
  const int LPH = lanes_per_head<kWeightLanes>(Hq);
  const int hl = tid & (LPH - 1);
  const float* parts_b = a.parts + (int64_t)b * Hq * a.parts_pitch * kPartFloats;
  const float* scores_b = a.scores + (int64_t)b * Hq * a.sp;
  // (records group-major: a wave's loads of one group of consecutive records
  // are contiguous.  Every load of this phase is unconditional, its index
  // clamped in bounds: the compiler counts outstanding loads per path and, where
  // paths join, waits as if the fewest had been issued, so one load under a
  // branch before the tile loads makes the first use of the records wait for
  // the tiles too)
  auto rec4 = [&](int hh, int j, int g) {    // 16-byte group g of record j of head hh
    return *reinterpret_cast<const float4*>(parts_b + ((int64_t)(hh * kPartGroups + g) * a.parts_pitch +
                                                       min(j, max(n_ck - 1, 0))) * 4);
  };
  auto extra = [&](int hh, int e) { return scores_b[hh * a.sp + min(rows_in_chunks + e, nb - 1)]; };
  const int hh0 = div_u(tid, LPH);
  const int hs0 = min(hh0, Hq - 1);
  float4 R[kRecsUpFront];
#pragma unroll
  for (int u = 0; u < kRecsUpFront; ++u) R[u] = rec4(hs0, hl + LPH * u, 0);
  const float X0 = extra(hs0, hl);
  // the nucleus policy's weights, written by the nucleus kernel before this launch
  const double W0 = a.wbuf[(int64_t)b * Hq + min(tid, Hq - 1)];
  __builtin_amdgcn_sched_barrier(0);
  // (b) this head's candidate pool (every wave holds all of it): lane l the
  //     top two of the 4 sub-chunks of record l, their bounds, and appended
  //     row l (the pool serves heads with at most 64 records)
  const bool pool_ok = n_ck <= kWave && n_extra <= kWave;
  const float4 C1 = rec4(h, lane, 1), C2 = rec4(h, lane, 2), C3 = rec4(h, lane, 3), C4 = rec4(h, lane, 4);
  const float XE = extra(h, lane);
  // (b') the 512-thread kernel serves large budgets, whose heads mostly take
  //      the full selection: this head's scores are loaded now (thread t owns
  //      blocks [t*IPT, (t+1)*IPT)) rather than after the count
  constexpr bool kPreScores = NT == 512;
  float vpre[kPreScores ? IPT : 1];
  if constexpr (kPreScores) {
    const float* srow = scores_b + h * a.sp;
#pragma unroll
    for (int i = 0; i < IPT; i += 4) {
      const float4 f = *reinterpret_cast<const float4*>(srow + min(tid * IPT + i, a.sp - 4));
      vpre[i] = f.x; vpre[i + 1] = f.y; vpre[i + 2] = f.z; vpre[i + 3] = f.w;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // (c) the query (same 16-bit type as K, 16-byte aligned rows): 16 bytes per
  //     thread of the first D / 8, stored to LDS at the end of phase 1 (a store
  //     now would wait for this wave's loads before its tile loads issue)
  const uint4 qv = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(d.q) + (int64_t)b * d.qsb +
                                                   (int64_t)h * d.qsh + 8 * (tid & (D / 8 - 1)));
  __builtin_amdgcn_sched_barrier(0);
  // (d) the decode's items: item j is 16-token sub-tile j % n_sub of list
  //     entry j / n_sub; entries [0, nf) are the sink then the local blocks
  //     (the table row's order), later ones the content blocks by rank.  The
  //     first PF items of this wave, when forced, are loaded now; a wave with
  //     fewer forced items re-reads the last forced one (cache hits), so that
  //     the load count is the same on every path)
  const int n_sub = (a.bs + 15) >> 4;
  const int nf_items = nf * n_sub;
  const int64_t head_off = ((int64_t)b * d.sb + (int64_t)div_u(h, d.G) * d.sh + (D / 4) * grp) * 2;
  const char* kbase = reinterpret_cast<const char*>(d.k) + head_off;
  const char* vbase = reinterpret_cast<const char*>(d.v) + head_off;
  const int64_t row_bytes = d.ss * 2;
  auto tokens = [&](int blk, int sub, int& t0, int& t_hi) {
    t0 = blk * a.bs + sub * 16;
    t_hi = min(min(blk * a.bs + a.bs, len), t0 + 16);
  };
  auto forced_block = [&](int e) { return e < bb.sink ? e : local_lo + (e - bb.sink); };
  // PF forced items per wave are prefetched (one with 512 threads: 8 waves
  // cover the usual sink + local count, and two waves per SIMD halve the
  // register file)
  constexpr int PF = NT == 256 ? 2 : 1;
  TileBuf<D> P0, P1;
  int p00 = 0, p01 = 1, p10 = 0, p11 = 1;
  auto forced_item = [&](int j, int& t0, int& t_hi) {      // j clamped to the forced items
    j = min(j, max(nf_items - 1, 0));
    tokens(min(forced_block(div_u(j, n_sub)), nb - 1), mod_u(j, n_sub), t0, t_hi);
  };
  if constexpr (PF >= 1) {
    forced_item(wu, p00, p01);
    tile_load<D>(kbase, vbase, row_bytes, p00, p01, P0);
  }
  if constexpr (PF >= 2) {
    forced_item(wu + NW, p10, p11);
    tile_load<D>(kbase, vbase, row_bytes, p10, p11, P1);
  }
  __builtin_amdgcn_sched_barrier(0);
  const double lognb = a.seq_lens == nullptr ? a.lognb_uniform : log((double)max(nb, 2));

  // ---- 1. the candidate pool's first NW ranks on the pool wave, the weights of
  //      every head on waves 0..2 (two independent chains on separate SIMDs) ----
  // The pool: entries (score, block) of this lane; every content block outside
  // it scores at most the largest bound of its sub-chunk.  Set up by the pool
  // wave here, by another wave only when it needs more ranks (phase 3).
  float pv[kPool];
  int pr[kPool];
  float bound = -INFINITY, lm = -INFINITY;
  int lr = 0x7fffffff;
  auto pool_setup = [&]() {
    const bool rl = lane < n_ck;
    const float v1[4] = {C1.x, C1.y, C1.z, C1.w}, v2[4] = {C2.x, C2.y, C2.z, C2.w};
    const float v3[4] = {C3.x, C3.y, C3.z, C3.w};
    const uint32_t rr[4] = {__float_as_uint(C4.x), __float_as_uint(C4.y), __float_as_uint(C4.z), __float_as_uint(C4.w)};
    bound = -INFINITY;
#pragma unroll
    for (int sc = 0; sc < 4; ++sc) {
      pv[2 * sc] = rl ? v1[sc] : -INFINITY;
      pv[2 * sc + 1] = rl ? v2[sc] : -INFINITY;
      pr[2 * sc] = (int)(rr[sc] & 0xffffu);
      pr[2 * sc + 1] = (int)(rr[sc] >> 16);
      bound = fmaxf(bound, rl ? v3[sc] : -INFINITY);
    }
    const int re = rows_in_chunks + lane;
    pv[8] = (lane < n_extra && re >= c_lo && re < c_hi) ? sanitize(XE) : -INFINITY;
    pr[8] = re;
    bound = wave_allreduce(bound, OpMax());
    // lane maximum (score, then lowest block among equal scores)
    lm = pv[0];
#pragma unroll
    for (int e = 1; e < kPool; ++e) lm = fmaxf(lm, pv[e]);
    lr = 0x7fffffff;
#pragma unroll
    for (int e = 0; e < kPool; ++e) lr = (pv[e] == lm && pr[e] < lr) ? pr[e] : lr;
  };
  // Ranks of the pool's top K: the candidates are the entries >= the K-th
  // largest lane maximum (at least K of them, the top K among them),
  // compacted in lane order into this wave's LDS list, then lane c holds
  // candidate c's key and rank.  Returns the number of candidates (-1: more
  // than a wave holds).
  uint64_t pk = 0;
  int prank = 1 << 30;
  auto pool_rank = [&](int K) -> int {
    const float tau = kth_of_lanes(lm, K);
    int c = 0;
#pragma unroll
    for (int e = 0; e < kPool; ++e) c += (pv[e] >= tau && pv[e] != -INFINITY) ? 1 : 0;
    const int incl = wave_incl_scan(c);
    const int n_c = __builtin_amdgcn_readlane(incl, kWave - 1);
    if (n_c > kWave) return -1;
    if (c == 1) {
      L.cand[wu][incl - 1] = sel_key(lm, lr);        // the lane maximum is its one candidate
    } else if (c > 1) {
      int o = incl - c;
#pragma unroll
      for (int e = 0; e < kPool; ++e)
        if (pv[e] >= tau && pv[e] != -INFINITY) L.cand[wu][o++] = sel_key(pv[e], pr[e]);
    }
    __builtin_amdgcn_wave_barrier();                  // this wave's LDS writes are read back in order
    pk = lane < n_c ? L.cand[wu][lane] : 0ull;
    int r = 0;
    for (int j = 0; j < n_c; ++j) r += readlane_u64(pk, j) > pk;
    prank = lane < n_c ? r : 1 << 30;
    __builtin_amdgcn_wave_barrier();                  // reads done before the list is rewritten
    return n_c;
  };
  // this wave's content tile of the decode: rank rho (content item rho is item
  // nf_items + rho, on wave (nf_items + rho) % NW), loaded once the ranks are known
  const int rho = (wu - nf_items % NW + NW) % NW;
  int n_pre = -1;
  TileBuf<D> CA;
  int ca0 = 0, ca1 = 1, cablk = -1;
  auto prefetch_content = [&]() {
    if (n_sub == 1 && rho < n_pre) {
      const uint64_t hit = __ballot(prank == rho);
      cablk = min(max(key_index(readlane_u64(pk, (int)__builtin_ctzll(hit))), 0), nb - 1);
      tokens(cablk, 0, ca0, ca1);
      tile_load<D>(kbase, vbase, row_bytes, ca0, ca1, CA);
    }
  };
  // with entropy weights to compute the pool wave ranks alone; otherwise
  // (fixed budget, nucleus weights from their own kernel) every wave does
  const bool own_pool = !adaptive || wu == kPoolWave;
  if (own_pool && pool_ok) {
    pool_setup();
    n_pre = pool_rank(NW);
    prefetch_content();
    L.pool_pk[lane] = pk;
    L.pool_rank[lane] = prank;
    if (lane == 0) {
      L.pool_n = n_pre;
      L.pool_bound = bound;
    }
  }
  const float tf = (float)fmax(a.cfg.temperature, 1e-6);
  // A head's softmax partial over its records and appended rows: each lane
  // merges its up-front records against their common maximum (independent
  // exponentials), then the rest one by one, then the lane group.
  auto merge_head = [&](int hh, const float4 (&Q)[kRecsUpFront], float X) {
    const bool on = hh < Hq;
    SoftPart pt = soft_empty();
    if (on) {
      const float zx = hl < n_extra ? (tf == 1.f ? X : __fdiv_rn(X, tf)) : -INFINITY;
      float M = zx;
#pragma unroll
      for (int u = 0; u < kRecsUpFront; ++u)
        if (hl + LPH * u < n_ck) M = fmaxf(M, Q[u].x);
      if (M != -INFINITY) {
        float S = 0.f, T = 0.f;
#pragma unroll
        for (int u = 0; u < kRecsUpFront; ++u)
          if (hl + LPH * u < n_ck && Q[u].x != -INFINITY) {
            const float dm = Q[u].x - M, f = __expf(dm);
            S = fmaf(Q[u].y, f, S);
            T = fmaf(f, fmaf(dm, Q[u].y, Q[u].z), T);
          }
        if (zx != -INFINITY) {
          const float dz = zx - M, f = __expf(dz);
          S += f;
          T = fmaf(f, dz, T);
        }
        pt = SoftPart{M, S, T};
      }
      // long contexts: kRecsUpFront more records per lane at a time, their
      // loads issued together
      for (int j0 = hl + LPH * kRecsUpFront; j0 < n_ck; j0 += LPH * kRecsUpFront) {
        float4 Q2[kRecsUpFront];
#pragma unroll
        for (int u = 0; u < kRecsUpFront; ++u) Q2[u] = rec4(hh, j0 + LPH * u, 0);
#pragma unroll
        for (int u = 0; u < kRecsUpFront; ++u)
          if (j0 + LPH * u < n_ck) pt = soft_merge(pt, SoftPart{Q2[u].x, Q2[u].y, Q2[u].z});
      }
      for (int e = hl + LPH; e < n_extra; e += LPH) {
        const float x = extra(hh, e);
        pt = soft_merge(pt, SoftPart{tf == 1.f ? x : __fdiv_rn(x, tf), 1.f, 0.f});
      }
    }
    switch (LPH) {                          // uniform
      case 16: pt = soft_group_merge<16>(pt); break;
      case 8: pt = soft_group_merge<8>(pt); break;
      case 4: pt = soft_group_merge<4>(pt); break;
      case 2: pt = soft_group_merge<2>(pt); break;
      default: break;
    }
    if (on && hl == 0) s_w[hh] = entropy_weight(pt, lognb);
  };
  if (adaptive) {
    if (wu < kPoolWave) {
      merge_head(hh0, R, X0);
      for (int p = 1; p * div_u(kWeightLanes, LPH) < Hq; ++p) {    // more heads than the weight lanes hold
        const int hh = p * div_u(kWeightLanes, LPH) + div_u(tid, LPH);
        const int hs = min(hh, Hq - 1);
        float4 Q[kRecsUpFront];
#pragma unroll
        for (int u = 0; u < kRecsUpFront; ++u) Q[u] = rec4(hs, hl + LPH * u, 0);
        merge_head(hh, Q, extra(hs, hl));
      }
    }
  } else if (nucleus) {
    if (tid < Hq) s_w[tid] = W0;
    for (int hh = tid + NT; hh < Hq; hh += NT) s_w[hh] = a.wbuf[(int64_t)b * Hq + hh];
  }
  if (tid < D / 8) *reinterpret_cast<uint4*>(&L.q[8 * tid]) = qv;
  lds_barrier();
  // the other waves take the pool wave's ranks and prefetch their content tiles
  if (!own_pool && pool_ok) {
    n_pre = L.pool_n;
    bound = L.pool_bound;
    pk = L.pool_pk[lane];
    prank = L.pool_rank[lane];
    prefetch_content();
  }

  // ---- 2. the head's count (every wave) ----
  const bool weighted = adaptive || nucleus;
  const double wsum = !weighted ? 0.0 : Hq <= 128 ? wave_pairwise_sum(s_w, Hq) : numpy_pairwise_sum<6>(s_w, Hq);
  const int k = min(head_count(bb, a.cfg.policy, weighted ? s_w[h] : 0.0, wsum, Hq), a.T);
  const int KC = max(k - nf, 0);
  if (tid == 0) {
    if (d.sel_lens_out) d.sel_lens_out[(int64_t)b * Hq + h] = k;
    if (adaptive) a.wbuf[(int64_t)b * Hq + h] = s_w[h];
  }
  for (int j = tid; j < nf; j += NT) trow[j] = forced_block(j);
  for (int j = k + tid; j < a.T; j += NT) trow[j] = -1;

  // ---- 3. the content selection ----
  // pool path: the top KC of the pool, exact when no content block outside
  // it can rank among them: every bound below the KC-th score
  bool use_pool = false;
  if (KC > 0 && pool_ok && KC <= kFastKC) {
    int n_c = n_pre;
    if (KC > NW) {
      if (!own_pool) pool_setup();
      n_c = pool_rank(KC);
    }
    if (n_c >= KC) {
      const uint64_t hit = __ballot(prank == KC - 1);
      const uint64_t kth = readlane_u64(pk, (int)__builtin_ctzll(hit));
      const uint32_t u = (uint32_t)(kth >> 32);     // the KC-th score, back from its order-preserving bits
      const float v_kth = __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
      use_pool = bound < v_kth;
    }
    if (use_pool && wu == 0 && prank < KC) trow[nf + prank] = key_index(pk);
  }
  // full path: every score of the head (thread t owns blocks [t*IPT,
  // (t+1)*IPT)); the ranked candidates (ck, cr) or the general selection's list
  constexpr int kBig = 1 << 30;
  bool fast = false, split = false;
  uint64_t ck0 = 0, ck1 = 0;
  int cr0 = kBig, cr1 = kBig;
  if (KC > 0 && !use_pool) {
    const int base = tid * IPT;
    float v[IPT];
    if constexpr (kPreScores) {
#pragma unroll
      for (int i = 0; i < IPT; ++i) v[i] = vpre[i];
    } else {
      const float* srow = scores_b + h * a.sp;
#pragma unroll
      for (int i = 0; i < IPT; i += 4) {
        const float4 f = *reinterpret_cast<const float4*>(srow + min(base + i, a.sp - 4));
        v[i] = f.x; v[i + 1] = f.y; v[i + 2] = f.z; v[i + 3] = f.w;
      }
    }
    Mask content;
    float vmax;
    if (base >= c_lo && base + IPT <= c_hi) {
      // every block of the thread is content: sanitize() of the plain maximum
      // (fmaxf skips NaN, which sanitize() maps to its lowest value anyway)
      float mx = v[0];
#pragma unroll
      for (int i = 1; i < IPT; ++i) mx = fmaxf(mx, v[i]);
      vmax = sanitize(mx);
      content = (Mask)~Mask(0) >> (8 * sizeof(Mask) - IPT);
    } else {
      content = 0;
      vmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < IPT; ++i) {
        const bool is_c = base + i >= c_lo && base + i < c_hi;
        if (is_c) content |= kOne << i;
        vmax = fmaxf(vmax, is_c ? sanitize(v[i]) : -INFINITY);
      }
    }
    L.maxv[tid] = vmax;
    lds_barrier();
    fast = KC <= kRadixKC;
    if (fast) {
      float tau;
      if (KC <= kFastKC) {
        tau = kth_largest<NT>(L.maxv, NT, KC);
      } else {
        if (wu == 0) {
          const float t = kth_largest_radix<NT>(L.maxv, KC, L.hist, L.rd);
          if (lane == 0) L.tau = t;
        }
        lds_barrier();
        tau = L.tau;
      }
      Mask cm = 0;
      if (vmax >= tau) {
        if (tau == -FLT_MAX) {               // the bottom of the range: compare sanitised scores
#pragma unroll
          for (int i = 0; i < IPT; ++i) cm |= (sanitize(v[i]) >= tau) ? (kOne << i) : Mask(0);
        } else {
#pragma unroll
          for (int i = 0; i < IPT; ++i) cm |= (v[i] >= tau) ? (kOne << i) : Mask(0);
        }
        cm &= content;
      }
      // per-wave compaction in lane order (the same order on every run)
      constexpr int kCap = kCandLanes * kWave;
      const int c = popcnt(cm);
      const int incl = wave_incl_scan(c);
      const int wtot = __builtin_amdgcn_readlane(incl, kWave - 1);
      if (wtot <= kCap && c == 1) {
        // one candidate: it is the thread's largest content score (that is >= tau)
        L.cand[wu][incl - 1] = sel_key(vmax, base + (int)__builtin_ctzll((uint64_t)cm));
      } else if (wtot <= kCap && c > 1) {   // ties and close scores: rare
        int o = incl - c;
#pragma unroll
        for (int i = 0; i < IPT; ++i)
          if ((cm >> i) & kOne) L.cand[wu][o++] = sel_key(sanitize(v[i]), base + i);
      }
      if (lane == 0) L.wn[wu] = wtot <= kCap ? wtot : -1;
      lds_barrier();
      int n_cand = 0;
      bool over = false;
      int wn[NW];
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) {
        wn[ww] = L.wn[ww];
        over = over || wn[ww] < 0;
        n_cand += max(wn[ww], 0);
      }
      fast = !over && n_cand <= kCap;
      // (the split ranking below in the 512-thread kernel of large budgets,
      // where eight waves would each rank every candidate: measured at
      // avg_budget 32, 29.3 -> 28.2 us per step; in the 256-thread kernel of
      // small budgets its code cost the step ~0.1 us)
      split = NT == 512 && fast;
      if (fast && !split) {
        // every wave ranks all candidates in registers (candidate c on lane
        // c % 64 of ck0 / ck1; the block of rank r a ballot away)
        auto fetch = [&](int idx) -> uint64_t {   // candidate idx of the concatenated lists
          int src = 0;
#pragma unroll
          for (int ww = 0; ww < NW - 1; ++ww)
            if (src == ww && idx >= wn[ww]) { idx -= wn[ww]; src = ww + 1; }
          return L.cand[src][min(idx, kCap - 1)];
        };
        ck0 = lane < n_cand ? fetch(lane) : 0ull;
        ck1 = lane + kWave < n_cand ? fetch(lane + kWave) : 0ull;
        int r0 = 0, r1 = 0;
        const int n0 = min(n_cand, kWave);
        for (int j = 0; j < n0; ++j) {
          const uint64_t kj = readlane_u64(ck0, j);
          r0 += kj > ck0;
          r1 += kj > ck1;
        }
        for (int j = kWave; j < n_cand; ++j) {
          const uint64_t kj = readlane_u64(ck1, j - kWave);
          r0 += kj > ck0;
          r1 += kj > ck1;
        }
        cr0 = lane < n_cand ? r0 : kBig;
        cr1 = lane + kWave < n_cand ? r1 : kBig;
        if (wu == 0) {
          if (cr0 < KC) trow[nf + cr0] = key_index(ck0);
          if (cr1 < KC) trow[nf + cr1] = key_index(ck1);
        }
      } else if (fast) {
        // Many candidates: their exact ranks split over the waves (every wave
        // ranking every candidate cost up to 128 dependent readlane steps
        // per wave): the per-wave lists are first made one contiguous list
        // in L.keys; lane (c, part) of wave w then takes candidate w*CPW + c
        // and counts the keys of its part of the list above it; the parts'
        // counts meet through the lane swaps; the block of rank r goes to
        // L.list[r] (and to the table for r < KC).
        constexpr int CPW = kCap / NW;              // candidates per wave
        constexpr int PARTS = kWave / CPW;          // lane groups per candidate
        static_assert(CPW * NW == kCap && PARTS * CPW == kWave && (PARTS == 2 || PARTS == 4), "rank split");
        int off = 0;
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) off += ww < wu ? wn[ww] : 0;
        if (lane < wn[wu]) L.keys[off + lane] = L.cand[wu][lane];
        if (lane + kWave < wn[wu]) L.keys[off + lane + kWave] = L.cand[wu][lane + kWave];
        lds_barrier();
        const int c_local = lane % CPW, part = lane / CPW;
        const int ci = wu * CPW + c_local;
        const uint64_t key = L.keys[min(ci, kCap - 1)];
        const int per = (n_cand + PARTS - 1) / PARTS;
        const int j1 = min((part + 1) * per, n_cand);
        int r = 0;
        for (int j = part * per; j < j1; ++j) r += L.keys[j] > key;
        {
          LanePair q = swap32(__int_as_float(r));
          r = __float_as_int(q.a) + __float_as_int(q.b);
          if constexpr (PARTS == 4) {
            q = swap16(__int_as_float(r));
            r = __float_as_int(q.a) + __float_as_int(q.b);
          }
        }
        if (part == 0 && ci < n_cand) {
          L.list[r] = key_index(key);
          if (r < KC) trow[nf + r] = key_index(key);
        }
        lds_barrier();
      }
    }
    if (!fast) {
      select_general<NT, IPT, D>(L, scores_b + h * a.sp, a.sp, c_lo, c_hi, base, KC, [&](int r, int blk) {
        L.list[r] = blk;
        trow[nf + r] = blk;
      });
      lds_barrier();
    }
  }

  // ---- 4. flash-decode over the k blocks ----
  // the query as the B operand of S^T: lane (col, grp) holds
  // q[D/4*grp + 8*s .. +7] in every column (columns other than 0 are masked
  // out of the softmax)
  uint4 qf[D / 32];
#pragma unroll
  for (int s2 = 0; s2 < D / 32; ++s2) qf[s2] = *reinterpret_cast<const uint4*>(&L.q[(D / 4) * grp + 8 * s2]);
  TileState<D> st;
  tile_init(st);
  {
    uint32_t* vt = L.vt + wu * TileShape<D>::VT_WORDS;
    const float scale = d.scale_log2;
    bool started = false;                    // uniform: a tile is in the accumulators
    auto compute = [&](int t0, int t_hi, const TileBuf<D>& r) {
      tile_update<KVDT, D>(st, r, qf, vt, t0, t_hi, col == 0, scale, started);
      started = true;
    };
    auto load_compute = [&](int blk, int sub) {
      TileBuf<D> X;
      int x0, x1;
      tokens(blk, sub, x0, x1);
      tile_load<D>(kbase, vbase, row_bytes, x0, x1, X);
      __builtin_amdgcn_sched_barrier(0);
      compute(x0, x1, X);
    };
    // (a) the forced items wu, wu + NW, ... (the first two loaded in phase 0)
    const int n_items = k * n_sub;
    const bool f0 = PF >= 1 && wu < n_items && wu < nf_items;
    const bool f1 = PF >= 2 && wu + NW < n_items && wu + NW < nf_items;
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PF >= 1) {
      if (f0) compute(p00, p01, P0);
    }
    if constexpr (PF >= 2) {
      if (f1) compute(p10, p11, P1);
    }
    for (int j = wu + PF * NW; j < min(nf_items, n_items); j += NW) load_compute(forced_block(div_u(j, n_sub)), mod_u(j, n_sub));
    // (b) the content blocks: item i (sub-tile i % n_sub of the block of rank
    // i / n_sub) on wave (nf_items + i) % NW, so this wave's are rho, rho + NW,
    // ...; the block of a rank is a ballot away in the pool and fast paths
    // (every wave holds all ranked candidates), in LDS for the general one
    auto block_of = [&](int r) -> int {
      if (use_pool) {
        const uint64_t hit = __ballot(prank == r);
        return key_index(readlane_u64(pk, hit ? (int)__builtin_ctzll(hit) : 0));
      }
      if (fast && !split) {
        const uint64_t h0 = __ballot(cr0 == r);
        if (h0) return key_index(readlane_u64(ck0, (int)__builtin_ctzll(h0)));
        const uint64_t h1 = __ballot(cr1 == r);
        return key_index(readlane_u64(ck1, h1 ? (int)__builtin_ctzll(h1) : 0));
      }
      return L.list[r];                      // split fast path and general path
    };
    // up to three tiles in flight: item n + 3's load is issued right after
    // item n's compute; the first item may be the tile prefetched before the
    // count
    auto fetch = [&](int it, TileBuf<D>& T, int& t0, int& t1) {
      const int blk = block_of(div_u(it, n_sub));
      if (it == rho && n_sub == 1 && blk == cablk) {
        T = CA;
        t0 = ca0;
        t1 = ca1;
      } else {
        tokens(blk, mod_u(it, n_sub), t0, t1);
        tile_load<D>(kbase, vbase, row_bytes, t0, t1, T);
      }
    };
    constexpr int kRing = 3;
    const int n_ci = KC * n_sub;
    TileBuf<D> R[kRing];
    int r0[kRing], r1[kRing];
#pragma unroll
    for (int u = 0; u < kRing; ++u) {
      r0[u] = 0;
      r1[u] = 1;
      if (rho + u * NW < n_ci) fetch(rho + u * NW, R[u], r0[u], r1[u]);
    }
    for (int base = rho; base < n_ci; base += kRing * NW) {
#pragma unroll
      for (int u = 0; u < kRing; ++u) {
        const int it = base + u * NW;
        if (it < n_ci) {
          __builtin_amdgcn_sched_barrier(0);
          compute(r0[u], r1[u], R[u]);
          if (it + kRing * NW < n_ci) fetch(it + kRing * NW, R[u], r0[u], r1[u]);
        }
      }
    }
  }
  tile_finish(st);
  if (lane == 0) {
    L.m[wu] = st.m_h;
    L.l[wu] = st.l_h;
  }
  if (grp == 0) {
#pragma unroll
    for (int n = 0; n < NT16; ++n) L.acc[wu][n * 16 + col] = st.acc[n][0];   // O[head 0][16n + col]
  }
  lds_barrier();
  for (int i = tid; i < D; i += NT) {
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, L.m[ww]);
    float Ls = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int ww = 0; ww < NW; ++ww) {
        const float f = L.m[ww] == -INFINITY ? 0.f : exp2f(L.m[ww] - M);
        Ls += L.l[ww] * f;
        O += L.acc[ww][i] * f;
      }
    }
    store_elt(d.out, d.odt, oo + i, O / Ls);   // no block at all: 0/0 as the reference kernel
  }
}

// Threads and scores per thread for a row bound and the budget's mean count
// avg: 256 threads up to 16 scores each (4096 blocks); up to 8192 blocks,
// 256 threads with 32 when avg <= kWideBudget (a few content tiles per head:
// four waves, fewer barrier partners), else 512 threads with 16 (eight waves
// halve a large budget's serial decode); 512 threads with 32 up to 16384
// blocks; {0, 0}: not served.  Measured at 128K: avg 8, 17.9 us with 256
// threads against 18.7 with 512; avg 32, 40.6 against 30.2.
constexpr double kWideBudget = 12.0;
struct StepShape { int nt, ipt; };
inline StepShape step_shape(int rows, double avg) {
  for (int ipt = 4; ipt <= 16; ipt *= 2)
    if (rows <= 256 * ipt) return {256, ipt};
  if (rows <= 256 * 32 && avg <= kWideBudget) return {256, 32};
  if (rows <= 512 * 16) return {512, 16};
  if (rows <= 512 * 32) return {512, 32};
  return {0, 0};
}

template <int KVDT, int D, int NT, int IPT>
void launch_one(const FusedArgs& a, hipStream_t s) {
  const dim3 grid(a.s.Hq, a.s.B);
  const size_t dyn = (size_t)a.s.Hq * sizeof(double);
  hipLaunchKernelGGL((select_decode_kernel<KVDT, D, NT, IPT>), grid, dim3(NT), dyn, s, a);
}

template <int KVDT, int D>
hipError_t launch_fd(const FusedArgs& a, int rows, hipStream_t s) {
  const StepShape sh = step_shape(rows, a.s.cfg.avg);
  if (sh.nt == 512) {
    if (sh.ipt == 16) launch_one<KVDT, D, 512, 16>(a, s);
    else launch_one<KVDT, D, 512, 32>(a, s);
  } else {
    switch (sh.ipt) {
      case 4: launch_one<KVDT, D, 256, 4>(a, s); break;
      case 8: launch_one<KVDT, D, 256, 8>(a, s); break;
      case 16: launch_one<KVDT, D, 256, 16>(a, s); break;
      case 32: launch_one<KVDT, D, 256, 32>(a, s); break;
      default: return hipErrorInvalidValue;
    }
  }
  return hipGetLastError();
}

template <int KVDT>
hipError_t launch_fk(const FusedArgs& a, int D, int rows, hipStream_t s) {
  switch (D) {
    case 32: return launch_fd<KVDT, 32>(a, rows, s);
    case 64: return launch_fd<KVDT, 64>(a, rows, s);
    case 128: return launch_fd<KVDT, 128>(a, rows, s);
    default: return hipErrorInvalidValue;
  }
}

template <int NT>
size_t step_lds(int D) {
  switch (D) {
    case 32: return sizeof(StepLds<NT, 32>);
    case 64: return sizeof(StepLds<NT, 64>);
    case 128: return sizeof(StepLds<NT, 128>);
    default: return (size_t)-1;
  }
}

}  // namespace

// The fused kernel serves head_dim <= 128 and up to 16384 blocks; other
// shapes take the three-kernel path.
bool select_decode_supported(int D, int max_blocks, int table_width, int Hq, int sp, int parts_pitch) {
  return D <= 128 && step_shape(max_blocks, 0.0).nt > 0 && table_width <= kSortCap &&
         (int64_t)Hq * sp < (1ll << 31) && (int64_t)Hq * parts_pitch * kPartFloats < (1ll << 31);
}

size_t select_decode_lds(int D, int Hq, int max_blocks, double avg) {
  const StepShape sh = step_shape(max_blocks, avg);
  const size_t st = sh.nt == 512 ? step_lds<512>(D) : step_lds<256>(D);
  if (st == (size_t)-1) return st;
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
