// Ragged block-sparse split-K flash-decode (adakv/kernels/block_sparse_decode.py:51-100)
// and the dense split-K flash-decode baseline.
//
// Grid (split, KV head, sequence).  A workgroup serves the G q-heads of one KV
// head.  Sparse mode first fixes each head's block count -- read from sel_lens,
// or derived from the per-head entropy weights exactly as the budget allocator
// does (every workgroup of the sequence evaluates the same sum of weights, so
// no inter-workgroup hand-off is needed) -- then forms the union of the heads'
// listed blocks as a byte-per-block head bitmap in LDS (duplicates and
// out-of-range ids fall out here) and enumerates it in block order.  A
// sequence's union is split into at most `nsplit` slices of at least
// `min_per` blocks, so the common small selection is served by one workgroup
// and needs no merge.
//
// Streaming, bf16 / fp16 K and V (matrix cores): each wave takes 16-token
// tiles.  S^T = K . Q^T runs on v_mfma_f32_16x16x32 -- K is loaded straight
// into the A-operand layout (lane l holds token l%16 and a contiguous D/2-byte
// slice of its row, so a tile is D/32 coalesced 16-byte loads per lane) and
// the group's q-heads, zero-padded to 16, form the B operand.  The online
// softmax runs on the 16x16 result (4 tokens per lane, the cross-lane max over
// the 4 lane groups by permlane swaps), and O += P . V runs on
// v_mfma_f32_16x16x16 with P taken directly from the S^T result layout and V
// transposed through a per-wave LDS tile.  A 16-token tile costs 3*D/32
// matrix instructions and a few dozen VALU instructions.
//
// Streaming, fp32 K and V (exact-parity mode): VALU dot products, a lane owns
// a 16-byte slice of head_dim of one token row, each group of lanes sharing a
// token row keeps its own online softmax and the row groups are combined once
// at the end.
//
// Several active slices write (m, l, acc[D]) partials; in sparse mode the last
// slice to arrive merges them, in dense mode merge_kernel does.
#include <algorithm>

#include "attend.hpp"
#include "common.hpp"
#include "internal.hpp"

namespace adakv {
namespace {

constexpr int kSparseThreads = 512;
constexpr int kDenseThreads = 256;

// ---------------------------------------------------------------------------
// Prologue: per-head counts and the union list of one (sequence, KV head), and
// this workgroup's slice [lo, hi) of it.
// ---------------------------------------------------------------------------
struct Slice {
  int U, lo, hi, n_active;
};

// The q-heads a workgroup serves: the G heads of one KV head, or (sparse
// per-head mode) a single q-head, which then reads its own selection only.
struct Grp {
  int unit;   // group index within the sequence
  int ng;     // groups per sequence
  int G;      // q-heads in the group
  int h0;     // first q-head of the group
  int kv;     // KV head the group reads
};
__device__ __forceinline__ Grp group_of(const DecodeArgs& a, int x) {
  if (a.per_head) return Grp{x, a.Hq, 1, x, x / a.G};
  return Grp{x, a.Hkv, a.G, x * a.G, x};
}

// Dynamic LDS of the sparse mode: fp64 weights [Hq], the union bitmap (one
// byte of head bits per block, rounded up to whole 16-byte quads), the list.
__device__ __forceinline__ int bitmap_words(int max_blocks) { return ceil_div(ceil_div(max_blocks, 4), 4) * 4; }
__device__ __forceinline__ uint32_t* bitmap_base(const DecodeArgs& a, unsigned char* s_dyn_raw) {
  return reinterpret_cast<uint32_t*>(s_dyn_raw + ((a.Hq * 8 + 15) / 16) * 16);
}
__device__ __forceinline__ uint32_t* list_base(const DecodeArgs& a, unsigned char* s_dyn_raw) {
  return bitmap_base(a, s_dyn_raw) + bitmap_words(a.max_blocks);
}

// Bit 4k + i of the result is set when byte i of word k of the quad is non-zero.
__device__ __forceinline__ uint32_t nonzero_bytes(uint32_t x) {
  x |= x >> 4;
  x |= x >> 2;
  x |= x >> 1;
  x &= 0x01010101u;
  return (x | (x >> 7) | (x >> 14) | (x >> 21)) & 0xfu;
}
__device__ __forceinline__ uint32_t quad_mask(const uint4& q) {
  return nonzero_bytes(q.x) | (nonzero_bytes(q.y) << 4) | (nonzero_bytes(q.z) << 8) | (nonzero_bytes(q.w) << 12);
}

template <int NT>
__device__ Slice build_slice(const DecodeArgs& a, int b, const Grp& gr, int split, int nb,
                             unsigned char* s_dyn_raw, int* s_cnt, int* s_misc) {
  const int tid = threadIdx.x, G = gr.G;
  double* s_w = reinterpret_cast<double*>(s_dyn_raw);
  uint32_t* s_bits = bitmap_base(a, s_dyn_raw);
  uint4* s_quads = reinterpret_cast<uint4*>(s_bits);
  uint32_t* s_list = list_base(a, s_dyn_raw);
  // bitmap quads (16 blocks each) owned by this thread: [q0, q0 + qpt)
  const int nquads = ceil_div(nb, 16);
  const int qpt = ceil_div(nquads, NT), q0 = tid * qpt, q1 = min(q0 + qpt, nquads);
  int U = nb, off = 0;
  if (a.table != nullptr) {
    // The table entries that can be selected are loaded up front (before the
    // counts are known); the counts then decide which of them enter the union.
    const Bounds bb = budget_bounds(nb, a.cfg);
    const bool derive = a.sel_lens == nullptr;
    const bool adaptive = derive && a.cfg.policy != ADAKV_POLICY_FIXED && nb > 1;   // weights in wbuf
    const int width = derive ? min(a.T, max(bb.kcap, 0)) : a.T;
    constexpr int EPT = 4;                       // table entries per thread
    int ent[EPT];
#pragma unroll
    for (int u = 0; u < EPT; ++u) {
      const int e = min(tid + u * NT, max(G * width - 1, 0));   // in bounds; extra entries unused
      ent[u] = a.table[((int64_t)b * a.Hq + gr.h0 + e / width) * a.T + e % width];
    }
    // a single head whose listed blocks are known distinct needs no union:
    // its list is the valid prefix of its own table row
    const bool direct = a.table_unique && G == 1 && width <= NT;
    if (!direct)
      for (int i = tid; i < nquads; i += NT) s_quads[i] = make_uint4(0, 0, 0, 0);
    if (adaptive)
      for (int h = tid; h < a.Hq; h += NT) s_w[h] = a.wbuf[(int64_t)b * a.Hq + h];
    if (!derive && tid < G) s_cnt[tid] = min(max(a.sel_lens[(int64_t)b * a.Hq + gr.h0 + tid], 0), a.T);
    __syncthreads();
    if (derive) {
      if (tid < kWave) {
        // one wave evaluates the sum of weights in NumPy's order
        const double wsum = adaptive ? numpy_pairwise_sum<6>(s_w, a.Hq) : 0.0;
        if (tid < G) {
          const int k = head_count(bb, a.cfg.policy, adaptive ? s_w[gr.h0 + tid] : 0.0, wsum, a.Hq);
          s_cnt[tid] = min(k, a.T);
          if (split == 0 && a.sel_lens_out) a.sel_lens_out[(int64_t)b * a.Hq + gr.h0 + tid] = k;
        }
      }
      __syncthreads();
    }
    if (direct) {
      const int blk = ent[0];
      const bool ok = tid < s_cnt[0] && blk >= 0 && blk < nb;
      off = block_excl_scan<NT>(ok ? 1 : 0, s_misc, &U);
      Slice r;
      r.U = U;
      const int per = U > 0 ? max(ceil_div(U, a.nsplit), a.min_per) : 0;
      r.n_active = U > 0 ? ceil_div(U, per) : 0;
      r.lo = split * per;
      r.hi = min(U, r.lo + per);
      if (ok && off >= r.lo && off < r.hi) s_list[off - r.lo] = (uint32_t)blk | (1u << 24);
      __syncthreads();
      return r;
    }
#pragma unroll
    for (int u = 0; u < EPT; ++u) {
      const int e = tid + u * NT;
      if (e < G * width) {
        const int g = e / width, j = e % width, blk = ent[u];
        if (j < s_cnt[g] && blk >= 0 && blk < nb) atomicOr(&s_bits[blk >> 2], 1u << ((blk & 3) * 8 + g));
      }
    }
    for (int e = EPT * NT + tid; e < G * width; e += NT) {   // tables wider than EPT*NT/G
      const int g = e / width, j = e % width;
      const int blk = a.table[((int64_t)b * a.Hq + gr.h0 + g) * a.T + j];
      if (j < s_cnt[g] && blk >= 0 && blk < nb) atomicOr(&s_bits[blk >> 2], 1u << ((blk & 3) * 8 + g));
    }
    __syncthreads();
    int cnt = 0;
#pragma nounroll
    for (int qi = q0; qi < q1; ++qi) cnt += __popc(quad_mask(s_quads[qi]));
    off = block_excl_scan<NT>(cnt, s_misc, &U);
  }
  Slice r;
  r.U = U;
  const int per = U > 0 ? max(ceil_div(U, a.nsplit), a.min_per) : 0;
  r.n_active = U > 0 ? ceil_div(U, per) : 0;
  r.lo = split * per;
  r.hi = min(U, r.lo + per);
  if (a.table != nullptr && r.lo < r.hi) {
    // list entries in block order: block id | head mask << 24
    int p = off;
#pragma nounroll
    for (int qi = q0; qi < q1 && p < r.hi; ++qi) {
      const uint4 q = s_quads[qi];
      uint32_t m = quad_mask(q);
      while (m) {
        const int j = __builtin_ctz(m);
        m &= m - 1;
        const uint32_t wd = j < 8 ? (j < 4 ? q.x : q.y) : (j < 12 ? q.z : q.w);
        if (p >= r.lo && p < r.hi)
          s_list[p - r.lo] = (uint32_t)(16 * qi + j) | (((wd >> (8 * (j & 3))) & 0xffu) << 24);
        ++p;
      }
    }
  }
  __syncthreads();
  return r;
}

// Block id and head mask of entry e (slice-relative) of the list.
__device__ __forceinline__ void list_entry(const DecodeArgs& a, const Grp& gr, const uint32_t* s_list, int lo,
                                           int e, int& blk, uint32_t& hm) {
  if (a.table == nullptr) {
    blk = lo + e;
    hm = (1u << gr.G) - 1u;
  } else {
    const uint32_t ent = s_list[e];
    blk = (int)(ent & 0xffffffu);
    hm = ent >> 24;
  }
}

__device__ __forceinline__ void write_nan_outputs(const DecodeArgs& a, int b, const Grp& gr, int D, int NT) {
  // no valid block for any head of the group: 0/0, as the reference kernel
  for (int i = threadIdx.x; i < gr.G * D; i += NT)
    store_elt(a.out, a.odt, (int64_t)b * a.osb + (int64_t)(gr.h0 + i / D) * a.osh + i % D,
              __builtin_nanf(""));
}

// ---------------------------------------------------------------------------
// Epilogue: combine the waves' (m, l, acc) through LDS -- s_m, s_l [NW][GMAX],
// s_acc [NW][HC][D] reused for head chunks of HC; stage(g0, n) writes the acc
// of heads g0 .. g0+n-1 of the calling wave -- then write the output (single
// active slice) or this slice's partials; in sparse mode the last slice to
// arrive merges all partials.
// ---------------------------------------------------------------------------
template <int NT, int D, int GMAX, int HC, typename Stage>
__device__ void finish(const DecodeArgs& a, int b, const Grp& gr, int split, const Slice& sl,
                       float (*s_m)[GMAX], float (*s_l)[GMAX], float (*s_acc)[HC][D], int* s_misc,
                       Stage stage) {
  constexpr int NW = NT / kWave;
  const int tid = threadIdx.x, G = gr.G;
  float* part = a.partials + (((int64_t)b * gr.ng + gr.unit) * a.nsplit) * G * (D + 2);
  const int64_t pstride = (int64_t)G * (D + 2);
#pragma unroll
  for (int g0 = 0; g0 < GMAX; g0 += HC) {
    if (g0 >= G) break;                      // uniform over the workgroup
    const int n = min(HC, G - g0);
    stage(g0, n);
    __syncthreads();
    for (int i = tid; i < n * D; i += NT) {
      const int gg = i / D, g = g0 + gg, d = i % D;
      float M = s_m[0][g];
#pragma unroll
      for (int ww = 1; ww < NW; ++ww) M = fmaxf(M, s_m[ww][g]);
      float L = 0.f, O = 0.f;
      if (M != -INFINITY) {
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) {
          const float f = s_m[ww][g] == -INFINITY ? 0.f : exp2f(s_m[ww][g] - M);
          L += s_l[ww][g] * f;
          O += s_acc[ww][gg][d] * f;
        }
      }
      if (sl.n_active == 1) {
        store_elt(a.out, a.odt, (int64_t)b * a.osb + (int64_t)(gr.h0 + g) * a.osh + d, O / L);
      } else {
        float* pg = part + split * pstride + g * (D + 2);
        pg[2 + d] = O;
        if (d == 0) { pg[0] = M; pg[1] = L; }
      }
    }
    __syncthreads();
  }
  if (sl.n_active == 1 || !a.merge_in_kernel) return;

  // sparse: the last active slice merges (at most nsplit <= 16 of them)
  __threadfence();
  __syncthreads();
  if (tid == 0) s_misc[NW] = arrive(&a.counters[(int64_t)b * gr.ng + gr.unit]) == sl.n_active - 1;
  __syncthreads();
  if (!s_misc[NW]) return;
  __threadfence();
  for (int i = tid; i < G * D; i += NT) {
    const int g = i / D, d = i % D;
    const float* pg = part + g * (D + 2);
    float ms[16], ls[16], os[16];
#pragma unroll
    for (int sp = 0; sp < 16; ++sp) {
      const bool ok = sp < sl.n_active;
      ms[sp] = ok ? pg[sp * pstride] : -INFINITY;
      ls[sp] = ok ? pg[sp * pstride + 1] : 0.f;
      os[sp] = ok ? pg[sp * pstride + 2 + d] : 0.f;
    }
    float M = -INFINITY;
#pragma unroll
    for (int sp = 0; sp < 16; ++sp) M = fmaxf(M, ms[sp]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int sp = 0; sp < 16; ++sp) {
        const float f = ms[sp] == -INFINITY ? 0.f : exp2f(ms[sp] - M);
        L += ls[sp] * f;
        O += os[sp] * f;
      }
    }
    store_elt(a.out, a.odt, (int64_t)b * a.osb + (int64_t)(gr.h0 + g) * a.osh + d, O / L);
  }
  if (tid == 0) reset_counter(&a.counters[(int64_t)b * gr.ng + gr.unit]);
}

// Streams items j = w, w + NW, ... of a slice.  item(j, t_lo, t_hi, hm)
// describes item j, load(t_lo, t_hi, buf) issues its loads, compute(t_lo,
// t_hi, hm, buf) consumes them.  Up to three items per wave are loaded at
// once; beyond that two items are in flight (the next item's loads are
// outstanding while the current one is computed, and a buffer is refilled
// right after its compute; past the end a look-ahead re-reads the last item).
template <int NW, typename Buf, typename Item, typename Load, typename Compute>
__device__ __forceinline__ void stream_items(int w, int n_items, Item item, Load load, Compute compute) {
  if (w >= n_items) return;
  const int mine = (n_items - w + NW - 1) / NW;    // items of this wave (wave-uniform)
  Buf A, B;
  int alo, ahi, blo, bhi;
  uint32_t ahm, bhm;
  int j = w;
  if (mine <= 3) {
    // the common sparse case: straight-line code per count, every tile's
    // loads issued before the first wait and no load issued for nothing
    // (a wave's loads share the CU's vector-memory pipeline with the others)
    item(j, alo, ahi, ahm);
    load(alo, ahi, A);
    if (mine == 1) {
      __builtin_amdgcn_sched_barrier(0);
      compute(alo, ahi, ahm, A);
      return;
    }
    item(j + NW, blo, bhi, bhm);
    load(blo, bhi, B);
    if (mine == 2) {
      __builtin_amdgcn_sched_barrier(0);
      compute(alo, ahi, ahm, A);
      compute(blo, bhi, bhm, B);
      return;
    }
    Buf C;
    int clo, chi;
    uint32_t chm;
    item(j + 2 * NW, clo, chi, chm);
    load(clo, chi, C);
    __builtin_amdgcn_sched_barrier(0);
    compute(alo, ahi, ahm, A);
    compute(blo, bhi, bhm, B);
    compute(clo, chi, chm, C);
    return;
  }
  item(j, alo, ahi, ahm);
  load(alo, ahi, A);
  item(j + NW, blo, bhi, bhm);
  load(blo, bhi, B);
  for (;;) {
    __builtin_amdgcn_sched_barrier(0);
    compute(alo, ahi, ahm, A);
    j += NW;
    if (j >= n_items) break;
    item(min(j + NW, n_items - 1), alo, ahi, ahm);
    load(alo, ahi, A);
    __builtin_amdgcn_sched_barrier(0);
    compute(blo, bhi, bhm, B);
    j += NW;
    if (j >= n_items) break;
    item(min(j + NW, n_items - 1), blo, bhi, bhm);
    load(blo, bhi, B);
  }
}

// ---------------------------------------------------------------------------
// VALU streaming kernel (fp32 K/V).
// ---------------------------------------------------------------------------
template <int KVDT, int D, int GMAX, int NT>
__global__ __launch_bounds__(NT) void decode_kernel(DecodeArgs a) {
  constexpr int NW = NT / kWave;
  constexpr int EPV = Elt<KVDT>::kPerVec;
  constexpr int EB = Elt<KVDT>::kBytes;
  constexpr int LPR = D / EPV;                 // lanes per token row
  constexpr int RPL = kWave / LPR;             // token rows per wave-wide load
  constexpr int NLD0 = 16 / RPL;
  constexpr int NLD = NLD0 < 1 ? 1 : (NLD0 > 4 ? 4 : NLD0);   // <= 64 VGPRs of K/V tiles
  constexpr int TT = RPL * NLD;                // tokens per sub-tile
  constexpr int HC0 = 8192 / (NW * D);         // heads merged per pass: <= 32 KiB of LDS
  constexpr int HC = HC0 < 1 ? 1 : (HC0 > GMAX ? GMAX : HC0);
  extern __shared__ __align__(16) unsigned char s_dyn_raw[];
  __shared__ float s_q[GMAX][D];
  __shared__ float s_acc[NW][HC][D];
  __shared__ float s_m[NW][GMAX], s_l[NW][GMAX];
  __shared__ int s_cnt[GMAX];
  __shared__ int s_misc[NW + 2];

  // groups fastest in the grid: consecutive workgroups land on different XCDs
  const Grp gr = group_of(a, blockIdx.x);
  const int split = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int seg = lane % LPR, rsub = lane / LPR;
  const int G = gr.G;
  const int len = seq_len_of(a.seq_lens, a.uniform_len, b);
  const int nb = len > 0 ? ceil_div(len, a.bs) : 0;

  stage_q<NT, GMAX, D>(s_q, a.q, a.qdt, (int64_t)b * a.qsb + (int64_t)gr.h0 * a.qsh, a.qsh, G, a.scale_log2);
  const Slice sl = build_slice<NT>(a, b, gr, split, nb, s_dyn_raw, s_cnt, s_misc);
  if (sl.U == 0) {
    if (split == 0) write_nan_outputs(a, b, gr, D, NT);
    return;
  }
  if (sl.lo >= sl.hi) return;
  const uint32_t* s_list = list_base(a, s_dyn_raw);

  // q lives in registers, except for groups of 8 heads where it is read from
  // LDS at each use to leave the registers to the double-buffered K/V tiles.
  constexpr bool kQRegs = GMAX < 8;
  constexpr int QG = kQRegs ? GMAX : 1;
  float qr[QG][EPV];
  if constexpr (kQRegs) {
#pragma unroll
    for (int g = 0; g < QG; ++g)
#pragma unroll
      for (int e = 0; e < EPV; ++e) qr[g][e] = g < G ? s_q[g][seg * EPV + e] : 0.f;
  }
  auto qv = [&](int g, int e) -> float {
    if constexpr (kQRegs) return qr[g][e]; else return s_q[g][seg * EPV + e];
  };
  float m[GMAX], l[GMAX], acc[GMAX][EPV];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < EPV; ++e) acc[g][e] = 0.f;
  }
  const int64_t head_off = ((int64_t)b * a.sb + (int64_t)gr.kv * a.sh + seg * EPV) * EB;
  const char* kbase = reinterpret_cast<const char*>(a.k) + head_off;
  const char* vbase = reinterpret_cast<const char*>(a.v) + head_off;
  const int64_t row_bytes = a.ss * EB;
  const int n_sub = ceil_div(a.bs, TT);
  const int n_items = (sl.hi - sl.lo) * n_sub;

  struct Buf { uint4 k[NLD], v[NLD]; };
  // item j: sub-tile (j % n_sub) of list entry (j / n_sub)
  auto item = [&](int j, int& t_lo, int& t_hi, uint32_t& hm) {
    int blk;
    list_entry(a, gr, s_list, sl.lo, j / n_sub, blk, hm);
    t_lo = blk * a.bs + (j % n_sub) * TT;
    t_hi = min(min(blk * a.bs + a.bs, len), t_lo + TT);
  };
  // Rows past the tile's end load the tile's last row instead (always in
  // bounds, so the loads need no predication); their scores are masked.
  auto load = [&](int t_lo, int t_hi, Buf& r) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int64_t o = (int64_t)min(t_lo + i * RPL + rsub, t_hi - 1) * row_bytes;
      r.k[i] = load16(kbase + o);
      r.v[i] = load16(vbase + o);
    }
  };
  auto compute = [&](int t_lo, int t_hi, uint32_t hm, const Buf& r) {
    // scores of every active head for this lane's NLD token rows
    float s[GMAX][NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      float kx[EPV];
      unpack<KVDT>(r.k[i], kx);
      const bool valid = t_lo + i * RPL + rsub < t_hi;
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        if (g < G && ((hm >> g) & 1u)) {
          float p = qv(g, 0) * kx[0];
#pragma unroll
          for (int e = 1; e < EPV; ++e) p = fmaf(qv(g, e), kx[e], p);
          p = group_sum<LPR>(p);
          s[g][i] = valid ? p : -INFINITY;
        }
      }
    }
    // online-softmax update per head; s becomes the token weights
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      if (g < G && ((hm >> g) & 1u)) {
        float mt = s[g][0];
#pragma unroll
        for (int i = 1; i < NLD; ++i) mt = fmaxf(mt, s[g][i]);
        const float mn = fmaxf(m[g], mt);
        if (mn != -INFINITY) {
          const float alpha = exp2f(m[g] - mn);
          float ps = l[g] * alpha;
#pragma unroll
          for (int e = 0; e < EPV; ++e) acc[g][e] *= alpha;
#pragma unroll
          for (int i = 0; i < NLD; ++i) {
            s[g][i] = exp2f(s[g][i] - mn);
            ps += s[g][i];
          }
          l[g] = ps;
          m[g] = mn;
        } else {
#pragma unroll
          for (int i = 0; i < NLD; ++i) s[g][i] = 0.f;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      float vx[EPV];
      unpack<KVDT>(r.v[i], vx);
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        if (g < G && ((hm >> g) & 1u)) {
#pragma unroll
          for (int e = 0; e < EPV; ++e) acc[g][e] = fmaf(s[g][i], vx[e], acc[g][e]);
        }
      }
    }
  };
  stream_items<NW, Buf>(w, n_items, item, load, compute);

  // combine the row groups of the wave (lanes with the same slice)
  auto merge_pair = [&](int g, float ma, float mb, float la, float lb, const float* aa, const float* ab) {
    const float mn = fmaxf(ma, mb);
    const float fa = ma == -INFINITY ? 0.f : exp2f(ma - mn);
    const float fb = mb == -INFINITY ? 0.f : exp2f(mb - mn);
    m[g] = mn;
    l[g] = la * fa + lb * fb;
#pragma unroll
    for (int e = 0; e < EPV; ++e) acc[g][e] = aa[e] * fa + ab[e] * fb;
  };
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g < G) {
      // within a 16-lane row: rotations by 4 and 8 lanes keep the slice index
      if constexpr (LPR <= 4) {
        float ab[EPV];
#pragma unroll
        for (int e = 0; e < EPV; ++e) ab[e] = dpp_mov<0x124>(acc[g][e]);
        merge_pair(g, m[g], dpp_mov<0x124>(m[g]), l[g], dpp_mov<0x124>(l[g]), acc[g], ab);
      }
      if constexpr (LPR <= 8) {
        float ab[EPV];
#pragma unroll
        for (int e = 0; e < EPV; ++e) ab[e] = dpp_mov<0x128>(acc[g][e]);
        merge_pair(g, m[g], dpp_mov<0x128>(m[g]), l[g], dpp_mov<0x128>(l[g]), acc[g], ab);
      }
      if constexpr (LPR <= 16) {
        const LanePair pm = swap16(m[g]), pl = swap16(l[g]);
        float aa[EPV], ab[EPV];
#pragma unroll
        for (int e = 0; e < EPV; ++e) { const LanePair p = swap16(acc[g][e]); aa[e] = p.a; ab[e] = p.b; }
        merge_pair(g, pm.a, pm.b, pl.a, pl.b, aa, ab);
      }
      if constexpr (LPR <= 32) {
        const LanePair pm = swap32(m[g]), pl = swap32(l[g]);
        float aa[EPV], ab[EPV];
#pragma unroll
        for (int e = 0; e < EPV; ++e) { const LanePair p = swap32(acc[g][e]); aa[e] = p.a; ab[e] = p.b; }
        merge_pair(g, pm.a, pm.b, pl.a, pl.b, aa, ab);
      }
      if (lane == 0) {
        s_m[w][g] = m[g];
        s_l[w][g] = l[g];
      }
    }
  }
  finish<NT, D, GMAX, HC>(a, b, gr, split, sl, s_m, s_l, s_acc, s_misc, [&](int g0, int n) {
    if (rsub == 0) {
#pragma unroll
      for (int gg = 0; gg < HC; ++gg)
        if (gg < n)
#pragma unroll
          for (int e = 0; e < EPV; ++e) s_acc[w][gg][seg * EPV + e] = acc[g0 + gg][e];
    }
  });
}

// ---------------------------------------------------------------------------
// Matrix-core streaming kernel (bf16 / fp16 K/V).
// ---------------------------------------------------------------------------
template <int D, int NT, int GMAX>
struct MfmaShape {
  static constexpr int NW = NT / kWave;
  static constexpr int KS = TileShape<D>::KS;
  static constexpr int NT16 = TileShape<D>::NT16;
  static constexpr int VROW = TileShape<D>::VROW;
  static constexpr int VT_WORDS = TileShape<D>::VT_WORDS;
  static constexpr int HC0 = 8192 / (NW * D);
  static constexpr int HC = HC0 < 1 ? 1 : (HC0 > GMAX ? GMAX : HC0);   // heads merged per LDS pass
  static constexpr int BIG_WORDS = (NW * VT_WORDS > NW * HC * D) ? NW * VT_WORDS : NW * HC * D;
};

template <int KVDT, int D, int GMAX, int NT>
__global__ __launch_bounds__(NT) void decode_mfma_kernel(DecodeArgs a) {
  static_assert(D % 32 == 0 && GMAX <= 16, "16x16 tiles over head_dim, at most 16 q-heads per group");
  using S = MfmaShape<D, NT, GMAX>;
  constexpr int NW = S::NW, KS = S::KS, NT16 = S::NT16, VROW = S::VROW, HC = S::HC;
  extern __shared__ __align__(16) unsigned char s_dyn_raw[];
  __shared__ __align__(16) uint32_t s_big[S::BIG_WORDS];    // V tiles while streaming, then the merge
  __shared__ float s_m[NW][GMAX], s_l[NW][GMAX];
  __shared__ int s_cnt[GMAX];
  __shared__ int s_misc[NW + 2];

  // groups fastest in the grid: consecutive workgroups land on different XCDs
  const Grp gr = group_of(a, blockIdx.x);
  const int split = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int col = lane & 15, grp = lane >> 4;     // MFMA lane coordinates
  const int G = gr.G;
  const int len = seq_len_of(a.seq_lens, a.uniform_len, b);
  const int nb = len > 0 ? ceil_div(len, a.bs) : 0;

  uint4 qf[KS];
  load_q_frag<KVDT, D>(a.q, a.qdt, (int64_t)b * a.qsb + (int64_t)gr.h0 * a.qsh, a.qsh, G, qf);
  const Slice sl = build_slice<NT>(a, b, gr, split, nb, s_dyn_raw, s_cnt, s_misc);
  if (sl.U == 0) {
    if (split == 0) write_nan_outputs(a, b, gr, D, NT);
    return;
  }
  if (sl.lo >= sl.hi) return;
  const uint32_t* s_list = list_base(a, s_dyn_raw);

  // lane (col, grp) loads token col of a 16-token tile, elements [D/4*grp, D/4*(grp+1)) of its row
  const int64_t head_off = ((int64_t)b * a.sb + (int64_t)gr.kv * a.sh + (D / 4) * grp) * 2;
  const char* kbase = reinterpret_cast<const char*>(a.k) + head_off;
  const char* vbase = reinterpret_cast<const char*>(a.v) + head_off;
  const int64_t row_bytes = a.ss * 2;
  const int n_sub = ceil_div(a.bs, 16);
  const int n_items = (sl.hi - sl.lo) * n_sub;
  uint32_t* vt = s_big + w * S::VT_WORDS;         // this wave's V tile [16 tokens][VROW words]
  const float scale = a.scale_log2;
  TileState<D> st;
  tile_init(st);

  auto item = [&](int j, int& t0, int& t_hi, uint32_t& hm) {
    int blk;
    list_entry(a, gr, s_list, sl.lo, j / n_sub, blk, hm);
    t0 = blk * a.bs + (j % n_sub) * 16;
    t_hi = min(min(blk * a.bs + a.bs, len), t0 + 16);
  };
  auto load = [&](int t0, int t_hi, TileBuf<D>& r) { tile_load<D>(kbase, vbase, row_bytes, t0, t_hi, r); };
  auto compute = [&](int t0, int t_hi, uint32_t hm, const TileBuf<D>& r) {
    tile_update<KVDT, D>(st, r, qf, vt, t0, t_hi, col < G && ((hm >> col) & 1u), scale);
  };
  stream_items<NW, TileBuf<D>>(w, n_items, item, load, compute);

  tile_finish(st);
  if (grp == 0 && col < G) {
    s_m[w][col] = st.m_h;
    s_l[w][col] = st.l_h;
  }
  __syncthreads();                                  // the V tiles are dead: s_big becomes s_acc
  auto s_acc = reinterpret_cast<float (*)[HC][D]>(s_big);
  finish<NT, D, GMAX, HC>(a, b, gr, split, sl, s_m, s_l, s_acc, s_misc, [&](int g0, int n) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int head = 4 * grp + i;
      if (head >= g0 && head < g0 + n)
#pragma unroll
        for (int t = 0; t < NT16; ++t) s_acc[w][head - g0][t * 16 + col] = st.acc[t][i];
    }
  });
}

// Dense split-K merge: one workgroup per (q-head of the group, KV head, sequence).
__global__ __launch_bounds__(256) void merge_kernel(MergeArgs a) {
  __shared__ float s_f[256];
  __shared__ float s_red[256];
  __shared__ float s_scr[4];
  const int g = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int len = seq_len_of(a.seq_lens, a.uniform_len, b);
  const int nb = len > 0 ? ceil_div(len, a.bs) : 0;
  const int D = a.D;
  const int64_t pstride = (int64_t)a.G * (D + 2);
  const float* pg = a.partials + (((int64_t)b * a.Hkv + kvh) * a.nsplit) * pstride + g * (D + 2);
  const int per = nb > 0 ? ceil_div(nb, a.nsplit) : 0;
  const int n_active = nb > 0 ? ceil_div(nb, per) : 0;
  if (n_active <= 1) return;                 // the decode kernel wrote the output itself
  const int64_t oo = (int64_t)b * a.osb + (int64_t)(kvh * a.G + g) * a.osh;
  const float ms = tid < n_active ? pg[tid * pstride] : -INFINITY;
  const float ls = tid < n_active ? pg[tid * pstride + 1] : 0.f;
  const float M = block_reduce<256>(ms, s_scr, OpMax());
  const float f = (ms == -INFINITY) ? 0.f : exp2f(ms - M);
  s_f[tid] = f;
  const float L = block_reduce<256>(ls * f, s_scr, OpAdd());
  // thread t sums splits part, part + np, ... of dim t % D
  const int np = 256 / D;
  const int d = tid % D, part = tid / D;
  float O = 0.f;
  if (part < np) {
    for (int s0 = part; s0 < n_active; s0 += 8 * np) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int s = s0 + u * np;
        v[u] = s < n_active ? pg[s * pstride + 2 + d] * s_f[s] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) O += v[u];
    }
  }
  s_red[tid] = O;
  __syncthreads();
  if (tid < D) {
    float t = 0.f;
    for (int p = 0; p < np; ++p) t += s_red[p * D + tid];
    store_elt(a.out, a.odt, oo + tid, t / L);
  }
}

template <int KVDT, int D, int NT, bool MFMA>
hipError_t launch_g(const DecodeArgs& a, size_t dyn, hipStream_t s) {
  dim3 grid(a.per_head ? a.Hq : a.Hkv, a.nsplit, a.B);
  const int ge = a.per_head ? 1 : a.G;
#define ADAKV_LAUNCH(GM)                                                                          \
  do {                                                                                            \
    if constexpr (MFMA)                                                                           \
      hipLaunchKernelGGL((decode_mfma_kernel<KVDT, D, GM, NT>), grid, dim3(NT), dyn, s, a);       \
    else                                                                                          \
      hipLaunchKernelGGL((decode_kernel<KVDT, D, GM, NT>), grid, dim3(NT), dyn, s, a);            \
  } while (0)
  if (ge <= 1) ADAKV_LAUNCH(1);
  else if (ge <= 2) ADAKV_LAUNCH(2);
  else if (ge <= 4) ADAKV_LAUNCH(4);
  else if (ge <= 8) ADAKV_LAUNCH(8);
  else ADAKV_LAUNCH(16);
#undef ADAKV_LAUNCH
  return hipGetLastError();
}

template <int KVDT, int D>
hipError_t launch_d(const DecodeArgs& a, hipStream_t s) {
  constexpr bool kMfma = KVDT != ADAKV_F32;
  if (a.table) {
    const size_t dyn = ((size_t)a.Hq * 8 + 15) / 16 * 16 + (size_t)(((a.max_blocks + 3) / 4 + 3) / 4 * 4 + a.list_cap) * 4;
    // head_dim 256 in matrix-core mode: 4 waves keep the V tiles within 64 KiB
    constexpr int NT = (kMfma && D >= 256) ? 256 : kSparseThreads;
    return launch_g<KVDT, D, NT, kMfma>(a, dyn, s);
  }
  return launch_g<KVDT, D, kDenseThreads, kMfma>(a, 16, s);
}

template <int KVDT>
hipError_t launch_k(const DecodeArgs& a, int D, hipStream_t s) {
  switch (D) {
    case 32: return launch_d<KVDT, 32>(a, s);
    case 64: return launch_d<KVDT, 64>(a, s);
    case 128: return launch_d<KVDT, 128>(a, s);
    case 256: return launch_d<KVDT, 256>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int decode_threads(int kvdt, int D, bool sparse) {
  if (!sparse) return kDenseThreads;
  return (kvdt != ADAKV_F32 && D >= 256) ? 256 : kSparseThreads;
}

size_t decode_static_lds(int kvdt, int D, int gmax, bool sparse) {
  const int NW = decode_threads(kvdt, D, sparse) / kWave;
  const size_t common = (size_t)2 * NW * gmax * 4 + (size_t)gmax * 4 + (size_t)(NW + 2) * 4;
  if (kvdt == ADAKV_F32) {
    const int hc = std::max(1, std::min(gmax, 8192 / (NW * D)));
    return common + (size_t)gmax * D * 4 + (size_t)NW * hc * D * 4;
  }
  const int hc = std::max(1, std::min(gmax, 8192 / (NW * D)));
  const size_t vt = (size_t)NW * 16 * (D / 2 + 2) * 4, mrg = (size_t)NW * hc * D * 4;
  return common + std::max(vt, mrg);
}

hipError_t launch_decode(const DecodeArgs& a, int kvdt, int D, hipStream_t s) {
  switch (kvdt) {
    case ADAKV_F32: return launch_k<ADAKV_F32>(a, D, s);
    case ADAKV_F16: return launch_k<ADAKV_F16>(a, D, s);
    case ADAKV_BF16: return launch_k<ADAKV_BF16>(a, D, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_merge(const MergeArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(merge_kernel, dim3(a.G, a.Hkv, a.B), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace adakv
