// Ragged block-sparse split-K flash-decode (adakv/kernels/block_sparse_decode.py:51-100)
// and the dense split-K flash-decode baseline, one kernel for both.
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
// Inside a workgroup every wave streams its blocks with double-buffered 16-byte
// loads: a lane owns one 16-byte slice of head_dim for one token row, so a
// 16-token bf16 block of K (or V) is four coalesced loads per lane.  Scores of
// every q-head that selected the block come from one read of K; each group of
// lanes sharing a token row keeps its own online softmax (running max,
// denominator, fp32 accumulator, exp2 domain), so no cross-row exchange happens
// per block.  Row groups and waves are combined once at the end.  Several
// active slices write (m, l, acc[D]) partials; in sparse mode the last slice
// to arrive merges them, in dense mode merge_kernel does.
#include "common.hpp"
#include "internal.hpp"

namespace adakv {
namespace {

constexpr int kSparseThreads = 512;

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
  extern __shared__ __align__(16) unsigned char s_dyn_raw[];
  __shared__ float s_q[GMAX][D];
  constexpr int HC0 = 8192 / (NW * D);          // heads merged per pass: <= 32 KiB of LDS
  constexpr int HC = HC0 < 1 ? 1 : (HC0 > GMAX ? GMAX : HC0);
  __shared__ float s_acc[NW][HC][D];
  __shared__ float s_m[NW][GMAX], s_l[NW][GMAX];
  __shared__ int s_cnt[GMAX];
  __shared__ double s_wsum;
  __shared__ int s_misc[NW + 2];

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), w = tid / kWave;
  const int seg = lane % LPR, rsub = lane / LPR;
  const int G = a.G;
  const int len = seq_len_of(a.seq_lens, a.uniform_len, b);
  const int nb = len > 0 ? ceil_div(len, a.bs) : 0;
  const bool dense = a.table == nullptr;
  double* s_w = reinterpret_cast<double*>(s_dyn_raw);
  uint32_t* s_bits = reinterpret_cast<uint32_t*>(s_dyn_raw + ((a.Hq * 8 + 15) / 16) * 16);
  uint32_t* s_list = s_bits + ceil_div(a.max_blocks, 4);

  for (int i = tid; i < G * D; i += NT)
    s_q[i / D][i % D] = load_elt(a.q, a.qdt, (int64_t)b * a.qsb + (int64_t)(kvh * G + i / D) * a.qsh + i % D) *
                        a.scale_log2;

  // ---- per-head counts and the union of the group's blocks ----
  // The table entries that can be selected are loaded up front (before the
  // counts are known); the counts then decide which of them enter the union.
  int U = nb, off = 0, w0 = 0, w1 = 0;
  if (!dense) {
    const Bounds bb = budget_bounds(nb, a.cfg);
    const bool derive = a.sel_lens == nullptr;
    const bool adaptive = derive && a.cfg.policy == ADAKV_POLICY_ADAPTIVE && nb > 1;
    const int width = derive ? min(a.T, max(bb.kcap, 0)) : a.T;
    const int nwords = ceil_div(nb, 4);
    for (int i = tid; i < nwords; i += NT) s_bits[i] = 0;
    if (adaptive)
      for (int h = tid; h < a.Hq; h += NT) s_w[h] = a.wbuf[(int64_t)b * a.Hq + h];
    if (!derive && tid < G) s_cnt[tid] = min(max(a.sel_lens[(int64_t)b * a.Hq + kvh * G + tid], 0), a.T);
    constexpr int EPT = 4;                       // table entries per thread
    int ent[EPT];
#pragma unroll
    for (int u = 0; u < EPT; ++u) {
      const int e = tid + u * NT;
      ent[u] = -1;
      if (e < G * width) {
        const int g = e / width, j = e % width;
        ent[u] = a.table[((int64_t)b * a.Hq + kvh * G + g) * a.T + j];
      }
    }
    __syncthreads();
    if (derive) {
      // every thread evaluates the same sum of weights in NumPy's order
      const double wsum = adaptive ? numpy_pairwise_sum<6>(s_w, a.Hq) : 0.0;
      if (tid < G) {
        const int k = head_count(bb, a.cfg.policy, adaptive ? s_w[kvh * G + tid] : 0.0, wsum, a.Hq);
        s_cnt[tid] = min(k, a.T);
        if (split == 0 && a.sel_lens_out) a.sel_lens_out[(int64_t)b * a.Hq + kvh * G + tid] = k;
      }
      __syncthreads();
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
      const int blk = a.table[((int64_t)b * a.Hq + kvh * G + g) * a.T + j];
      if (j < s_cnt[g] && blk >= 0 && blk < nb) atomicOr(&s_bits[blk >> 2], 1u << ((blk & 3) * 8 + g));
    }
    __syncthreads();
    const int wpt = ceil_div(nwords, NT);
    w0 = min(tid * wpt, nwords);
    w1 = min(w0 + wpt, nwords);
    int cnt = 0;
    for (int i = w0; i < w1; ++i) {
      const uint32_t x = s_bits[i];
      cnt += ((x & 0xffu) != 0) + ((x & 0xff00u) != 0) + ((x & 0xff0000u) != 0) + ((x >> 24) != 0);
    }
    off = block_excl_scan<NT>(cnt, s_misc, &U);
  }
  const int per = U > 0 ? max(ceil_div(U, a.nsplit), a.min_per) : 0;
  const int n_active = U > 0 ? ceil_div(U, per) : 0;
  const int lo_e = split * per, hi_e = min(U, lo_e + per);
  if (U == 0) {
    // no valid block for any head of the group: 0/0, as the reference kernel
    if (split == 0)
      for (int i = tid; i < G * D; i += NT)
        store_elt(a.out, a.odt, (int64_t)b * a.osb + (int64_t)(kvh * G + i / D) * a.osh + i % D, __builtin_nanf(""));
    return;
  }
  if (lo_e >= hi_e) return;
  if (!dense) {
    int p = off;
    for (int i = w0; i < w1; ++i) {
      const uint32_t x = s_bits[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t m8 = (x >> (8 * j)) & 0xffu;
        if (m8) {
          if (p >= lo_e && p < hi_e) s_list[p - lo_e] = (uint32_t)(4 * i + j) | (m8 << 24);
          ++p;
        }
      }
    }
  }
  __syncthreads();

  // ---- stream this split's blocks ----
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
  const int64_t head_off = ((int64_t)b * a.sb + (int64_t)kvh * a.sh + seg * EPV) * EB;
  const char* kbase = reinterpret_cast<const char*>(a.k) + head_off;
  const char* vbase = reinterpret_cast<const char*>(a.v) + head_off;
  const int64_t row_bytes = a.ss * EB;
  const uint32_t all_heads = (1u << G) - 1u;
  const int n_sub = ceil_div(a.bs, TT);
  const int n_items = (hi_e - lo_e) * n_sub;

  // item j: sub-tile (j % n_sub) of list entry (j / n_sub)
  auto item = [&](int j, int& t_lo, int& t_hi, uint32_t& hm) {
    const int e = lo_e + j / n_sub;
    int blk;
    if (dense) {
      blk = e;
      hm = all_heads;
    } else {
      const uint32_t ent = s_list[e - lo_e];
      blk = (int)(ent & 0xffffffu);
      hm = ent >> 24;
    }
    t_lo = blk * a.bs + (j % n_sub) * TT;
    t_hi = min(min(blk * a.bs + a.bs, len), t_lo + TT);
  };
  auto load = [&](int t_lo, int t_hi, uint4* kr, uint4* vr) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int t = t_lo + i * RPL + rsub;
      const int64_t o = (int64_t)t * row_bytes;
      kr[i] = t < t_hi ? load16(kbase + o) : make_uint4(0, 0, 0, 0);
      vr[i] = t < t_hi ? load16(vbase + o) : make_uint4(0, 0, 0, 0);
    }
  };
  auto compute = [&](int t_lo, int t_hi, uint32_t hm, const uint4* kr, const uint4* vr) {
    // scores of every active head for this lane's NLD token rows
    float s[GMAX][NLD];
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      float kx[EPV];
      unpack<KVDT>(kr[i], kx);
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
      unpack<KVDT>(vr[i], vx);
#pragma unroll
      for (int g = 0; g < GMAX; ++g) {
        if (g < G && ((hm >> g) & 1u)) {
#pragma unroll
          for (int e = 0; e < EPV; ++e) acc[g][e] = fmaf(s[g][i], vx[e], acc[g][e]);
        }
      }
    }
  };

  {
    uint4 ka[NLD], va[NLD], kb[NLD], vb[NLD];
    int alo = 0, ahi = 0, blo = 0, bhi = 0;
    uint32_t ahm = 0, bhm = 0;
    int j = w;
    if (j < n_items) {
      item(j, alo, ahi, ahm);
      load(alo, ahi, ka, va);
    }
    while (j < n_items) {
      const int j2 = j + NW;
      if (j2 < n_items) {
        item(j2, blo, bhi, bhm);
        load(blo, bhi, kb, vb);
      }
      compute(alo, ahi, ahm, ka, va);
      if (j2 >= n_items) break;
      const int j3 = j2 + NW;
      if (j3 < n_items) {
        item(j3, alo, ahi, ahm);
        load(alo, ahi, ka, va);
      }
      compute(blo, bhi, bhm, kb, vb);
      j = j3;
    }
  }

  // ---- combine the row groups of the wave (lanes with the same slice) ----
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

  // ---- combine the waves, HC heads per LDS pass ----
  float* part = a.partials + (((int64_t)b * a.Hkv + kvh) * a.nsplit) * G * (D + 2);
  const int64_t pstride = (int64_t)G * (D + 2);
#pragma unroll
  for (int g0 = 0; g0 < GMAX; g0 += HC) {
    if (g0 >= G) break;                      // uniform over the workgroup
    if (rsub == 0) {
#pragma unroll
      for (int gg = 0; gg < HC; ++gg)
        if (g0 + gg < G)
#pragma unroll
          for (int e = 0; e < EPV; ++e) s_acc[w][gg][seg * EPV + e] = acc[g0 + gg][e];
    }
    __syncthreads();
    for (int i = tid; i < min(HC, G - g0) * D; i += NT) {
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
      if (n_active == 1) {
        store_elt(a.out, a.odt, (int64_t)b * a.osb + (int64_t)(kvh * G + g) * a.osh + d, O / L);
      } else {
        float* pg = part + split * pstride + g * (D + 2);
        pg[2 + d] = O;
        if (d == 0) { pg[0] = M; pg[1] = L; }
      }
    }
    __syncthreads();
  }
  if (n_active == 1 || !a.merge_in_kernel) return;

  // ---- sparse: the last active split merges (at most nsplit <= 16 of them) ----
  __threadfence();
  __syncthreads();
  if (tid == 0) s_misc[NW] = arrive(&a.counters[(int64_t)b * a.Hkv + kvh]) == n_active - 1;
  __syncthreads();
  if (!s_misc[NW]) return;
  __threadfence();
  for (int i = tid; i < G * D; i += NT) {
    const int g = i / D, d = i % D;
    const float* pg = part + g * (D + 2);
    float ms[16], ls[16], os[16];
#pragma unroll
    for (int sp = 0; sp < 16; ++sp) {
      const bool ok = sp < n_active;
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
    store_elt(a.out, a.odt, (int64_t)b * a.osb + (int64_t)(kvh * G + g) * a.osh + d, O / L);
  }
  if (tid == 0) reset_counter(&a.counters[(int64_t)b * a.Hkv + kvh]);
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

template <int KVDT, int D, int NT>
hipError_t launch_g(const DecodeArgs& a, size_t dyn, hipStream_t s) {
  dim3 grid(a.nsplit, a.Hkv, a.B);
  if (a.G <= 1) hipLaunchKernelGGL((decode_kernel<KVDT, D, 1, NT>), grid, dim3(NT), dyn, s, a);
  else if (a.G <= 2) hipLaunchKernelGGL((decode_kernel<KVDT, D, 2, NT>), grid, dim3(NT), dyn, s, a);
  else if (a.G <= 4) hipLaunchKernelGGL((decode_kernel<KVDT, D, 4, NT>), grid, dim3(NT), dyn, s, a);
  else hipLaunchKernelGGL((decode_kernel<KVDT, D, 8, NT>), grid, dim3(NT), dyn, s, a);
  return hipGetLastError();
}

template <int KVDT, int D>
hipError_t launch_d(const DecodeArgs& a, hipStream_t s) {
  if (a.table) {
    const size_t dyn = ((size_t)a.Hq * 8 + 15) / 16 * 16 + (size_t)(((a.max_blocks + 3) / 4) + a.list_cap) * 4;
    return launch_g<KVDT, D, kSparseThreads>(a, dyn, s);
  }
  return launch_g<KVDT, D, 256>(a, 16, s);
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
