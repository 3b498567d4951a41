// One wave's flash-decode step over a 16-token tile of K and V on the matrix
// cores (bf16 / fp16), shared by the table-driven decode kernel and the fused
// selection + decode kernel (adakv/kernels/block_sparse_decode.py:64-100).
//
// S^T = K . Q^T runs on v_mfma_f32_16x16x32: K is loaded straight into the
// A-operand layout (lane (col, grp) = (l % 16, l / 16) holds token col of the
// tile and the contiguous D/4 elements [D/4*grp, D/4*(grp+1)) of its row, so a
// tile is D/32 coalesced 16-byte loads per lane), and up to 16 q-heads,
// zero-padded, form the B operand with the same permutation of head_dim.  The
// online softmax runs on the 16x16 result (lane (col, grp) holds tokens
// 4*grp .. +3 for head col; the cross-lane max over the 4 lane groups uses
// permlane swaps), and O += P . V runs on v_mfma_f32_16x16x16 with P taken
// directly from the S^T result layout and V transposed through a per-wave LDS
// tile.  A tile costs 3*D/32 matrix instructions and a few dozen VALU ones.
#pragma once

#include "common.hpp"

namespace adakv {

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));

template <int KVDT>
__device__ __forceinline__ float4_t mfma_qk(const uint4& k, const uint4& q, float4_t c) {
  if constexpr (KVDT == ADAKV_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, k),
                                                   __builtin_bit_cast(bf16x8_t, q), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, k),
                                                  __builtin_bit_cast(f16x8_t, q), c, 0, 0, 0);
}
template <int KVDT>
__device__ __forceinline__ float4_t mfma_pv(const uint2& p, const uint2& v, float4_t c) {
  if constexpr (KVDT == ADAKV_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(short4_t, p),
                                                     __builtin_bit_cast(short4_t, v), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, p),
                                                 __builtin_bit_cast(f16x4_t, v), c, 0, 0, 0);
}
// Two floats to the 16-bit type, round to nearest even (one packed convert
// instruction on gfx950: v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32).
template <int KVDT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  if constexpr (KVDT == ADAKV_BF16) {
    typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2_t{lo, hi}), b2_t));
  } else {
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2_t{lo, hi}), h2_t));
  }
}

template <int D>
struct TileShape {
  static constexpr int KS = D / 32;            // k-steps of S^T = K . Q^T (16-byte loads per lane)
  static constexpr int NT16 = D / 16;          // 16-column tiles of O
  static constexpr int VROW = D / 2 + 2;       // V tile row stride in 4-byte words (conflict-free reads)
  static constexpr int VT_WORDS = 16 * VROW;   // one wave's V tile
};

// K and V fragments of one tile, as loaded by a lane.
template <int D>
struct TileBuf {
  uint4 k[D / 32], v[D / 32];
};

// Per-wave online-softmax state: m_h, l_h of head col (l over this lane's
// tokens until tile_finish), acc[n][i] = O[head 4*grp+i][16*n + col].
template <int D>
struct TileState {
  float m_h, l_h;
  float4_t acc[D / 16];
};

template <int D>
__device__ __forceinline__ void tile_init(TileState<D>& st) {
  st.m_h = -INFINITY;
  st.l_h = 0.f;
#pragma unroll
  for (int n = 0; n < D / 16; ++n) st.acc[n] = float4_t{0.f, 0.f, 0.f, 0.f};
}

// B operand of S^T: lane (col, grp) holds q[head col][D/4*grp + 8*s .. +7] at
// step s, heads col >= G zero.  Row of head col at element qbase + col * qsh
// (clamped to the last head, so every load is in bounds).
template <int KVDT, int D>
__device__ __forceinline__ void load_q_frag(const void* q, int qdt, int64_t qbase, int64_t qsh, int G,
                                            uint4 (&qf)[D / 32]) {
  constexpr int KS = D / 32;
  const int lane = threadIdx.x & (kWave - 1), col = lane & 15, grp = lane >> 4;
  with_dtype(qdt, [&](auto tag) {
    constexpr int QDT = decltype(tag)::value;
    const int64_t qo = qbase + (int64_t)min(col, G - 1) * qsh + (D / 4) * grp;
    float x[KS][8];
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int t = 0; t < 8; ++t) x[s][t] = load_t<QDT>(q, qo + 8 * s + t);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      uint32_t wv[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) wv[t] = col < G ? pack2<KVDT>(x[s][2 * t], x[s][2 * t + 1]) : 0u;
      qf[s] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
    }
  });
}

// Loads of the tile [t0, t_hi) (t_hi - t0 <= 16, t_hi >= 1): tokens past the
// tile's end load its last row instead (always in bounds, so the loads need no
// predication); their weights are zeroed by tile_update.  kbase / vbase point
// at element D/4*grp of token 0 of the KV head.
template <int D>
__device__ __forceinline__ void tile_load(const char* kbase, const char* vbase, int64_t row_bytes, int t0, int t_hi,
                                          TileBuf<D>& r) {
  const int col = threadIdx.x & 15;
  const int64_t o = (int64_t)min(t0 + col, t_hi - 1) * row_bytes;
#pragma unroll
  for (int s = 0; s < D / 32; ++s) {
    r.k[s] = load16(kbase + o + 16 * s);
    r.v[s] = load16(vbase + o + 16 * s);
  }
}

// One tile into the state.  head_on: head col takes part in this tile (lanes
// whose head is off give it zero weight).  vt: this wave's V tile in LDS.
// scale: sm_scale * log2(e).  rescale (uniform): false for the wave's first
// tile, whose accumulators are still zero and need no rescaling.
template <int KVDT, int D>
__device__ __forceinline__ void tile_update(TileState<D>& st, const TileBuf<D>& r, const uint4 (&qf)[D / 32],
                                            uint32_t* vt, int t0, int t_hi, bool head_on, float scale,
                                            bool rescale = true) {
  using S = TileShape<D>;
  constexpr int KS = S::KS, NT16 = S::NT16, VROW = S::VROW;
  const int lane = threadIdx.x & (kWave - 1), col = lane & 15, grp = lane >> 4;
  const uint16_t* vt16 = reinterpret_cast<const uint16_t*>(vt);
  // V rows to this wave's LDS tile for the transposed B-operand reads; the
  // previous tile's reads were issued before these writes (LDS operations of
  // a wave complete in order), the compiler barriers keep that order.
  __asm__ volatile("" ::: "memory");
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    uint32_t* p = vt + col * VROW + (D / 8) * grp + 4 * s;
    *reinterpret_cast<uint2*>(p) = make_uint2(r.v[s].x, r.v[s].y);
    *reinterpret_cast<uint2*>(p + 2) = make_uint2(r.v[s].z, r.v[s].w);
  }
  __asm__ volatile("" ::: "memory");
  // S^T[token 4*grp+i][head col]
  float4_t sc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < KS; ++s) sc = mfma_qk<KVDT>(r.k[s], qf[s], sc);
  float sv[4];
  float mt = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bool ok = head_on && (t0 + 4 * grp + i < t_hi);
    sv[i] = ok ? sc[i] * scale : -INFINITY;
    mt = fmaxf(mt, sv[i]);
  }
  LanePair pr = swap16(mt);
  mt = fmaxf(pr.a, pr.b);
  pr = swap32(mt);
  mt = fmaxf(pr.a, pr.b);
  const float mn = fmaxf(st.m_h, mt);
  const float alpha = (mn == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(st.m_h - mn);
  float ps = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sv[i] = sv[i] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sv[i] - mn);
    ps += sv[i];
  }
  st.l_h = st.l_h * alpha + ps;
  st.m_h = mn;
  // rescale the O rows (heads 4*grp+i) by their heads' alpha, held by lanes col == head
  if (rescale) {
    float al[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      al[i] = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * grp + i) * 4, __float_as_int(alpha)));
#pragma unroll
    for (int n = 0; n < NT16; ++n)
#pragma unroll
      for (int i = 0; i < 4; ++i) st.acc[n][i] *= al[i];
  }
  // O += P . V: A = P[head col][tokens 4*grp .. +3] (the S^T layout), B = V[tokens][16 dims]
  const uint2 pf = make_uint2(pack2<KVDT>(sv[0], sv[1]), pack2<KVDT>(sv[2], sv[3]));
#pragma unroll
  for (int n = 0; n < NT16; ++n) {
    const int c16 = n * 16 + col;
    const uint32_t v0 = vt16[(4 * grp + 0) * 2 * VROW + c16], v1 = vt16[(4 * grp + 1) * 2 * VROW + c16];
    const uint32_t v2 = vt16[(4 * grp + 2) * 2 * VROW + c16], v3 = vt16[(4 * grp + 3) * 2 * VROW + c16];
    st.acc[n] = mfma_pv<KVDT>(pf, make_uint2(v0 | (v1 << 16), v2 | (v3 << 16)), st.acc[n]);
  }
}

// Denominator of head col over the wave's 4 lane groups (every lane receives it).
template <int D>
__device__ __forceinline__ void tile_finish(TileState<D>& st) {
  LanePair pr = swap16(st.l_h);
  st.l_h = pr.a + pr.b;
  pr = swap32(st.l_h);
  st.l_h = pr.a + pr.b;
}

}  // namespace adakv
