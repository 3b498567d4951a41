// Block-summary kernels over each block_size-token block's real tokens:
//
// * centroid: the mean key (adakv/estimator.py:27-48, adakv/attention.py:119-139).
//   Each lane owns one 16-byte slice of head_dim for one block and adds the
//   block's tokens in order, in fp32, then divides once by the token count
//   with IEEE round-to-nearest.  That is the same operation sequence as
//   NumPy's keys[:, s:e].mean(axis=1) on fp32 data, so fp32 centroids are
//   bit-identical to the oracle; bf16 / fp16 centroids are that value rounded
//   once.
// * minmax: the per-dimension max and min of the keys (Quest's block bounds,
//   adakv/estimator.py:50-57, adakv/attention.py:131-138), stored as one row
//   of 2*head_dim elements, [max | min].  Both are exact in the key type and
//   in fp32, so they are bit-identical to the oracle whatever the order.
//
// Append mode recomputes only the blocks that hold the newest n_new tokens.
// Because the reduction restarts from the block's first token, an appended
// summary has the same bits as a full rebuild (the reference's running mean,
// adakv/runtime.py:52-59, drifts by rounding instead).
#include "common.hpp"
#include "internal.hpp"

namespace adakv {
namespace {

template <int CDT, int N>
__device__ __forceinline__ void store_row(void* base, int64_t off, const float* x) {
  if constexpr (CDT == ADAKV_F32) {
    float4* p = reinterpret_cast<float4*>(reinterpret_cast<float*>(base) + off);
#pragma unroll
    for (int i = 0; i < N / 4; ++i) p[i] = make_float4(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
  } else {
    uint32_t w[N / 2];
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const uint32_t lo = CDT == ADAKV_BF16 ? f32_to_bf16_bits(x[2 * i]) : f32_to_f16_bits(x[2 * i]);
      const uint32_t hi = CDT == ADAKV_BF16 ? f32_to_bf16_bits(x[2 * i + 1]) : f32_to_f16_bits(x[2 * i + 1]);
      w[i] = lo | (hi << 16);
    }
    uint16_t* p16 = reinterpret_cast<uint16_t*>(base) + off;
    if constexpr (N == 8) {
      *reinterpret_cast<uint4*>(p16) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      *reinterpret_cast<uint2*>(p16) = make_uint2(w[0], w[1]);
    }
  }
}

template <int KDT, int CDT, int D, bool MM>
__global__ __launch_bounds__(256) void centroid_kernel(CentroidArgs a) {
  constexpr int EPV = Elt<KDT>::kPerVec;
  constexpr int EB = Elt<KDT>::kBytes;
  constexpr int LPR = D / EPV;            // lanes per key row
  constexpr int RPL = kWave / LPR;        // blocks per wave
  constexpr int BPW = 4 * RPL;            // blocks per workgroup
  constexpr int U = 8;                    // tokens loaded before they are summed
  const int kvh = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int seg = lane % LPR, rsub = lane / LPR;
  const int len = seq_len_of(a.seq_lens, a.uniform_len, b);
  const int nb = len > 0 ? ceil_div(len, a.bs) : 0;
  const int first = a.n_new > 0 ? max(len - a.n_new, 0) / a.bs : 0;
  const int blk = first + blockIdx.x * BPW + w * RPL + rsub;
  if (blk >= nb) return;
  const int t0 = blk * a.bs, t1 = min(t0 + a.bs, len);
  const char* kp = reinterpret_cast<const char*>(a.k) +
                   ((int64_t)b * a.sb + (int64_t)kvh * a.sh + (int64_t)t0 * a.ss + seg * EPV) * EB;
  const int64_t step = a.ss * EB;
  float acc[EPV], lo[EPV];
  for (int t = t0; t < t1; t += U) {
    uint4 raw[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      raw[u] = (t + u < t1) ? load16(kp + (int64_t)(t - t0 + u) * step) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (t + u < t1) {
        float x[EPV];
        unpack<KDT>(raw[u], x);
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
          if constexpr (MM) {
            acc[e] = (t + u == t0) ? x[e] : fmaxf(acc[e], x[e]);
            lo[e] = (t + u == t0) ? x[e] : fminf(lo[e], x[e]);
          } else {
            acc[e] = (t + u == t0) ? x[e] : acc[e] + x[e];
          }
        }
      }
    }
  }
  if constexpr (MM) {
    // row of 2*D elements: the maxima, then the minima
    const int64_t row = (((int64_t)b * a.Hkv + kvh) * a.max_blocks + blk) * (2 * D) + seg * EPV;
    store_row<CDT, EPV>(a.c, row, acc);
    store_row<CDT, EPV>(a.c, row + D, lo);
  } else {
    const float cnt = (float)(t1 - t0);
#pragma unroll
    for (int e = 0; e < EPV; ++e) acc[e] = __fdiv_rn(acc[e], cnt);
    const int64_t row = (((int64_t)b * a.Hkv + kvh) * a.max_blocks + blk) * D + seg * EPV;
    store_row<CDT, EPV>(a.c, row, acc);
  }
}

template <int KDT, int CDT, bool MM>
hipError_t launch_d(const CentroidArgs& a, int D, hipStream_t s) {
  auto go = [&](auto kern, int bpw) {
    int span = a.max_blocks;
    if (a.n_new > 0) span = min(a.max_blocks, a.n_new / a.bs + 2);
    dim3 grid((span + bpw - 1) / bpw, a.Hkv, a.B);
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, a);
    return hipGetLastError();
  };
  constexpr int EPV = Elt<KDT>::kPerVec;
  switch (D) {
    case 32: return go(centroid_kernel<KDT, CDT, 32, MM>, 4 * (kWave / (32 / EPV)));
    case 64: return go(centroid_kernel<KDT, CDT, 64, MM>, 4 * (kWave / (64 / EPV)));
    case 128: return go(centroid_kernel<KDT, CDT, 128, MM>, 4 * (kWave / (128 / EPV)));
    case 256: return go(centroid_kernel<KDT, CDT, 256, MM>, 4 * (kWave / (256 / EPV)));
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_centroid(const CentroidArgs& a, int kdt, int cdt, int D, hipStream_t s) {
#define ADAKV_C(K, C) if (kdt == K && cdt == C) return launch_d<K, C, false>(a, D, s);
  ADAKV_C(ADAKV_BF16, ADAKV_BF16) ADAKV_C(ADAKV_BF16, ADAKV_F32)
  ADAKV_C(ADAKV_F16, ADAKV_F16) ADAKV_C(ADAKV_F16, ADAKV_F32)
  ADAKV_C(ADAKV_F32, ADAKV_F32) ADAKV_C(ADAKV_F32, ADAKV_BF16)
#undef ADAKV_C
  return hipErrorInvalidValue;
}

hipError_t launch_minmax(const CentroidArgs& a, int kdt, int cdt, int D, hipStream_t s) {
  if (D > 128) return hipErrorInvalidValue;
#define ADAKV_C(K, C) if (kdt == K && cdt == C) return launch_d<K, C, true>(a, D, s);
  ADAKV_C(ADAKV_BF16, ADAKV_BF16) ADAKV_C(ADAKV_BF16, ADAKV_F32)
  ADAKV_C(ADAKV_F16, ADAKV_F16) ADAKV_C(ADAKV_F16, ADAKV_F32)
  ADAKV_C(ADAKV_F32, ADAKV_F32)
#undef ADAKV_C
  return hipErrorInvalidValue;
}

}  // namespace adakv
