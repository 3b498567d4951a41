// Shared device helpers for the AdaKV gfx950 kernels: element types, 16-byte
// vector loads, wave64 / workgroup reductions and scans.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "adakv_amd.h"

namespace adakv {

constexpr int kWave = 64;
constexpr int kMaxBlocksDev = 32768;     // largest max_blocks the kernels are built for

// ---- element types ---------------------------------------------------------
// 16-byte vectors carry 4 fp32 or 8 fp16/bf16 elements.
template <int DT> struct Elt;
template <> struct Elt<ADAKV_F32> { static constexpr int kPerVec = 4; static constexpr int kBytes = 4; };
template <> struct Elt<ADAKV_F16> { static constexpr int kPerVec = 8; static constexpr int kBytes = 2; };
template <> struct Elt<ADAKV_BF16> { static constexpr int kPerVec = 8; static constexpr int kBytes = 2; };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;           // NaN stays NaN
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;                  // round to nearest even
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 x;
  uint16_t b = (uint16_t)h;
  __builtin_memcpy(&x, &b, 2);
  return (float)x;
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 x = (_Float16)f;                                       // round to nearest even
  uint16_t b;
  __builtin_memcpy(&b, &x, 2);
  return b;
}

// Unpack one 16-byte vector into fp32 values.
template <int DT>
__device__ __forceinline__ void unpack(const uint4& v, float* out) {
  if constexpr (DT == ADAKV_F32) {
    out[0] = __uint_as_float(v.x); out[1] = __uint_as_float(v.y);
    out[2] = __uint_as_float(v.z); out[3] = __uint_as_float(v.w);
  } else {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (DT == ADAKV_BF16) {
        out[2 * i] = __uint_as_float(w[i] << 16);
        out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      } else {
        out[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
        out[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
      }
    }
  }
}

// Element i of an array of compile-time type DT, widened to fp32.
template <int DT>
__device__ __forceinline__ float load_t(const void* p, int64_t i) {
  if constexpr (DT == ADAKV_F32) {
    return reinterpret_cast<const float*>(p)[i];
  } else {
    const uint16_t h = reinterpret_cast<const uint16_t*>(p)[i];
    if constexpr (DT == ADAKV_BF16) return bf16_bits_to_f32(h); else return f16_bits_to_f32(h);
  }
}

// Calls f(std::integral_constant<int, DT>) for the runtime dtype dt, so that
// the loads inside f are typed at compile time (a runtime type test between
// loads makes the compiler wait for each load before issuing the next).
template <typename F>
__device__ __forceinline__ void with_dtype(int dt, F&& f) {
  if (dt == ADAKV_BF16) f(std::integral_constant<int, ADAKV_BF16>{});
  else if (dt == ADAKV_F16) f(std::integral_constant<int, ADAKV_F16>{});
  else f(std::integral_constant<int, ADAKV_F32>{});
}

// Rows [G][D] of q (row g at element base + g * qsh) into LDS as fp32 times
// `scale`; all loads of a thread are issued before the first is consumed.
// SPLIT: the rows are [max(q, 0) | min(q, 0)] of q rows of D/2 elements (the
// query side of a minmax block summary).
template <int NT, int GMAX, int D, bool SPLIT = false>
__device__ __forceinline__ void stage_q(float (*s_q)[D], const void* q, int qdt, int64_t base, int64_t qsh,
                                        int G, float scale) {
  constexpr int IT = (GMAX * D + NT - 1) / NT;
  constexpr int DQ = SPLIT ? D / 2 : D;
  with_dtype(qdt, [&](auto tag) {
    constexpr int DT = decltype(tag)::value;
    float x[IT];
#pragma unroll
    for (int u = 0; u < IT; ++u) {
      const int i = min((int)threadIdx.x + u * NT, G * D - 1);     // in-bounds for every lane
      x[u] = load_t<DT>(q, base + (int64_t)(i / D) * qsh + (i % D) % DQ);
    }
#pragma unroll
    for (int u = 0; u < IT; ++u) {
      const int i = threadIdx.x + u * NT;
      float y = x[u];
      if constexpr (SPLIT) y = (i % D) < DQ ? fmaxf(y, 0.f) : fminf(y, 0.f);
      if (i < G * D) s_q[i / D][i % D] = y * scale;
    }
  });
}

// Scalar load of element i of a typed array (used for q and small tails).
__device__ __forceinline__ float load_elt(const void* p, int dt, int64_t i) {
  if (dt == ADAKV_F32) return reinterpret_cast<const float*>(p)[i];
  const uint16_t h = reinterpret_cast<const uint16_t*>(p)[i];
  return dt == ADAKV_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

__device__ __forceinline__ void store_elt(void* p, int dt, int64_t i, float x) {
  if (dt == ADAKV_F32) {
    reinterpret_cast<float*>(p)[i] = x;
  } else {
    reinterpret_cast<uint16_t*>(p)[i] =
        (uint16_t)(dt == ADAKV_BF16 ? f32_to_bf16_bits(x) : f32_to_f16_bits(x));
  }
}

__device__ __forceinline__ uint4 load16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// A 16-byte load of data read once (a streaming scan): non-temporal, so it
// does not displace what the caches hold for later kernels.
__device__ __forceinline__ uint4 load16_stream(const void* p) {
  typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// ---- kernel arguments ----------------------------------------------------------
// Scalar-cache warm-up of the first BYTES bytes (<= 768) of the kernel-argument
// segment: one scalar load per 64-byte line, issued back to back, then one
// wait.  The compiler issues argument loads where each value is first needed
// and waits on them in turn; on a cold scalar cache every such wait is a
// memory round trip (measured: 3 us before a fused step's first vector load).
// After this, those loads hit the cache.  Reads only.
template <int BYTES>
__device__ __forceinline__ void warm_kernargs() {
  static_assert(BYTES > 0 && BYTES <= 768, "up to 12 lines");
  constexpr int kLast = ((BYTES + 63) / 64 - 1) * 64;
#define ADAKV_KA_OFF(i) ((i) * 64 < kLast ? (i) * 64 : kLast)
  const char* p = (const char*)__builtin_amdgcn_kernarg_segment_ptr();
  int x0, x1, x2, x3, x4, x5, x6, x7, x8, x9, x10, x11;
  asm volatile(
      "s_load_dword %0, %12, %13\n\t"
      "s_load_dword %1, %12, %14\n\t"
      "s_load_dword %2, %12, %15\n\t"
      "s_load_dword %3, %12, %16\n\t"
      "s_load_dword %4, %12, %17\n\t"
      "s_load_dword %5, %12, %18\n\t"
      "s_load_dword %6, %12, %19\n\t"
      "s_load_dword %7, %12, %20\n\t"
      "s_load_dword %8, %12, %21\n\t"
      "s_load_dword %9, %12, %22\n\t"
      "s_load_dword %10, %12, %23\n\t"
      "s_load_dword %11, %12, %24\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=s"(x0), "=s"(x1), "=s"(x2), "=s"(x3), "=s"(x4), "=s"(x5), "=s"(x6), "=s"(x7), "=s"(x8), "=s"(x9),
        "=s"(x10), "=s"(x11)
      : "s"(p), "i"(ADAKV_KA_OFF(0)), "i"(ADAKV_KA_OFF(1)), "i"(ADAKV_KA_OFF(2)), "i"(ADAKV_KA_OFF(3)),
        "i"(ADAKV_KA_OFF(4)), "i"(ADAKV_KA_OFF(5)), "i"(ADAKV_KA_OFF(6)), "i"(ADAKV_KA_OFF(7)),
        "i"(ADAKV_KA_OFF(8)), "i"(ADAKV_KA_OFF(9)), "i"(ADAKV_KA_OFF(10)), "i"(ADAKV_KA_OFF(11)));
#undef ADAKV_KA_OFF
}

// ---- cross-lane data movement --------------------------------------------------
// DPP moves (full-rate VALU, no LDS traffic).  Controls: quad_perm [1,0,3,2] = 0xB1,
// quad_perm [2,3,0,1] = 0x4E, row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// Sum over each aligned group of N lanes (N a power of two <= 64); every lane
// of the group receives the group's sum.  Must be reached by all 64 lanes.
// Values of a lane and its partner across 16-lane rows (xor 16) or wave
// halves (xor 32), in an order that is the same for both partners; any
// symmetric combine of the pair gives both lanes the same result.
struct LanePair { float a, b; };
__device__ __forceinline__ LanePair swap16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ LanePair swap32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return {__uint_as_float(r[0]), __uint_as_float(r[1])};
}

template <int N>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (N >= 2) x += dpp_mov<0xB1>(x);
  if constexpr (N >= 4) x += dpp_mov<0x4E>(x);
  if constexpr (N >= 8) x += dpp_mov<0x141>(x);
  if constexpr (N >= 16) x += dpp_mov<0x140>(x);
  if constexpr (N >= 32) { const LanePair p = swap16(x); x = p.a + p.b; }
  if constexpr (N >= 64) { const LanePair p = swap32(x); x = p.a + p.b; }
  return x;
}

// All-lane reductions over the whole wave (every lane receives the result).
template <typename Op>
__device__ __forceinline__ float wave_allreduce(float x, Op op) {
  x = op(x, dpp_mov<0xB1>(x));
  x = op(x, dpp_mov<0x4E>(x));
  x = op(x, dpp_mov<0x141>(x));
  x = op(x, dpp_mov<0x140>(x));
  LanePair p = swap16(x);
  x = op(p.a, p.b);
  p = swap32(x);
  return op(p.a, p.b);
}

// ---- wave64 reductions -------------------------------------------------------
// Sum over the wave (every lane receives it) of a 4- or 8-byte value: the
// DPP / permlane butterfly of group_sum on each 32-bit half (a __shfl_xor
// butterfly goes through ds_bpermute: one LDS round trip per step and half).
// Every lane adds the same two terms at each step, so all lanes agree.
template <typename T>
__device__ __forceinline__ T wave_sum(T x) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit values");
  using U = typename std::conditional<sizeof(T) == 8, uint64_t, uint32_t>::type;
  auto mov = [](T v, auto ctrl) -> T {
    constexpr int C = decltype(ctrl)::value;
    const U u = __builtin_bit_cast(U, v);
    U r = (U)__float_as_uint(dpp_mov<C>(__uint_as_float((uint32_t)u)));
    if constexpr (sizeof(T) == 8)
      r |= (U)__float_as_uint(dpp_mov<C>(__uint_as_float((uint32_t)(u >> 32)))) << 32;
    return __builtin_bit_cast(T, r);
  };
  auto swap_add = [](T v, bool wide) -> T {
    const U u = __builtin_bit_cast(U, v);
    auto sw = [&](uint32_t h) {
      return wide ? __builtin_amdgcn_permlane32_swap(h, h, false, false)
                  : __builtin_amdgcn_permlane16_swap(h, h, false, false);
    };
    const auto lo = sw((uint32_t)u);
    U a = (U)lo[0], b = (U)lo[1];
    if constexpr (sizeof(T) == 8) {
      const auto hi = sw((uint32_t)(u >> 32));
      a |= (U)hi[0] << 32;
      b |= (U)hi[1] << 32;
    }
    return __builtin_bit_cast(T, a) + __builtin_bit_cast(T, b);
  };
  x += mov(x, std::integral_constant<int, 0xB1>{});
  x += mov(x, std::integral_constant<int, 0x4E>{});
  x += mov(x, std::integral_constant<int, 0x141>{});
  x += mov(x, std::integral_constant<int, 0x140>{});
  x = swap_add(x, false);
  return swap_add(x, true);
}
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}
__device__ __forceinline__ float wave_min(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = fminf(x, __shfl_xor(x, o));
  return x;
}

// Inclusive prefix sum over the 64 lanes of a wave: a Hillis-Steele scan
// inside each 16-lane row with DPP row shifts (lanes shifted in from outside
// the row read 0), then the totals of the lower rows added from lanes 15, 31
// and 47.  No LDS traffic.
template <int CTRL>
__device__ __forceinline__ int dpp_row_shr(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ int wave_incl_scan(int x) {
  const int lane = threadIdx.x & (kWave - 1);
  x += dpp_row_shr<0x111>(x);
  x += dpp_row_shr<0x112>(x);
  x += dpp_row_shr<0x114>(x);
  x += dpp_row_shr<0x118>(x);
  const int r0 = __builtin_amdgcn_readlane(x, 15);
  const int r1 = __builtin_amdgcn_readlane(x, 31);
  const int r2 = __builtin_amdgcn_readlane(x, 47);
  const int row = lane >> 4;
  return x + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

// Workgroup barrier for data exchanged through LDS only: it waits for this
// wave's LDS operations but not for its outstanding global loads (the
// workgroup fence of __syncthreads waits for those too), so loads issued
// before it stay in flight.  The memory clobber keeps the compiler from moving
// memory accesses across it.  Not for global-memory hand-offs between waves.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ---- workgroup reductions (NT threads, scratch of >= NT/64 slots) ------------
// All-lane reduction over the wave of a 4-byte value with a symmetric op
// (DPP moves, then the permlane swaps; no LDS traffic).
template <typename T, typename Op>
__device__ __forceinline__ T wave_allreduce_b32(T x, Op op) {
  static_assert(sizeof(T) == 4, "4-byte values");
  auto mov = [](T v, auto ctrl) -> T {
    constexpr int C = decltype(ctrl)::value;
    return __builtin_bit_cast(T, __float_as_uint(dpp_mov<C>(__uint_as_float(__builtin_bit_cast(uint32_t, v)))));
  };
  x = op(x, mov(x, std::integral_constant<int, 0xB1>{}));
  x = op(x, mov(x, std::integral_constant<int, 0x4E>{}));
  x = op(x, mov(x, std::integral_constant<int, 0x141>{}));
  x = op(x, mov(x, std::integral_constant<int, 0x140>{}));
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  x = op(__builtin_bit_cast(T, (uint32_t)r16[0]), __builtin_bit_cast(T, (uint32_t)r16[1]));
  u = __builtin_bit_cast(uint32_t, x);
  const auto r32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return op(__builtin_bit_cast(T, (uint32_t)r32[0]), __builtin_bit_cast(T, (uint32_t)r32[1]));
}

template <int NT, typename T, typename Op>
__device__ __forceinline__ T block_reduce(T x, T* scratch, Op op) {
  constexpr int NW = NT / kWave;
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  x = wave_allreduce_b32(x, op);
  __syncthreads();
  if (lane == 0) scratch[w] = x;
  __syncthreads();
  T r = scratch[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = op(r, scratch[i]);
  return r;
}

struct OpAdd { template <typename T> __device__ T operator()(T a, T b) const { return a + b; } };
struct OpMax { __device__ float operator()(float a, float b) const { return fmaxf(a, b); } };
struct OpMin { __device__ float operator()(float a, float b) const { return fminf(a, b); } };

// Exclusive prefix sum over the workgroup; returns this thread's offset and the total.
template <int NT>
__device__ __forceinline__ int block_excl_scan(int x, int* scratch, int* total) {
  constexpr int NW = NT / kWave;
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int inc = wave_incl_scan(x);
  __syncthreads();
  if (lane == kWave - 1) scratch[w] = inc;
  __syncthreads();
  int base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const int s = scratch[i];
    base += (i < w) ? s : 0;
    tot += s;
  }
  *total = tot;
  return base + inc - x;
}

// Agent-scope publication helpers for the "last workgroup to arrive" hand-offs.
__device__ __forceinline__ int arrive(int* counter) {
  __threadfence();
  return __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void reset_counter(int* counter) {
  __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

// ---- per-head block budget (adakv/budget.py:45-86, adakv/selector.py:49-52) -----
// The bounds exactly as sparse_attention feeds them to the allocator and the
// selector (adakv/reference.py:71-74): k_min and k_max are first clipped to nb,
// the allocator floor is sink + local + c_min, the selector floor is the same
// clipped to nb.
struct BudgetCfg {
  double avg;
  int k_min, k_max, sink, local, c_min, policy;
  double temperature;
  float nucleus_p;             // the nucleus policy's mass target, rounded to fp32 as NumPy compares it
};

struct Bounds {
  int nb, sink, local, n_forced, floor_sel, lo, hi, kmin_a, kcap;
  double target;
};

__device__ __forceinline__ Bounds budget_bounds(int nb, const BudgetCfg& p) {
  Bounds r;
  r.nb = nb;
  r.kmin_a = min(p.k_min, nb);
  r.hi = min(p.k_max, nb);
  r.sink = min(p.sink, nb);
  r.local = min(p.local, nb);
  r.lo = min(max(max(r.sink + r.local + p.c_min, r.kmin_a), 1), nb);
  r.target = fmin(fmax(p.avg, (double)r.lo), (double)r.hi);   // np.clip: hi wins when lo > hi
  r.floor_sel = min(r.sink + r.local + p.c_min, nb);
  r.n_forced = min(r.sink + r.local, nb);
  // the largest count any head can receive: k <= hi for every policy, then the floor
  r.kcap = nb <= 1 ? nb : min(max(r.hi, r.floor_sel), nb);
  return r;
}

// Selected-block count of one head given its weight w and the sequence's sum of
// weights (fp64, as NumPy promotes after dividing by np.log(nb) or counting
// the nucleus); round half to even.  Every policy but fixed shares the formula.
__device__ __forceinline__ int head_count(const Bounds& r, int policy, double w, double wsum, int Hq) {
  int k;
  if (r.nb <= 1) {
    k = min(max(r.kmin_a, 1), r.nb);
  } else if (policy == ADAKV_POLICY_FIXED) {
    k = (int)rint(r.target);
  } else {
    const double surplus = fmax(r.target - (double)r.lo, 0.0) * (double)Hq;
    const double x = rint((double)r.lo + surplus * w / fmax(wsum, 1e-9));
    k = (int)fmin(fmax(x, (double)r.lo), (double)r.hi);
  }
  return min(max(k, r.floor_sel), r.nb);
}

// NumPy's pairwise summation of a contiguous fp64 array (8 accumulators for
// blocks of <= 128 elements, halving above), so that the device reproduces
// w.sum() of adakv/budget.py:84 bit for bit.
__device__ __forceinline__ double pairwise_block(const double* a, int n) {   // n <= 128
  if (n < 8) {
    double r = 0.0;
    for (int i = 0; i < n; ++i) r += a[i];
    return r;
  }
  double r[8];
  for (int j = 0; j < 8; ++j) r[j] = a[j];
  int i = 8;
  for (; i < n - (n % 8); i += 8)
    for (int j = 0; j < 8; ++j) r[j] += a[i + j];
  double res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (; i < n; ++i) res += a[i];
  return res;
}
template <int DEPTH>
__device__ double numpy_pairwise_sum(const double* a, int n) {
  if (n <= 128 || DEPTH == 0) return pairwise_block(a, n);
  int n2 = n / 2;
  n2 -= n2 % 8;
  if constexpr (DEPTH > 0)
    return numpy_pairwise_sum<DEPTH - 1>(a, n2) + numpy_pairwise_sum<DEPTH - 1>(a + n2, n - n2);
  return 0.0;
}

// True token count of sequence b, clamped to the capacity of the K/V views so
// that a bad length can never move an access out of bounds.
__device__ __forceinline__ int seq_len_of(const int32_t* seq_lens, int capacity, int b) {
  return seq_lens ? min(max(seq_lens[b], 0), capacity) : capacity;
}

}  // namespace adakv
