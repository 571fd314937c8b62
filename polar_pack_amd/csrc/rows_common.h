// Device helpers shared by the fused row kernels (quad_rows.hip, dual_rows.hip):
// buffer resources and compiler-tracked buffer loads/stores, the transposing wave
// reduction, and the step cursor of a segment walk.
#pragma once

#include "pp_common.h"

#include <algorithm>

namespace pp {

constexpr int NT_AUX = 2;                 // non-temporal cache policy for streamed codes
constexpr uint32_t OOB = 0x80000000u;     // buffer offset past any num_records: reads 0

// Buffer resource (V#): base, stride 0, num_records bytes.  Offsets at or past
// num_records read 0 and drop writes.  The fields go through readfirstlane so the
// resource lives in scalar registers.
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* u = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// Loads and stores of the decode loop.  They are compiler-visible buffer operations:
// the compiler tracks every outstanding load and waits for it before the first
// instruction that reads the register (including any register copy it inserts), so the
// pipeline below only has to keep the number of memory operations per step fixed and
// avoid reading a result early.
__device__ __forceinline__ void vload128(u32x4& d, uint32_t off, rsrc_t r) {
  d = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, NT_AUX);
}
// The same without the streaming cache policy: for data that many wavefronts re-read
// (activations), which should stay in the caches.
__device__ __forceinline__ void vload128c(u32x4& d, uint32_t off, rsrc_t r) {
  d = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}
__device__ __forceinline__ void vload64(u32x2& d, uint32_t off, rsrc_t r) {
  d = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
}
__device__ __forceinline__ void vload32(uint32_t& d, uint32_t off, rsrc_t r) {
  d = __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ __forceinline__ void vload16(uint32_t& d, uint32_t off, rsrc_t r) {
  d = __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}
__device__ __forceinline__ void vstore16(uint32_t v, uint32_t off, rsrc_t r) {
  __builtin_amdgcn_raw_buffer_store_b16((unsigned short)v, r, (int)off, 0, 0);
}
__device__ __forceinline__ float h2f(uint32_t bits) { return (float)__builtin_bit_cast(f16, (unsigned short)bits); }

// ------------------------------------------------------------------ reduction
template <int P>
__device__ __forceinline__ float dpp_partner(float v) {
  // partner across lane bit P: 3 -> row_ror:8, 2 -> row_half_mirror, 1 -> quad_perm
  // [2,3,0,1], 0 -> quad_perm [1,0,3,2]
  constexpr int ctrl = P == 3 ? 0x128 : P == 2 ? 0x141 : P == 1 ? 0x4E : 0xB1;
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false));
}

// One halving step over lane bit P on C values: lanes with the bit clear keep
// v[i] + partner's v[i], lanes with it set keep v[i + C/2] + partner's v[i + C/2].
template <int P, int C>
__device__ __forceinline__ void halve(float* v, int lane) {
  constexpr int H = C / 2;
#pragma unroll
  for (int i = 0; i < H; ++i) {
    if constexpr (P == 5) {
      // swap(a, b): a' = (a_lo, b_lo), b' = (a_hi, b_hi) over the wave halves
      const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + H]), false, false);
      v[i] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    } else if constexpr (P == 4) {
      // swap(a, b): a' = rows (a0, b0, a2, b2), b' = rows (a1, b1, a3, b3)
      const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + H]), false, false);
      v[i] = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    } else {
      const bool hi = (lane >> P) & 1;
      const float send = hi ? v[i] : v[i + H];
      const float keep = hi ? v[i + H] : v[i];
      v[i] = keep + dpp_partner<P>(send);
    }
  }
}

// Sum v[0] over lane bits [0, NB).
template <int NB>
__device__ __forceinline__ float sum_low_bits(float v) {
  if constexpr (NB >= 3) v += dpp_partner<2>(v);
  if constexpr (NB >= 2) v += dpp_partner<1>(v);
  if constexpr (NB >= 1) v += dpp_partner<0>(v);
  return v;
}

// Reduce NV = 2^LNV values per lane over the wave; afterwards the lanes whose low
// (6 - LNV) bits are zero hold value (lane >> (6 - LNV)) in v[0].
template <int LNV>
__device__ __forceinline__ float wave_transpose_reduce(float* v, int lane) {
  static_assert(LNV >= 3 && LNV <= 6, "the reduction assumes 8..64 values per lane");
  if constexpr (LNV >= 1) halve<5, (1 << LNV)>(v, lane);
  if constexpr (LNV >= 2) halve<4, (1 << (LNV - 1))>(v, lane);
  if constexpr (LNV >= 3) halve<3, (1 << (LNV - 2))>(v, lane);
  if constexpr (LNV >= 4) halve<2, (1 << (LNV - 3))>(v, lane);
  if constexpr (LNV >= 5) halve<1, (1 << (LNV - 4))>(v, lane);
  if constexpr (LNV >= 6) halve<0, (1 << (LNV - 5))>(v, lane);
  return sum_low_bits<6 - LNV>(v[0]);
}

template <int N>
struct Log2 {
  static constexpr int v = N <= 1 ? 0 : 1 + Log2<N / 2>::v;
};
template <>
struct Log2<1> {
  static constexpr int v = 0;
};

// A wavefront's segment range [seg_bounds[gw], seg_bounds[gw + 1]) (seg_bounds holds
// n_waves + 1 entries).  issue() starts vector loads, so the round trip runs under the
// LDS table build instead of before it (a scalar load there would be waited for by the
// kernel-argument loads that follow it); lo() / hi() wait for them.
struct SegRange {
  u32x2 b0 = {0u, 0u}, b1 = {0u, 0u};
  __device__ __forceinline__ void issue(const int64_t* seg_bounds, int64_t gw, int64_t n_waves) {
    const rsrc_t r = make_rsrc(seg_bounds, 8u * (uint32_t)(n_waves + 1));
    vload64(b0, 8u * (uint32_t)gw, r);
    vload64(b1, 8u * (uint32_t)gw + 8u, r);
  }
  __device__ __forceinline__ int64_t lo() const { return uniform64((int64_t)(((uint64_t)b0[1] << 32) | b0[0])); }
  __device__ __forceinline__ int64_t hi() const { return uniform64((int64_t)(((uint64_t)b1[1] << 32) | b1[0])); }
};

// Cursor over the steps (task ti, chunk ck) of a segment.
struct Cursor {
  int ti, ck;
};

}  // namespace pp
