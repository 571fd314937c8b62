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

// One-Linear launches (quad_rows.hip, dual_rows.hip): wave gw's column slice and run of row
// tasks, from the launch shape alone (no descriptor to read).  The slices take whole chunks,
// dealt as evenly as possible (slice s: chunks [s*C/parts, (s+1)*C/parts)); the waves are dealt
// to the slices alike (slice s: waves [s*W/parts, (s+1)*W/parts)).  A slice with at least as
// many tasks as waves gives its j-th wave q or q + 1 of its T tasks (q = T / nw, the first
// T % nw waves one more); one with fewer gives each workgroup the tasks an even spread gives
// its waves, one per wave from its lowest slot (slots 0 .. G/2-1 are on distinct SIMDs).
// 32-bit arithmetic (W < 2^16, T < 2^31, parts * C < 2^31): the wave computes this before
// issuing its first chunk, and 64-bit divisions there cost ~1,200 instructions.
struct DirectItem {
  int t0, t1, kbeg, kend;
};
template <int G>
__device__ __host__ __forceinline__ DirectItem direct_item(uint32_t gw, uint32_t W, uint32_t T, uint32_t parts,
                                                           uint32_t n_chunks, uint32_t chunk, uint32_t K) {
  const uint32_t s = ((gw + 1) * parts - 1) / W;      // the slice whose waves hold gw
  const uint32_t w0 = s * W / parts, w1 = (s + 1) * W / parts;
  const uint32_t j = gw - w0, nw = w1 - w0;
  DirectItem d;
  if (T >= nw) {
    const uint32_t q = T / nw, r = T - q * nw;
    d.t0 = (int)(j * q + std::min(j, r));
    d.t1 = d.t0 + (int)(q + (j < r ? 1u : 0u));
  } else {
    // each workgroup takes the tasks an even spread gives its waves, on its lowest slots
    // (gate_proj 11008x2048 at one token, 1,376 tasks for 2,048 waves: 22.9 us; 23.0 with the
    // tasks spread over the slots too; 27.6 with all first half-waves taken before any second
    // one, which gives a third of the workgroups twice the tasks of the rest)
    const uint32_t g0 = gw / G * G;
    const uint32_t a = std::max(g0, w0) - w0, b = std::min(g0 + G, w1) - w0;
    const uint32_t fa = a * T / nw, fb = b * T / nw, p = j - a;
    d.t0 = (int)std::min(fa + p, fb);
    d.t1 = (int)std::min(fa + p + 1, fb);
  }
  d.kbeg = (int)(s * n_chunks / parts * chunk);
  d.kend = (int)std::min<uint32_t>(K, (s + 1) * n_chunks / parts * chunk);
  return d;
}

// The K parts of a task in one workgroup (parts divides G, T * parts <= W): wave w of
// workgroup b takes part w % parts of task b + grid * (w / parts), so every workgroup gets a
// task before any gets two and the parts' sums can meet in the workgroup's LDS.
template <int G>
__device__ __host__ __forceinline__ DirectItem wg_item(uint32_t block, uint32_t grid, uint32_t wave, uint32_t T,
                                                       uint32_t parts, uint32_t n_chunks, uint32_t chunk, uint32_t K) {
  const uint32_t s = wave % parts, t = block + grid * (wave / parts);
  DirectItem d;
  d.t0 = (int)std::min(t, T);
  d.t1 = (int)std::min(t + 1, T);
  d.kbeg = (int)(s * n_chunks / parts * chunk);
  d.kend = (int)std::min<uint32_t>(K, (s + 1) * n_chunks / parts * chunk);
  return d;
}

// Whether the K parts of a one-Linear launch meet in LDS (wg_item) rather than through the
// workspace: a power of two that divides the workgroup's waves, one task per part group.
inline bool wg_parts_ok(int64_t T, int64_t W, int parts, int waves_per_wg) {
  return parts > 1 && waves_per_wg % parts == 0 && (parts & (parts - 1)) == 0 && T * parts <= W;
}

// Column slices of one Linear's T row tasks for W wavefronts and C chunks (the stream
// planner's rule, stream.split_factors): r = W / T; r < 1.5 whole rows; 1.5 <= r < 4 two
// slices when K holds at least 8 chunks; r >= 4 ceil(r / 2) slices, at most one per chunk.
inline int direct_parts(int64_t T, int64_t W, int64_t C) {
  int64_t want = 1;
  if (T > 0) {
    if (W >= 4 * T) want = (W + 2 * T - 1) / (2 * T);
    else if (2 * W >= 3 * T) want = C >= 8 ? 2 : 1;
  }
  return (int)std::max<int64_t>(1, std::min<int64_t>(want, C));
}

}  // namespace pp
