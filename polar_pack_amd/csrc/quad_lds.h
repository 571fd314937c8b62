// LDS decode tables of the quad-pack kernels (quad_rows.hip, quad_mfma.hip): per code byte
// the norm and the (cos, sin) pairs of the three angles, replicated so that a wavefront's
// lookups are conflict-free (see quad_rows.hip for the layouts and their measurement).
#pragma once

#include "rows_common.h"

namespace pp {

constexpr uint32_t QLDS_BYTES = 0x28000;  // 160 KiB: all of a gfx950 CU's LDS  // 160 KiB: all of a gfx950 CU's LDS
// ------------------------------------------------------------------ LDS tables
struct LaneOff {
  uint32_t r, c1, c2, c3;
};

// LDS byte address of the table row of code byte B (3 = nq, 2 = q1, 1 = q2, 0 = q3):
// byte 1 of the address is the code byte, bytes 0 and 2 come from the lane constant.
template <int B>
__device__ __forceinline__ uint32_t perm_addr(uint32_t cw, uint32_t lane_off) {
  return __builtin_amdgcn_perm(cw, lane_off, 0x0C020000u | ((4u + B) << 8));
}

// q1 and q2 share one table.  [0, 64K): (cos,sin)(pi i/255) rows of 32 x 8 B;
// [64K, 128K): (cos,sin)(2 pi i/255); [128K, 160K): norm rows of 32 x 4 B.
struct LayShared {
  static __device__ __forceinline__ LaneOff lane(int l) {
    LaneOff o;
    o.r = 0x20000u | (4u * (l & 31));
    o.c1 = o.c2 = 8u * (l & 31);
    o.c3 = 0x10000u | (8u * (l & 31));
    return o;
  }
  static __device__ __forceinline__ uint32_t addr_r(uint32_t cw, const LaneOff& o) {
    return ((cw >> 17) & 0x7F80u) | o.r;
  }
  static __device__ __forceinline__ void build(char* lds, int e, int grp, int ngrp, const float (&v)[7]) {
    for (int j = grp; j < 32; j += ngrp) {
      *reinterpret_cast<float*>(lds + 0x20000 + e * 128 + 4 * j) = v[0];
      *reinterpret_cast<float2*>(lds + e * 256 + 8 * j) = make_float2(v[1], v[2]);
      *reinterpret_cast<float2*>(lds + 0x10000 + e * 256 + 8 * j) = make_float2(v[5], v[6]);
    }
  }
};

// Four tables.  [0, 64K): rows [norm x 32 (4 B) | (cos3,sin3) x 16 (8 B)];
// [64K, 128K): rows [(cos1,sin1) x 16 | (cos2,sin2) x 16].
struct LaySplit {
  static __device__ __forceinline__ LaneOff lane(int l) {
    LaneOff o;
    o.r = 4u * (l & 31);
    o.c3 = 128u + 8u * (l & 15);
    o.c1 = 0x10000u | (8u * (l & 15));
    o.c2 = 0x10000u | (128u + 8u * (l & 15));
    return o;
  }
  static __device__ __forceinline__ uint32_t addr_r(uint32_t cw, const LaneOff& o) { return perm_addr<3>(cw, o.r); }
  static __device__ __forceinline__ void build(char* lds, int e, int grp, int ngrp, const float (&v)[7]) {
    float* row0 = reinterpret_cast<float*>(lds + e * 256);
    float* row1 = reinterpret_cast<float*>(lds + 0x10000 + e * 256);
    for (int j = grp; j < 32; j += ngrp) row0[j] = v[0];
    for (int j = grp; j < 16; j += ngrp) {
      row0[32 + 2 * j] = v[5];
      row0[33 + 2 * j] = v[6];
      row1[2 * j] = v[1];
      row1[2 * j + 1] = v[2];
      row1[32 + 2 * j] = v[3];
      row1[33 + 2 * j] = v[4];
    }
  }
};

template <class L>
__device__ __forceinline__ void lookup(const char* lds, uint32_t cw, const LaneOff& o, float& r, float2& a, float2& b,
                                       float2& c) {
  r = *reinterpret_cast<const float*>(lds + L::addr_r(cw, o));
  a = *reinterpret_cast<const float2*>(lds + perm_addr<2>(cw, o.c1));
  b = *reinterpret_cast<const float2*>(lds + perm_addr<1>(cw, o.c2));
  c = *reinterpret_cast<const float2*>(lds + perm_addr<0>(cw, o.c3));
}

// Build the tables of a workgroup (all of its threads; blockDim.x a multiple of 256) from
// the 7 header LUTs (256 entries each, fp16 or fp32) into T (QLDS_BYTES).  Returns true
// for the shared layout (the t1 and t2 tables equal), false for the split one.
__device__ __forceinline__ bool quad_tables(uint32_t* T, const QuadLuts& luts) {
  char* lds = reinterpret_cast<char*>(T);
  const int e = threadIdx.x & 255, grp = threadIdx.x >> 8, ngrp = blockDim.x >> 8;
  float v[7];
  if (luts.dtype == PP_F16) {
#pragma unroll
    for (int i = 0; i < 7; ++i) v[i] = (float)reinterpret_cast<const f16*>(luts.p[i])[e];
  } else {
#pragma unroll
    for (int i = 0; i < 7; ++i) v[i] = reinterpret_cast<const float*>(luts.p[i])[e];
  }
  const bool same = __float_as_uint(v[1]) == __float_as_uint(v[3]) && __float_as_uint(v[2]) == __float_as_uint(v[4]);
  // workgroup-wide AND through the (not yet built) table memory: the tables fill all
  // of LDS, so there is no room for a separate flag
  if (threadIdx.x == 0) T[0] = 0u;
  __syncthreads();
  if (!same) T[0] = 1u;
  __syncthreads();
  const bool shared = T[0] == 0u;
  __syncthreads();
  if (shared) LayShared::build(lds, e, grp, ngrp, v);
  else LaySplit::build(lds, e, grp, ngrp, v);
  __syncthreads();
  return shared;
}

}  // namespace pp
