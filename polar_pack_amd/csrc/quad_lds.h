// LDS decode tables of the quad-pack kernels (quad_rows.hip, quad_mfma.hip): per code byte
// the norm and the (cos, sin) pairs of the three angles, replicated so that a wavefront's
// lookups are conflict-free (see quad_rows.hip for the layouts and their measurement).
#pragma once

#include "rows_common.h"

namespace pp {

constexpr uint32_t QLDS_BYTES = 0x28000;  // 160 KiB: all of a gfx950 CU's LDS
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

// Entry e of header LUT i, stored as E (fp16 or float32).
template <typename E>
__device__ __forceinline__ float lut_val(const QuadLuts& L, int i, int e) {
  return (float)reinterpret_cast<const E*>(L.p[i])[e];
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
  // 16-byte units in address order, so that a wavefront's 64 stores fill 1 KiB of
  // consecutive banks (a row-per-thread order puts all 64 lanes of a store on one bank).
  // The LUT loads (load) are issued before the layout check, the stores (store) after.
  template <int NT>
  struct Units {
    static constexpr int KN = 2048 / NT, KC = 4096 / NT;       // norm: 8 units per entry, (cos, sin): 16
    float r[KN], c1[KC], s1[KC], c3[KC], s3[KC];
    template <typename E>
    __device__ __forceinline__ void load(const QuadLuts& L) {
#pragma unroll
      for (int k = 0; k < KN; ++k) r[k] = lut_val<E>(L, 0, (threadIdx.x + k * NT) >> 3);
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        const int e = (threadIdx.x + k * NT) >> 4;
        c1[k] = lut_val<E>(L, 1, e);
        s1[k] = lut_val<E>(L, 2, e);
        c3[k] = lut_val<E>(L, 5, e);
        s3[k] = lut_val<E>(L, 6, e);
      }
    }
    __device__ __forceinline__ void store(char* lds) const {
#pragma unroll
      for (int k = 0; k < KN; ++k)
        *reinterpret_cast<float4*>(lds + 0x20000 + 16 * (threadIdx.x + k * NT)) = make_float4(r[k], r[k], r[k], r[k]);
#pragma unroll
      for (int k = 0; k < KC; ++k) {
        const int u = threadIdx.x + k * NT;
        *reinterpret_cast<float4*>(lds + 16 * u) = make_float4(c1[k], s1[k], c1[k], s1[k]);
        *reinterpret_cast<float4*>(lds + 0x10000 + 16 * u) = make_float4(c3[k], s3[k], c3[k], s3[k]);
      }
    }
  };
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
  template <int NT, typename E>
  static __device__ __forceinline__ void build(char* lds, const QuadLuts& L) {
    constexpr int KU = 8192 / NT;                                // 16 units per row, in address order
    float a[KU], b[KU];
#pragma unroll
    for (int k = 0; k < KU; ++k) {
      const int u = threadIdx.x + k * NT;
      const int reg = u >> 12, e = (u >> 4) & 255, c = u & 15;
      const int t = reg == 0 ? (c < 8 ? 0 : 5) : (c < 8 ? 1 : 3);
      a[k] = lut_val<E>(L, t, e);
      b[k] = lut_val<E>(L, t == 0 ? 0 : t + 1, e);
    }
#pragma unroll
    for (int k = 0; k < KU; ++k) {
      const int u = threadIdx.x + k * NT;
      *reinterpret_cast<float4*>(lds + ((u >> 12) << 16) + 16 * (u & 4095)) = make_float4(a[k], b[k], a[k], b[k]);
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

// Build the tables of a workgroup (all NT threads; NT a multiple of 256) from the 7
// header LUTs (256 entries each, of type E) into T (QLDS_BYTES), in two steps so that a
// kernel can issue other loads between them: load() issues every LUT load of the shared
// layout (and those of the layout check), finish() checks the layout across the workgroup,
// stores the tables and waits for them; it returns true for the shared layout (the t1 and
// t2 tables equal), false for the split one.
template <int NT, typename E>
struct QuadTableBuild {
  static_assert(NT % 256 == 0, "the table build takes a multiple of 256 threads");
  float v[4];
  LayShared::Units<NT> U;
  __device__ __forceinline__ void load(const QuadLuts& luts) {
    const int e = threadIdx.x & 255;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = lut_val<E>(luts, 1 + i, e);
    U.template load<E>(luts);
  }
  // Whether this thread's q1 and q2 entries agree (waits for the first LUT loads only).
  __device__ __forceinline__ bool same() const {
    return __float_as_uint(v[0]) == __float_as_uint(v[2]) && __float_as_uint(v[1]) == __float_as_uint(v[3]);
  }
  __device__ __forceinline__ bool finish(uint32_t* T, const QuadLuts& luts) { return finish(T, luts, same()); }
  __device__ __forceinline__ bool finish(uint32_t* T, const QuadLuts& luts, bool same) {
    char* lds = reinterpret_cast<char*>(T);
    // workgroup-wide AND through the (not yet built) table memory: the tables fill all
    // of LDS, so there is no room for a separate flag
    if (threadIdx.x == 0) T[0] = 0u;
    __syncthreads();
    if (!same) T[0] = 1u;
    __syncthreads();
    const bool shared = T[0] == 0u;
    __syncthreads();
    if (shared) U.store(lds);
    else LaySplit::build<NT, E>(lds, luts);
    __syncthreads();
    return shared;
  }
};

template <int NT, typename E>
__device__ __forceinline__ bool quad_tables_of(uint32_t* T, const QuadLuts& luts) {
  QuadTableBuild<NT, E> b;
  b.load(luts);
  return b.finish(T, luts);
}

template <int NT>
__device__ __forceinline__ bool quad_tables(uint32_t* T, const QuadLuts& luts) {
  return luts.dtype == PP_F16 ? quad_tables_of<NT, f16>(T, luts) : quad_tables_of<NT, float>(T, luts);
}

}  // namespace pp
