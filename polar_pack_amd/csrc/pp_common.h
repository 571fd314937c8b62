// Shared helpers for the polar_pack gfx950 kernels: status/error plumbing,
// vector types, fp16 helpers and the LDS lookup tables of the quad decode.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/polar_pack.h"

namespace pp {

// ---------------------------------------------------------------- host side
void set_error(const char* fmt, ...);

#define PP_REQUIRE(cond, ...)                 \
  do {                                        \
    if (!(cond)) {                            \
      ::pp::set_error(__VA_ARGS__);           \
      return PP_EINVAL;                       \
    }                                         \
  } while (0)

#define PP_HIP(call)                                                              \
  do {                                                                            \
    hipError_t e_ = (call);                                                       \
    if (e_ != hipSuccess) {                                                       \
      ::pp::set_error("%s failed: %s (%s:%d)", #call, hipGetErrorString(e_),      \
                      __FILE__, __LINE__);                                        \
      return PP_EHIP;                                                             \
    }                                                                             \
  } while (0)

#define PP_LAUNCH_CHECK() PP_HIP(hipGetLastError())

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int device_cu_count();  // cached per device

// ---------------------------------------------------------------- device side
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float lut_at(const void* p, int dtype, int i) {
  return dtype == PP_F16 ? (float)reinterpret_cast<const f16*>(p)[i]
                         : reinterpret_cast<const float*>(p)[i];
}

__device__ __forceinline__ u32x4 load_nt(const uint32_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Quad decode LUTs in LDS, each table replicated REPL times so that lanes that
// share a clock on the LDS crossbar read distinct banks whatever the codes are.
// Entry e of a table lives at [e][replica]; a lane reads replica lane % REPL.
template <int REPL_R, int REPL_C>
struct QuadLds {
  float r[256 * REPL_R];
  float2 cs1[256 * REPL_C];
  float2 cs2[256 * REPL_C];
  float2 cs3[256 * REPL_C];
};

struct QuadLuts {
  const void* p[7];  // norm, cos1, sin1, cos2, sin2, cos3, sin3
  int dtype;
};

template <int REPL_R, int REPL_C>
__device__ __forceinline__ void quad_build_lds(QuadLds<REPL_R, REPL_C>& T, const QuadLuts& L) {
  for (int i = threadIdx.x; i < 256 * REPL_R; i += blockDim.x) T.r[i] = lut_at(L.p[0], L.dtype, i / REPL_R);
  for (int i = threadIdx.x; i < 256 * REPL_C; i += blockDim.x) {
    const int e = i / REPL_C;
    T.cs1[i] = make_float2(lut_at(L.p[1], L.dtype, e), lut_at(L.p[2], L.dtype, e));
    T.cs2[i] = make_float2(lut_at(L.p[3], L.dtype, e), lut_at(L.p[4], L.dtype, e));
    T.cs3[i] = make_float2(lut_at(L.p[5], L.dtype, e), lut_at(L.p[6], L.dtype, e));
  }
}

// Normalised 4-tuple of one code word (w0..w3 before the RMS scale).
template <int REPL_R, int REPL_C>
__device__ __forceinline__ void quad_decode(const QuadLds<REPL_R, REPL_C>& T, uint32_t cw, int rr, int rc,
                                            float& w0, float& w1, float& w2, float& w3) {
  const float r = T.r[(cw >> 24) * REPL_R + rr];
  const float2 a = T.cs1[((cw >> 16) & 255u) * REPL_C + rc];
  const float2 b = T.cs2[((cw >> 8) & 255u) * REPL_C + rc];
  const float2 c = T.cs3[(cw & 255u) * REPL_C + rc];
  const float rs = r * a.y;
  const float rss = rs * b.y;
  w0 = r * a.x;
  w1 = rs * b.x;
  w2 = rss * c.x;
  w3 = rss * c.y;
}

}  // namespace pp
