// Shared helpers for the polar_pack gfx950 kernels: status/error plumbing,
// vector types, fp16 helpers and the LDS lookup tables of the quad decode.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <mutex>
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
// The current device's side stream with a fork and a join event (see capi.hip), and the
// lock that a fork / side launch / join sequence is enqueued under.
int side_stream(hipStream_t* side, hipEvent_t* fork, hipEvent_t* join);
std::mutex& side_lock();

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

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  return reinterpret_cast<T*>(uniform64(reinterpret_cast<int64_t>(p)));
}

__device__ __forceinline__ int64_t lane_read64(int64_t v, int lane) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, lane);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)v >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
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

// Fill the replicated tables: thread t owns entry t % 256 and every (blockDim/256)-th
// replica; all 7 LUT loads of a thread are issued before any LDS write, so the build
// costs one memory round trip.  blockDim.x must be a multiple of 256.
template <int REPL_R, int REPL_C>
__device__ __forceinline__ void quad_build_lds(QuadLds<REPL_R, REPL_C>& T, const QuadLuts& L) {
  const int e = threadIdx.x & 255;
  const int grp = threadIdx.x >> 8, ngrp = blockDim.x >> 8;
  float v[7];
  if (L.dtype == PP_F16) {
    f16 h[7];
#pragma unroll
    for (int i = 0; i < 7; ++i) h[i] = reinterpret_cast<const f16*>(L.p[i])[e];
#pragma unroll
    for (int i = 0; i < 7; ++i) v[i] = (float)h[i];
  } else {
#pragma unroll
    for (int i = 0; i < 7; ++i) v[i] = reinterpret_cast<const float*>(L.p[i])[e];
  }
  for (int j = grp; j < REPL_R; j += ngrp) T.r[e * REPL_R + j] = v[0];
  for (int j = grp; j < REPL_C; j += ngrp) {
    T.cs1[e * REPL_C + j] = make_float2(v[1], v[2]);
    T.cs2[e * REPL_C + j] = make_float2(v[3], v[4]);
    T.cs3[e * REPL_C + j] = make_float2(v[5], v[6]);
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
