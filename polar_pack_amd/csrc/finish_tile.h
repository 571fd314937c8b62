// Finish pass of the K-sliced matrix-core kernels (quad_mfma.hip, quad_big.hip,
// dual_mfma.hip): the float32 slice sums to fp16 outputs.
#pragma once

#include "pp_common.h"

namespace pp {

// ------------------------------------------------------------------ slice sums
// Finish pass of the K-sliced matrix-core kernels: their items add scaled float32 sums
// into acc[m][n][j] (a wave's atomics for one row cover 16 consecutive tokens), the outputs
// are out_m[j, n] in fp16.  A 256-thread workgroup takes FIN_T rows x FIN_T tokens of one
// model (a = acc + m*N*M, o = out_m), reads and clears them along the tokens, transposes
// them through LDS and stores along the rows; vec: o_sm % 4 == 0 and o 8-byte aligned
// (4 rows per store).  acc 16-byte aligned.  Runs after the item kernel has completed, so
// its atomics are visible to plain loads, and leaves acc zero for the next launch.
constexpr int FIN_T = 64;
__host__ __device__ inline int64_t finish_tiles(int models, int64_t N, int64_t M) {
  return models * ((N + FIN_T - 1) / FIN_T) * ((M + FIN_T - 1) / FIN_T);
}
__device__ __forceinline__ void finish_tile(float* a, f16* o, int64_t o_sm, int N, int M, int n0, int j0, bool vec) {
  __shared__ float tile[FIN_T][FIN_T + 1];
  const int t = threadIdx.x, c4 = 4 * (t & 15), r16 = t >> 4;
  const bool full = n0 + FIN_T <= N && j0 + FIN_T <= M && M % 4 == 0;
#pragma unroll
  for (int p = 0; p < FIN_T / 16; ++p) {
    const int n = n0 + 16 * p + r16;
    float* src = a + (int64_t)n * M + j0 + c4;
    float v[4];
    if (full) {
      const float4 x = *reinterpret_cast<const float4*>(src);
      *reinterpret_cast<float4*>(src) = make_float4(0.f, 0.f, 0.f, 0.f);
      v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool in = n < N && j0 + c4 + e < M;
        v[e] = in ? src[e] : 0.f;
        if (in) src[e] = 0.f;
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[16 * p + r16][c4 + e] = v[e];
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < FIN_T / 16; ++p) {
    const int j = j0 + 16 * p + r16, n = n0 + c4;
    if (j >= M) continue;
    f16* dst = o + (int64_t)j * o_sm + n;
    const int jl = 16 * p + r16;
    const f16x4 h = {(f16)tile[c4][jl], (f16)tile[c4 + 1][jl], (f16)tile[c4 + 2][jl], (f16)tile[c4 + 3][jl]};
    if (vec && n + 3 < N) {
      *reinterpret_cast<f16x4*>(dst) = h;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < N) dst[e] = h[e];
    }
  }
}
// The (model, row block, token block) of finish workgroup b.
__device__ __forceinline__ void finish_coords(int N, int M, int& m, int& n0, int& j0) {
  const int tn = (N + FIN_T - 1) / FIN_T, tj = (M + FIN_T - 1) / FIN_T;
  const int b = (int)blockIdx.x;
  m = b / (tn * tj);
  const int r = b % (tn * tj);
  n0 = (r / tj) * FIN_T;
  j0 = (r % tj) * FIN_T;
}
// vec for finish_tile: every output 8-byte aligned and o_sm % 4 == 0.
inline bool finish_vec(void* const* out, int models, int64_t o_sm) {
  bool v = o_sm % 4 == 0;
  for (int m = 0; m < models; ++m) v = v && reinterpret_cast<uintptr_t>(out[m]) % 8 == 0;
  return v;
}

}  // namespace pp
