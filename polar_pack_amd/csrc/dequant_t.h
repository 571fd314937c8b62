// Decode into transposed fp16 weights: codes (K,N) with unit column stride (the layouts
// pack_quad_layer and quantize_polar_bitpacked return) -> weights (N,K) row-major, the
// operand a library GEMM multiplies fastest (a @ W as a @ (W^T)^T: 63 against 69 us for two
// 1024 x 4096 x 4096 products, 22 against 33 us at 128 tokens, measured).
//
// A workgroup of 256 threads walks tiles of 64 k x 64 n: each thread decodes 8 consecutive
// codes of a row (one 16-byte load per 8 dual codes, two per 8 quad codes) into LDS, the
// tile transposed; then each thread writes 16-byte runs of 8 k values of an output row.
// The LDS tile holds a 128-byte row per n, its 16-byte units swizzled by (n / 8) % 8 so the
// 2-byte stores of the decode phase (8 lanes per k row, rows 8 n apart) spread over the banks.
#pragma once

#include "pp_common.h"

namespace pp {

constexpr int DQT_T = 64;     // tile edge
constexpr int DQT_NT = 256;   // threads per workgroup

__device__ __forceinline__ uint32_t dqt_off(int n, int k) {
  return (uint32_t)n * 128u + ((((uint32_t)k >> 3) ^ (((uint32_t)n >> 3) & 7u)) << 4) + (((uint32_t)k & 7u) << 1);
}

// Tiles of the (K, N) code matrix.  D::load(k, n) fetches what codes (k, n + i), i < 8, need
// from memory (a D::Raw); D::decode(raw, v) turns it into v[m][i] (fp32, final scale
// applied).  The next tile's loads are issued before this tile's LDS reads and output
// stores, so their latency hides behind the stores.  N % 8 == 0 and K % 8 == 0, outputs
// 16-byte aligned.
template <int NM, class D>
__device__ __forceinline__ void dequant_t_tiles(const D& dec, char* tile, int64_t N, int64_t K, f16* const (&out)[NM]) {
  const int t = threadIdx.x;
  const int64_t tn = (N + DQT_T - 1) / DQT_T, tiles = tn * ((K + DQT_T - 1) / DQT_T);
  const int n8 = (t & 7) * 8;
  typename D::Raw raw[2];
  auto fetch = [&](int64_t ti) {
    if (ti >= tiles) return;
    const int64_t k0 = (ti / tn) * DQT_T, n0 = (ti % tn) * DQT_T;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int kr = (t >> 3) + 32 * p;
      if (k0 + kr < K && n0 + n8 < N) raw[p] = dec.load(k0 + kr, n0 + n8);
    }
  };
  fetch(blockIdx.x);
  for (int64_t ti = blockIdx.x; ti < tiles; ti += gridDim.x) {
    const int64_t k0 = (ti / tn) * DQT_T, n0 = (ti % tn) * DQT_T;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int kr = (t >> 3) + 32 * p;
      if (k0 + kr < K && n0 + n8 < N) {
        float v[NM][8];
        dec.decode(raw[p], v);
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
          for (int i = 0; i < 8; ++i)
            *reinterpret_cast<f16*>(tile + m * (DQT_T * 128) + dqt_off(n8 + i, kr)) = (f16)v[m][i];
      }
    }
    __syncthreads();
    fetch(ti + gridDim.x);
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int rn = (t >> 3) + 32 * p, kc = (t & 7) * 8;
        if (n0 + rn < N && k0 + kc < K) {
          const u32x4 u = *reinterpret_cast<const u32x4*>(tile + m * (DQT_T * 128) + dqt_off(rn, kc));
          *reinterpret_cast<u32x4*>(out[m] + (n0 + rn) * K + k0 + kc) = u;
        }
      }
    __syncthreads();   // the next tile's decode overwrites the LDS
  }
}

}  // namespace pp
