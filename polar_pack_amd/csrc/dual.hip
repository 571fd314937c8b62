// Dual-pack fused decode GEMV/GEMM for gfx950.
//
// One 16-bit code per pair of weights: (amp_q << 10) | phase  (polar_bitpack.py:130,
// polar_kernels.py:9-11), decoded as
//   amp = amp_lut[amp_q] * scale[group],  w1 = amp cos_lut[phase],  w2 = amp sin_lut[phase]
// (polar_kernels.py:64-79, polar_bitpack.py:228-247).  Codes are either the kernel
// layout (native int16 = code - 32768) or the .dualpack file layout (big-endian uint16).
//
// Kernels:
//   dual_rows_kernel   -- batch <= 4 decode over the .dualpack stream layout ((N,K)
//                         row-major positions, groups of 32 that restart every chunk).
//                         A lane streams 8 pairs per 16-byte load; the 8 pairs share one
//                         group scale, so the scale multiplies a per-lane partial sum once
//                         per 8 pairs (x * amp_lut, then 2 fma per pair).  Plug entries
//                         replace the amplitude as exact corrections.
//   dual_kn_gemm       -- (dual_kn.hip) codes (K,N) with unit column stride, the layout
//                         quantize_polar_bitpacked returns, in blocks of up to 8 tokens.
//   dual_dequant_kernel / dual_plug_scatter_kernel / dual_ws_gemm_kernel -- generic path
//                         and parity export (any strides, both group-index modes).
#include "dequant_t.h"
#include "dual_kn.h"
#include "dual_lds.h"

#include <algorithm>

namespace pp {

constexpr int DREPL_A = 32;   // amplitude table replicas (b32 reads)
constexpr int DREPL_C = 16;   // (cos, sin) table replicas (b64 reads)
constexpr int DSEG = 512;     // codes per wave per row per step (64 lanes x 8)
constexpr int rows_threads_dual(int MT) { return MT >= 4 ? 512 : 1024; }

struct DualLds {
  float amp[64 * DREPL_A];
  float2 cs[1024 * DREPL_C];
};

__device__ __forceinline__ void dual_build_lds(DualLds& T, const DualLuts& L) {
  for (int i = threadIdx.x; i < 64 * DREPL_A; i += blockDim.x) {
    const int e = i / DREPL_A;
    T.amp[i] = e < L.amp_n ? lut_at(L.amp, L.dtype, e) : 0.f;
  }
  for (int i = threadIdx.x; i < 1024 * DREPL_C; i += blockDim.x) {
    const int e = i / DREPL_C;
    T.cs[i] = e < L.phase_n ? make_float2(lut_at(L.cs[0], L.dtype, e), lut_at(L.cs[1], L.dtype, e))
                            : make_float2(0.f, 0.f);
  }
}

// 16-bit word as stored -> code (amp << 10 | phase)
template <int LAYOUT>
__device__ __forceinline__ uint32_t dual_code(uint32_t half16) {
  if constexpr (LAYOUT == PP_DUAL_U16_BE) return ((half16 & 0xFFu) << 8) | (half16 >> 8);
  else return half16 ^ 0x8000u;
}

struct DualGroup {
  int64_t gs, chunk;  // chunk == 0: logical (k*N + n) // gs of a (K,N) matrix
  int64_t per_chunk;  // ceil(chunk / gs)
  int log2gs;         // fast path: gs is a power of two
  __device__ __forceinline__ int64_t of_pos(int64_t p) const {
    const int64_t c = p / chunk;
    return c * per_chunk + (p - c * chunk) / gs;
  }
};

struct DualRowsArgs {
  const void* codes;   // code of (row 0, k 0)
  int64_t ldc;         // row stride (elements)
  int64_t pos0;        // stream position of (row 0, 0)
  const f16* x;
  int64_t x_sm;
  f16* out[2];
  int64_t o_sm, o_sn;
  int N, K, M;
  int n_slices, slice_len;
  int64_t n_tasks;
  const f16* scales;
  DualGroup grp;
  DualLuts luts;
  const uint32_t* plug_idx;
  const f16* plug_amp;
  const int64_t* rg_plug;
  float* part;
  int64_t part_stride;
  uint32_t* counters;
};

template <int LAYOUT>
__device__ __forceinline__ void dual_decode_one(const DualLds& T, uint32_t code, int ra, int rc, float& amp_n,
                                                float2& cs) {
  amp_n = T.amp[((code >> 10) & 63u) * DREPL_A + ra];
  cs = T.cs[(code & 1023u) * DREPL_C + rc];
}

template <int MT, int RG, int LAYOUT>
__global__ __launch_bounds__(rows_threads_dual(MT)) void dual_rows_kernel(const DualRowsArgs A) {
  __shared__ DualLds T;
  dual_build_lds(T, A.luts);
  __syncthreads();
  constexpr int WAVES = rows_threads_dual(MT) / 64;
  constexpr int NV = RG * 2 * MT;
  const int lane = threadIdx.x & 63;
  const int ra = lane % DREPL_A, rc = lane % DREPL_C;
  const int64_t gw = (int64_t)blockIdx.x * WAVES + (threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * WAVES;
  const int64_t t_begin = gw * A.n_tasks / nw, t_end = (gw + 1) * A.n_tasks / nw;
  const uint16_t* codes16 = reinterpret_cast<const uint16_t*>(A.codes);
  for (int64_t ti = t_begin; ti < t_end; ++ti) {
    const int rg = (int)(ti / A.n_slices), slice = (int)(ti % A.n_slices);
    const int row0 = rg * RG;
    const int nrows = min(RG, A.N - row0);
    const int k0 = slice * A.slice_len, k1 = min(A.K, k0 + A.slice_len);
    const int len = k1 - k0;
    const int64_t pos_row0 = A.pos0 + (int64_t)row0 * A.ldc;
    float acc[RG][2][MT];
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
      for (int j = 0; j < MT; ++j) acc[r][0][j] = acc[r][1][j] = 0.f;
    const uint16_t* cb = codes16 + (int64_t)row0 * A.ldc + k0 + 8 * lane;
    const f16* xb = A.x + k0 + 8 * lane;
    // group of each row's first pair for this lane: (chunk index, offset in chunk), advanced
    // by DSEG per step; 8 consecutive pairs never straddle a group (8 | gs, 8 | chunk, 8 | pos)
    int64_t gc[RG], grem[RG];
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const int64_t p = pos_row0 + (int64_t)r * A.ldc + k0 + 8 * lane;
      gc[r] = p / A.grp.chunk;
      grem[r] = p - gc[r] * A.grp.chunk;
    }
    for (int kb = 0; kb < len; kb += DSEG) {
      const bool valid = kb + 8 * lane < len;
      u32x4 q[RG];
      float sc[RG];
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        if (r < nrows && valid) {
          q[r] = load_nt(reinterpret_cast<const uint32_t*>(cb + (int64_t)r * A.ldc + kb));
          sc[r] = (float)A.scales[gc[r] * A.grp.per_chunk + (grem[r] >> A.grp.log2gs)];
        } else {
          q[r] = u32x4{0u, 0u, 0u, 0u};
          sc[r] = 0.f;
        }
        grem[r] += DSEG;
        while (grem[r] >= A.grp.chunk) {
          grem[r] -= A.grp.chunk;
          ++gc[r];
        }
      }
      float xv[MT][8];
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        if (valid && j < A.M) {
          const f16x4 h0 = *reinterpret_cast<const f16x4*>(xb + (int64_t)j * A.x_sm + kb);
          const f16x4 h1 = *reinterpret_cast<const f16x4*>(xb + (int64_t)j * A.x_sm + kb + 4);
          xv[j][0] = (float)h0.x; xv[j][1] = (float)h0.y; xv[j][2] = (float)h0.z; xv[j][3] = (float)h0.w;
          xv[j][4] = (float)h1.x; xv[j][5] = (float)h1.y; xv[j][6] = (float)h1.z; xv[j][7] = (float)h1.w;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) xv[j][e] = 0.f;
        }
      }
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        const uint32_t d4[4] = {q[r].x, q[r].y, q[r].z, q[r].w};
        float l1[MT], l2[MT];
#pragma unroll
        for (int j = 0; j < MT; ++j) l1[j] = l2[j] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t code = dual_code<LAYOUT>((d4[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu);
          float an;
          float2 cs;
          dual_decode_one<LAYOUT>(T, code, ra, rc, an, cs);
#pragma unroll
          for (int j = 0; j < MT; ++j) {
            const float xa = an * xv[j][e];
            l1[j] = fmaf(xa, cs.x, l1[j]);
            l2[j] = fmaf(xa, cs.y, l2[j]);
          }
        }
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          acc[r][0][j] = fmaf(sc[r], l1[j], acc[r][0][j]);
          acc[r][1][j] = fmaf(sc[r], l2[j], acc[r][1][j]);
        }
      }
    }
    // plug: amplitude replaced by plug_amp at its position
    if (A.rg_plug != nullptr) {
      const int64_t plo = A.rg_plug[rg], phi = A.rg_plug[rg + 1];
      for (int64_t p0 = plo; p0 < phi; p0 += 64) {
        const int64_t p = p0 + lane;
        if (p >= phi) continue;
        const int64_t off = (int64_t)A.plug_idx[p] - pos_row0;
        if (off < 0) continue;
        const int64_t row = off / A.ldc;
        const int k = (int)(off - row * A.ldc);
        if (row >= nrows || k < k0 || k >= k1) continue;
        const uint32_t code = dual_code<LAYOUT>(codes16[(int64_t)(row0 + row) * A.ldc + k]);
        float an;
        float2 cs;
        dual_decode_one<LAYOUT>(T, code, ra, rc, an, cs);
        const float sc = (float)A.scales[A.grp.of_pos(pos_row0 + row * A.ldc + k)];
        const float d = (float)A.plug_amp[p] - an * sc;
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          if (j >= A.M) break;
          const float xk = (float)A.x[(int64_t)j * A.x_sm + k];
#pragma unroll
          for (int r = 0; r < RG; ++r) {
            if (r == row) {
              acc[r][0][j] = fmaf(xk * d, cs.x, acc[r][0][j]);
              acc[r][1][j] = fmaf(xk * d, cs.y, acc[r][1][j]);
            }
          }
        }
      }
    }
    float mine[2] = {0.f, 0.f};
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          const float v = wave_sum(acc[r][m][j]);
          if (lane == r * MT + j) mine[m] = v;
        }
    // lane r*MT + j owns (row r, token j) of both models
    const int r = lane / MT, j = lane % MT;
    const bool owner = lane < RG * MT && r < nrows && j < A.M;
    const int64_t off = (int64_t)j * A.o_sm + (int64_t)(row0 + r) * A.o_sn;
    if (A.n_slices <= 1) {
      if (owner) {
        A.out[0][off] = (f16)mine[0];
        A.out[1][off] = (f16)mine[1];
      }
      continue;
    }
    float* grp = A.part + (int64_t)rg * A.part_stride;
    if (lane < RG * MT) {
      grp[(int64_t)slice * NV + 2 * lane] = mine[0];
      grp[(int64_t)slice * NV + 2 * lane + 1] = mine[1];
    }
    __threadfence();
    uint32_t prev = 0;
    if (lane == 0) prev = atomicAdd(A.counters + rg, 1u);
    prev = __shfl(prev, 0, 64);
    if (prev != (uint32_t)(A.n_slices - 1)) continue;
    __threadfence();
    if (lane < RG * MT) {
      float s0 = 0.f, s1 = 0.f;
      for (int s = 0; s < A.n_slices; ++s) {
        s0 += __builtin_nontemporal_load(grp + (int64_t)s * NV + 2 * lane);
        s1 += __builtin_nontemporal_load(grp + (int64_t)s * NV + 2 * lane + 1);
      }
      if (owner) {
        A.out[0][off] = (f16)s0;
        A.out[1][off] = (f16)s1;
      }
    }
    if (lane == 0) A.counters[rg] = 0u;
  }
}

// ------------------------------------------------------------------------------------------
// generic path
struct DualDequantArgs {
  const void* codes;
  int layout;
  int64_t c_sk, c_sn, elem_base;
  const f16* scales;
  DualGroup grp;
  DualLuts luts;
  void* out[2];   // O[K*N] each
  int64_t N, K;
};

// Small decode tables for the element-wise kernel: a wave's random reads conflict in a
// few banks, which costs less than the three global gathers per element they replace.
struct DualDqLds {
  float amp[64];
  float2 cs[1024];
};

template <typename O>
__device__ __forceinline__ void dual_dequant_at(const DualDqLds& T, const DualDequantArgs& A, int64_t e, int64_t k,
                                                int64_t n, int64_t g) {
  const int64_t off = k * A.c_sk + n * A.c_sn;
  const uint32_t raw = reinterpret_cast<const uint16_t*>(A.codes)[off];
  const uint32_t code = A.layout == PP_DUAL_U16_BE ? (((raw & 0xFFu) << 8) | (raw >> 8)) : (raw ^ 0x8000u);
  if (g < 0) g = A.grp.of_pos(A.elem_base + off);
  const float amp = T.amp[(code >> 10) & 63u] * (float)A.scales[g];
  const float2 cs = T.cs[code & 1023u];
  reinterpret_cast<O*>(A.out[0])[e] = (O)(amp * cs.x);
  reinterpret_cast<O*>(A.out[1])[e] = (O)(amp * cs.y);
}

template <typename O>
__global__ __launch_bounds__(256) void dual_dequant_kernel(const DualDequantArgs A) {
  __shared__ DualDqLds T;
  const DualLuts& L = A.luts;
  for (int i = threadIdx.x; i < 1024; i += blockDim.x) {
    T.cs[i] = i < L.phase_n ? make_float2(lut_at(L.cs[0], L.dtype, i), lut_at(L.cs[1], L.dtype, i))
                            : make_float2(0.f, 0.f);
    if (i < 64) T.amp[i] = i < L.amp_n ? lut_at(L.amp, L.dtype, i) : 0.f;
  }
  __syncthreads();
  const int64_t total = A.N * A.K;
  if (total < (1ll << 32) && A.grp.chunk == 0 && (A.grp.gs & (A.grp.gs - 1)) == 0) {
    // 32-bit index arithmetic (a 64-bit division per element costs more than the decode)
    const uint32_t N = (uint32_t)A.N, tot = (uint32_t)total;
    for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < tot; e += gridDim.x * blockDim.x)
      dual_dequant_at<O>(T, A, e, e / N, e % N, e >> A.grp.log2gs);
  } else {
    // e = k*N + n: the kernel rule's group is e / gs; g < 0 asks for the chunked rule
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x)
      dual_dequant_at<O>(T, A, e, e / A.N, e % A.N, A.grp.chunk == 0 ? e / A.grp.gs : -1);
  }
}

// Rows contiguous across columns (c_sn == 1, N % 8 == 0, 16-byte aligned rows) and the
// kernel's group rule with gs a power of two >= 8: a thread decodes 8 consecutive
// columns of one row (one 16-byte code load, one group scale, two stores of 8 values).
template <typename O>
__global__ __launch_bounds__(256) void dual_dequant_vec_kernel(const DualDequantArgs A) {
  __shared__ DualDqLds T;
  const DualLuts& L = A.luts;
  for (int i = threadIdx.x; i < 1024; i += blockDim.x) {
    T.cs[i] = i < L.phase_n ? make_float2(lut_at(L.cs[0], L.dtype, i), lut_at(L.cs[1], L.dtype, i))
                            : make_float2(0.f, 0.f);
    if (i < 64) T.amp[i] = i < L.amp_n ? lut_at(L.amp, L.dtype, i) : 0.f;
  }
  __syncthreads();
  const uint32_t N8 = (uint32_t)(A.N / 8), tot8 = (uint32_t)(A.N * A.K / 8);
  for (uint32_t v = blockIdx.x * blockDim.x + threadIdx.x; v < tot8; v += gridDim.x * blockDim.x) {
    const uint32_t k = v / N8, n = 8u * (v - k * N8), e = 8u * v;
    const u32x4 q = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(A.codes) +
                                                    (int64_t)k * A.c_sk + n);
    const float sc = (float)A.scales[e >> A.grp.log2gs];
    const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
    float o1[8], o2[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t raw = (w4[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
      const uint32_t code = A.layout == PP_DUAL_U16_BE ? (((raw & 0xFFu) << 8) | (raw >> 8)) : (raw ^ 0x8000u);
      const float amp = T.amp[(code >> 10) & 63u] * sc;
      const float2 cs = T.cs[code & 1023u];
      o1[i] = amp * cs.x;
      o2[i] = amp * cs.y;
    }
    if constexpr (sizeof(O) == 2) {
      // 8 fp16 values as one 16-byte store per output
      u32x4 h1, h2;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t a = __builtin_bit_cast(unsigned short, (f16)o1[2 * i]);
        const uint32_t b = __builtin_bit_cast(unsigned short, (f16)o1[2 * i + 1]);
        const uint32_t c = __builtin_bit_cast(unsigned short, (f16)o2[2 * i]);
        const uint32_t d = __builtin_bit_cast(unsigned short, (f16)o2[2 * i + 1]);
        h1[i] = a | (b << 16);
        h2[i] = c | (d << 16);
      }
      *reinterpret_cast<u32x4*>(reinterpret_cast<O*>(A.out[0]) + e) = h1;
      *reinterpret_cast<u32x4*>(reinterpret_cast<O*>(A.out[1]) + e) = h2;
    } else {
      float4* d1 = reinterpret_cast<float4*>(reinterpret_cast<O*>(A.out[0]) + e);
      float4* d2 = reinterpret_cast<float4*>(reinterpret_cast<O*>(A.out[1]) + e);
      d1[0] = make_float4(o1[0], o1[1], o1[2], o1[3]);
      d1[1] = make_float4(o1[4], o1[5], o1[6], o1[7]);
      d2[0] = make_float4(o2[0], o2[1], o2[2], o2[3]);
      d2[1] = make_float4(o2[4], o2[5], o2[6], o2[7]);
    }
  }
}

struct DualPlugScatterArgs {
  const void* codes;
  int layout;
  int64_t c_sk, c_sn, elem_base;
  const uint32_t* plug_idx;
  const f16* plug_amp;
  int64_t plug_n;
  DualLuts luts;
  void* out[2];
  int64_t N, K;
  int64_t o_k, o_n;   // output element of (k, n): k*o_k + n*o_n
};

template <typename O>
__global__ void dual_plug_scatter_kernel(const DualPlugScatterArgs A) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= A.plug_n) return;
  const int64_t off = (int64_t)A.plug_idx[j] - A.elem_base;
  if (off < 0) return;
  int64_t k, n;
  if (A.c_sk == 1) {
    n = off / A.c_sn;
    k = off - n * A.c_sn;
  } else {
    k = off / A.c_sk;
    n = off - k * A.c_sk;
  }
  if (k >= A.K || n >= A.N) return;
  const uint32_t raw = reinterpret_cast<const uint16_t*>(A.codes)[off];
  const uint32_t code = A.layout == PP_DUAL_U16_BE ? (((raw & 0xFFu) << 8) | (raw >> 8)) : (raw ^ 0x8000u);
  const int ph = (int)(code & 1023u);
  const float amp = (float)A.plug_amp[j];
  const float c = ph < A.luts.phase_n ? lut_at(A.luts.cs[0], A.luts.dtype, ph) : 0.f;
  const float s = ph < A.luts.phase_n ? lut_at(A.luts.cs[1], A.luts.dtype, ph) : 0.f;
  reinterpret_cast<O*>(A.out[0])[k * A.o_k + n * A.o_n] = (O)(amp * c);
  reinterpret_cast<O*>(A.out[1])[k * A.o_k + n * A.o_n] = (O)(amp * s);
}

// Transposed decode (dequant_t.h): int16 / big-endian codes (K,N), row stride c_sk (unit
// column stride), the kernel group rule (k*N + n) / gs with gs a power of two >= 8 ->
// out_m (N,K) row-major fp16.  8 codes of a row share one group scale.
struct DualDequantTArgs {
  const void* codes;
  int layout;
  int64_t c_sk;
  const f16* scales;
  int log2gs;
  DualLuts luts;
  f16* out[2];
  int64_t N, K;
};

struct DualDecT {
  const DualDqLds& T;
  const DualDequantTArgs& A;
  struct Raw {
    u32x4 q;
    float sc;
  };
  __device__ __forceinline__ Raw load(int64_t k, int64_t n) const {
    return Raw{*reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(A.codes) + k * A.c_sk + n),
               (float)A.scales[(k * A.N + n) >> A.log2gs]};
  }
  __device__ __forceinline__ void decode(const Raw& r, float (&v)[2][8]) const {
    const uint32_t w4[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t raw = (w4[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
      const uint32_t code = A.layout == PP_DUAL_U16_BE ? (((raw & 0xFFu) << 8) | (raw >> 8)) : (raw ^ 0x8000u);
      const float amp = T.amp[(code >> 10) & 63u] * r.sc;
      const float2 cs = T.cs[code & 1023u];
      v[0][i] = amp * cs.x;
      v[1][i] = amp * cs.y;
    }
  }
};

__global__ __launch_bounds__(DQT_NT) void dual_dequant_t_kernel(const DualDequantTArgs A) {
  __shared__ DualDqLds T;
  __shared__ __attribute__((aligned(16))) char tile[2 * DQT_T * 128];
  const DualLuts& L = A.luts;
  for (int i = threadIdx.x; i < 1024; i += blockDim.x) {
    T.cs[i] = i < L.phase_n ? make_float2(lut_at(L.cs[0], L.dtype, i), lut_at(L.cs[1], L.dtype, i))
                            : make_float2(0.f, 0.f);
    if (i < 64) T.amp[i] = i < L.amp_n ? lut_at(L.amp, L.dtype, i) : 0.f;
  }
  __syncthreads();
  f16* const out[2] = {A.out[0], A.out[1]};
  dequant_t_tiles<2>(DualDecT{T, A}, tile, A.N, A.K, out);
}

struct DualWsGemmArgs {
  const f16* a;
  int64_t a_sm, a_sk;
  const float* w[2];
  f16* out[2];
  int64_t o_sm, o_sn;
  int64_t M, N, K;
};

__global__ __launch_bounds__(256) void dual_ws_gemm_kernel(const DualWsGemmArgs A) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t i = blockIdx.y;
  if (n >= A.N) return;
  float a0 = 0.f, a1 = 0.f;
  const f16* ar = A.a + i * A.a_sm;
  for (int64_t k = 0; k < A.K; ++k) {
    const float av = (float)ar[k * A.a_sk];
    a0 = fmaf(av, A.w[0][k * A.N + n], a0);
    a1 = fmaf(av, A.w[1][k * A.N + n], a1);
  }
  A.out[0][i * A.o_sm + n * A.o_sn] = (f16)a0;
  A.out[1][i * A.o_sm + n * A.o_sn] = (f16)a1;
}

__global__ void dual_zero_u32_kernel(uint32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

__global__ void dual_rowgroup_plug_kernel(const uint32_t* plug_idx, int64_t plug_n, int64_t pos0, int64_t ldc,
                                          int rows_per_group, int n_rowgroups, int N, int64_t* rg_plug) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;
  if (g > n_rowgroups) return;
  const int64_t row = min<int64_t>((int64_t)g * rows_per_group, N);
  const int64_t key = pos0 + row * ldc;
  int64_t lo = 0, hi = plug_n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)plug_idx[mid] < key) lo = mid + 1;
    else hi = mid;
  }
  rg_plug[g] = lo;
}

// ------------------------------------------------------------------------------------------
// host side
static int dual_round_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : 4; }
static int dual_rows_rg(int mt) { return mt == 1 ? 4 : (mt == 2 ? 2 : 1); }

static bool dual_fast_ok(const void* a, int64_t a_sm, int64_t a_sk, const void* codes, int64_t c_sk, int64_t c_sn,
                         int64_t elem_base, int64_t chunk, int64_t gs, int64_t M, int64_t K) {
  return c_sk == 1 && c_sn % 8 == 0 && c_sn >= K && K % 8 == 0 && K > 0 && aligned(codes, 16) && M >= 1 &&
         M <= 4 && chunk > 0 && chunk % 8 == 0 && gs >= 8 && (gs & (gs - 1)) == 0 && elem_base % 8 == 0 &&
         (a_sk == 1 || K == 1) && (M == 1 || a_sm % 4 == 0) && aligned(a, 8);
}

struct DualPlan {
  int rg, n_rowgroups, n_slices, slice_len;
  int64_t n_tasks, part_bytes, counter_bytes, plug_bytes;
  int64_t total() const { return part_bytes + counter_bytes + plug_bytes; }
};

static DualPlan dual_plan(int64_t M, int64_t N, int64_t K, int64_t plug_n) {
  DualPlan p;
  const int mt = dual_round_mt(M);
  p.rg = dual_rows_rg(mt);
  p.n_rowgroups = (int)((N + p.rg - 1) / p.rg);
  const int64_t waves = (int64_t)device_cu_count() * (rows_threads_dual(mt) / 64);
  const int64_t segs = (K + DSEG - 1) / DSEG;
  int64_t want = (4 * waves + p.n_rowgroups - 1) / p.n_rowgroups;
  want = std::max<int64_t>(1, std::min<int64_t>(want, std::max<int64_t>(1, K / 4096)));
  const int64_t sps = (segs + want - 1) / want;
  p.slice_len = (int)(sps * DSEG);
  p.n_slices = (int)((K + p.slice_len - 1) / p.slice_len);
  p.n_tasks = (int64_t)p.n_rowgroups * p.n_slices;
  const int nv = p.rg * 2 * mt;
  p.part_bytes = p.n_slices > 1 ? ((int64_t)p.n_rowgroups * p.n_slices * nv * 4 + 255) / 256 * 256 : 0;
  p.counter_bytes = p.n_slices > 1 ? ((int64_t)p.n_rowgroups * 4 + 255) / 256 * 256 : 0;
  p.plug_bytes = plug_n > 0 ? ((int64_t)(p.n_rowgroups + 1) * 8 + 255) / 256 * 256 : 0;
  return p;
}

template <int MT, int RG, int LAYOUT>
static int launch_dual_rows(const DualRowsArgs& A, hipStream_t st) {
  hipLaunchKernelGGL((dual_rows_kernel<MT, RG, LAYOUT>), dim3(device_cu_count()), dim3(rows_threads_dual(MT)), 0,
                     st, A);
  PP_LAUNCH_CHECK();
  return PP_OK;
}

template <int LAYOUT>
static int dispatch_dual_rows(const DualRowsArgs& A, int mt, hipStream_t st) {
  switch (mt) {
    case 1: return launch_dual_rows<1, 4, LAYOUT>(A, st);
    case 2: return launch_dual_rows<2, 2, LAYOUT>(A, st);
    default: return launch_dual_rows<4, 1, LAYOUT>(A, st);
  }
}

static DualLuts make_dual_luts(const void* amp, int amp_n, const void* c, const void* s, int phase_n, int dtype) {
  DualLuts L;
  L.amp = amp;
  L.cs[0] = c;
  L.cs[1] = s;
  L.amp_n = amp_n;
  L.phase_n = phase_n;
  L.dtype = dtype;
  return L;
}

}  // namespace pp

using namespace pp;

static int dual_common_checks(const void* codes, int code_layout, int64_t group_size, int64_t chunk_size,
                              const void* amp_lut, int amp_lut_n, const void* cos_lut, const void* sin_lut,
                              int phase_n, int lut_dtype, int64_t plug_n, const uint32_t* plug_idx,
                              const void* plug_amp, int64_t c_sk, int64_t c_sn, int64_t N, int64_t K) {
  PP_REQUIRE(code_layout == PP_DUAL_I16_OFFSET || code_layout == PP_DUAL_U16_BE, "bad code_layout");
  PP_REQUIRE(lut_dtype == PP_F16 || lut_dtype == PP_F32, "bad lut_dtype");
  PP_REQUIRE(amp_lut && cos_lut && sin_lut, "lut pointers are null");
  PP_REQUIRE(amp_lut_n >= 1 && amp_lut_n <= 64, "amp_lut_n must be 1..64 (6 amplitude bits)");
  PP_REQUIRE(phase_n >= 1 && phase_n <= 1024, "phase_n must be 1..1024 (10 phase bits)");
  PP_REQUIRE(group_size >= 1 && chunk_size >= 0, "bad group_size / chunk_size");
  PP_REQUIRE(plug_n >= 0 && (plug_n == 0 || (plug_idx && plug_amp)), "plug arrays are null");
  PP_REQUIRE(plug_n == 0 || (c_sk == 1 && c_sn >= K) || (c_sn == 1 && c_sk >= N),
             "plug entries need a unit-stride (K,N) view");
  PP_REQUIRE(codes != nullptr || N * K == 0, "codes is null");
  return PP_OK;
}

extern "C" int64_t pp_dual_gemm_workspace_size(const void* a, int64_t a_sm, int64_t a_sk, const void* codes,
                                               int64_t c_sk, int64_t c_sn, int64_t group_size, int64_t chunk_size,
                                               int64_t elem_base, int64_t plug_n, int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0) return 0;
  if (dual_fast_ok(a, a_sm, a_sk, codes, c_sk, c_sn, elem_base, chunk_size, group_size, M, K))
    return dual_plan(M, N, K, plug_n).total();
  // (K,N) codes: blocks of up to 8 tokens, one after another, sharing the workspace (the
  // last block may have 1..7 tokens: the larger of the 4- and 8-token needs covers it)
  if (dual_kn_ok(a, a_sm, a_sk, codes, c_sk, c_sn, group_size, chunk_size, std::min<int64_t>(M, 8), N, K))
    return std::max(dual_kn_workspace(std::min<int64_t>(M, 8), N, K, plug_n),
                    dual_kn_workspace(std::min<int64_t>(M, 4), N, K, plug_n));
  return 2 * N * K * (int64_t)sizeof(float);
}

template <typename O>
static int dual_dequant_to(const void* codes, int code_layout, int64_t c_sk, int64_t c_sn, const void* bmax,
                               int64_t group_size, int64_t chunk_size, const void* amp_lut, int amp_lut_n,
                               const void* cos_lut, const void* sin_lut, int phase_n, int lut_dtype,
                               const uint32_t* plug_idx, const void* plug_amp, int64_t plug_n, int64_t elem_base,
                               void* out1, void* out2, int64_t N, int64_t K, void* stream) {
  if (int rc = dual_common_checks(codes, code_layout, group_size, chunk_size, amp_lut, amp_lut_n, cos_lut, sin_lut,
                                  phase_n, lut_dtype, plug_n, plug_idx, plug_amp, c_sk, c_sn, N, K))
    return rc;
  PP_REQUIRE(out1 && out2 && bmax, "out / bmax pointers are null");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (N * K == 0) return PP_OK;
  DualDequantArgs A;
  A.codes = codes;
  A.layout = code_layout;
  A.c_sk = c_sk;
  A.c_sn = c_sn;
  A.elem_base = elem_base;
  A.scales = reinterpret_cast<const f16*>(bmax);
  A.grp.gs = group_size;
  A.grp.chunk = chunk_size;
  A.grp.per_chunk = chunk_size > 0 ? (chunk_size + group_size - 1) / group_size : 0;
  A.grp.log2gs = 0;
  while ((1ll << A.grp.log2gs) < group_size) ++A.grp.log2gs;
  A.luts = make_dual_luts(amp_lut, amp_lut_n, cos_lut, sin_lut, phase_n, lut_dtype);
  A.out[0] = out1;
  A.out[1] = out2;
  A.N = N;
  A.K = K;
  const bool vec = c_sn == 1 && c_sk % 8 == 0 && N % 8 == 0 && aligned(codes, 16) && chunk_size == 0 &&
                   group_size >= 8 && (group_size & (group_size - 1)) == 0 && N * K < (1ll << 32) &&
                   aligned(out1, 16) && aligned(out2, 16);
  if (vec) {
    const int64_t blocks = std::min<int64_t>((N * K / 8 + 255) / 256, (int64_t)device_cu_count() * 8);
    hipLaunchKernelGGL(dual_dequant_vec_kernel<O>, dim3((unsigned)blocks), dim3(256), 0, st, A);
  } else {
    const int64_t blocks = std::min<int64_t>((N * K + 255) / 256, (int64_t)device_cu_count() * 16);
    hipLaunchKernelGGL(dual_dequant_kernel<O>, dim3((unsigned)blocks), dim3(256), 0, st, A);
  }
  PP_LAUNCH_CHECK();
  if (plug_n > 0) {
    DualPlugScatterArgs P;
    P.codes = codes;
    P.layout = code_layout;
    P.c_sk = c_sk;
    P.c_sn = c_sn;
    P.elem_base = elem_base;
    P.plug_idx = plug_idx;
    P.plug_amp = reinterpret_cast<const f16*>(plug_amp);
    P.plug_n = plug_n;
    P.luts = A.luts;
    P.out[0] = out1;
    P.out[1] = out2;
    P.N = N;
    P.K = K;
    P.o_k = N;
    P.o_n = 1;
    hipLaunchKernelGGL(dual_plug_scatter_kernel<O>, dim3((unsigned)((plug_n + 255) / 256)), dim3(256), 0, st, P);
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
}

extern "C" int pp_dual_dequant(const void* codes, int code_layout, int64_t c_sk, int64_t c_sn, const void* bmax,
                               int64_t group_size, int64_t chunk_size, const void* amp_lut, int amp_lut_n,
                               const void* cos_lut, const void* sin_lut, int phase_n, int lut_dtype,
                               const uint32_t* plug_idx, const void* plug_amp, int64_t plug_n, int64_t elem_base,
                               float* out1, float* out2, int64_t N, int64_t K, void* stream) {
  return dual_dequant_to<float>(codes, code_layout, c_sk, c_sn, bmax, group_size, chunk_size, amp_lut, amp_lut_n,
                                cos_lut, sin_lut, phase_n, lut_dtype, plug_idx, plug_amp, plug_n, elem_base, out1,
                                out2, N, K, stream);
}

extern "C" int pp_dual_dequant_f16(const void* codes, int code_layout, int64_t c_sk, int64_t c_sn,
                                   const void* bmax, int64_t group_size, int64_t chunk_size, const void* amp_lut,
                                   int amp_lut_n, const void* cos_lut, const void* sin_lut, int phase_n,
                                   int lut_dtype, const uint32_t* plug_idx, const void* plug_amp, int64_t plug_n,
                                   int64_t elem_base, void* out1, void* out2, int64_t N, int64_t K, void* stream) {
  return dual_dequant_to<f16>(codes, code_layout, c_sk, c_sn, bmax, group_size, chunk_size, amp_lut, amp_lut_n,
                              cos_lut, sin_lut, phase_n, lut_dtype, plug_idx, plug_amp, plug_n, elem_base, out1,
                              out2, N, K, stream);
}

extern "C" int pp_dual_dequant_f16_t(const void* codes, int code_layout, int64_t c_sk, const void* bmax,
                                     int64_t group_size, const void* amp_lut, int amp_lut_n, const void* cos_lut,
                                     const void* sin_lut, int phase_n, int lut_dtype, const uint32_t* plug_idx,
                                     const void* plug_amp, int64_t plug_n, int64_t elem_base, void* out1,
                                     void* out2, int64_t N, int64_t K, void* stream) {
  if (int rc = dual_common_checks(codes, code_layout, group_size, 0, amp_lut, amp_lut_n, cos_lut, sin_lut, phase_n,
                                  lut_dtype, plug_n, plug_idx, plug_amp, c_sk, 1, N, K))
    return rc;
  PP_REQUIRE(out1 && out2 && bmax, "out / bmax pointers are null");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (N * K == 0) return PP_OK;
  PP_REQUIRE(N % 8 == 0 && K % 8 == 0 && c_sk >= N && c_sk % 8 == 0 && aligned(codes, 16),
             "the transposed decode needs N % 8 == 0, K % 8 == 0 and 16-byte aligned code rows "
             "(row stride >= N, a multiple of 8)");
  PP_REQUIRE(group_size >= 8 && (group_size & (group_size - 1)) == 0,
             "the transposed decode needs a power-of-two group_size >= 8");
  PP_REQUIRE(aligned(out1, 16) && aligned(out2, 16), "outputs must be 16-byte aligned");
  DualDequantTArgs A;
  A.codes = codes;
  A.layout = code_layout;
  A.c_sk = c_sk;
  A.scales = reinterpret_cast<const f16*>(bmax);
  A.log2gs = 0;
  while ((1ll << A.log2gs) < group_size) ++A.log2gs;
  A.luts = make_dual_luts(amp_lut, amp_lut_n, cos_lut, sin_lut, phase_n, lut_dtype);
  A.out[0] = reinterpret_cast<f16*>(out1);
  A.out[1] = reinterpret_cast<f16*>(out2);
  A.N = N;
  A.K = K;
  const int64_t tiles = ((N + DQT_T - 1) / DQT_T) * ((K + DQT_T - 1) / DQT_T);
  // 24.3 KiB of LDS a workgroup: six fit a CU (with the next-tile loads, 21.0 against 22.7 us
  // for a 4096 x 4096 pair with four and no prefetch)
  const int64_t blocks = std::min<int64_t>(tiles, (int64_t)device_cu_count() * 6);
  hipLaunchKernelGGL(dual_dequant_t_kernel, dim3((unsigned)blocks), dim3(DQT_NT), 0, st, A);
  PP_LAUNCH_CHECK();
  if (plug_n > 0) {
    DualPlugScatterArgs P;
    P.codes = codes;
    P.layout = code_layout;
    P.c_sk = c_sk;
    P.c_sn = 1;
    P.elem_base = elem_base;
    P.plug_idx = plug_idx;
    P.plug_amp = reinterpret_cast<const f16*>(plug_amp);
    P.plug_n = plug_n;
    P.luts = A.luts;
    P.out[0] = out1;
    P.out[1] = out2;
    P.N = N;
    P.K = K;
    P.o_k = 1;
    P.o_n = K;
    hipLaunchKernelGGL(dual_plug_scatter_kernel<f16>, dim3((unsigned)((plug_n + 255) / 256)), dim3(256), 0, st, P);
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
}

extern "C" int pp_dual_gemm_kernel(const void* a, int64_t a_sm, int64_t a_sk, const void* codes, int64_t c_sk,
                                   int64_t c_sn, int64_t group_size, int64_t chunk_size, int64_t elem_base,
                                   int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  if (dual_fast_ok(a, a_sm, a_sk, codes, c_sk, c_sn, elem_base, chunk_size, group_size, M, K)) return PP_GEMM_ROWS;
  if (dual_kn_ok(a, a_sm, a_sk, codes, c_sk, c_sn, group_size, chunk_size, std::min<int64_t>(M, 8), N, K))
    return PP_GEMM_KN;
  return PP_GEMM_GENERIC;
}

extern "C" int pp_dual_gemm(const void* a, int64_t a_sm, int64_t a_sk, const void* codes, int code_layout,
                            int64_t c_sk, int64_t c_sn, const void* bmax, int64_t group_size, int64_t chunk_size,
                            const void* amp_lut, int amp_lut_n, const void* cos_lut, const void* sin_lut,
                            int phase_n, int lut_dtype, const uint32_t* plug_idx, const void* plug_amp,
                            int64_t plug_n, int64_t elem_base, void* out1, void* out2, int64_t o_sm, int64_t o_sn,
                            int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                            void* stream) {
  if (int rc = dual_common_checks(codes, code_layout, group_size, chunk_size, amp_lut, amp_lut_n, cos_lut, sin_lut,
                                  phase_n, lut_dtype, plug_n, plug_idx, plug_amp, c_sk, c_sn, N, K))
    return rc;
  PP_REQUIRE(M >= 0 && N >= 0 && K >= 0, "negative shape");
  PP_REQUIRE(out1 && out2 && bmax, "out / bmax pointers are null");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (M == 0 || N == 0) return PP_OK;
  PP_REQUIRE(a != nullptr, "a is null");
  PP_REQUIRE(N < (1ll << 31) && K < (1ll << 31), "N and K must be < 2^31");
  const DualLuts L = make_dual_luts(amp_lut, amp_lut_n, cos_lut, sin_lut, phase_n, lut_dtype);
  if (dual_fast_ok(a, a_sm, a_sk, codes, c_sk, c_sn, elem_base, chunk_size, group_size, M, K)) {
    const DualPlan p = dual_plan(M, N, K, plug_n);
    PP_REQUIRE(workspace_bytes >= p.total() && (p.total() == 0 || workspace != nullptr),
               "workspace too small: need %lld bytes", (long long)p.total());
    char* ws = reinterpret_cast<char*>(workspace);
    DualRowsArgs A = {};
    A.codes = codes;
    A.ldc = c_sn;
    A.pos0 = elem_base;
    A.x = reinterpret_cast<const f16*>(a);
    A.x_sm = a_sm;
    A.out[0] = reinterpret_cast<f16*>(out1);
    A.out[1] = reinterpret_cast<f16*>(out2);
    A.o_sm = o_sm;
    A.o_sn = o_sn;
    A.N = (int)N;
    A.K = (int)K;
    A.M = (int)M;
    A.n_slices = p.n_slices;
    A.slice_len = p.slice_len;
    A.n_tasks = p.n_tasks;
    A.scales = reinterpret_cast<const f16*>(bmax);
    A.grp.gs = group_size;
    A.grp.chunk = chunk_size;
    A.grp.per_chunk = (chunk_size + group_size - 1) / group_size;
    A.grp.log2gs = 0;
    while ((1ll << A.grp.log2gs) < group_size) ++A.grp.log2gs;
    A.luts = L;
    A.plug_idx = plug_idx;
    A.plug_amp = reinterpret_cast<const f16*>(plug_amp);
    const int mt = dual_round_mt(M);
    A.part = p.part_bytes ? reinterpret_cast<float*>(ws) : nullptr;
    A.part_stride = (int64_t)p.n_slices * p.rg * 2 * mt;
    A.counters = p.counter_bytes ? reinterpret_cast<uint32_t*>(ws + p.part_bytes) : nullptr;
    if (p.counter_bytes) {
      const int64_t nc = p.counter_bytes / 4;
      hipLaunchKernelGGL(dual_zero_u32_kernel, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, st, A.counters, nc);
      PP_LAUNCH_CHECK();
    }
    if (plug_n > 0) {
      int64_t* rgp = reinterpret_cast<int64_t*>(ws + p.part_bytes + p.counter_bytes);
      hipLaunchKernelGGL(dual_rowgroup_plug_kernel, dim3((p.n_rowgroups + 1 + 255) / 256), dim3(256), 0, st,
                         plug_idx, plug_n, elem_base, c_sn, p.rg, p.n_rowgroups, (int)N, rgp);
      PP_LAUNCH_CHECK();
      A.rg_plug = rgp;
    }
    return code_layout == PP_DUAL_U16_BE ? dispatch_dual_rows<PP_DUAL_U16_BE>(A, mt, st)
                                         : dispatch_dual_rows<PP_DUAL_I16_OFFSET>(A, mt, st);
  }
  if (dual_kn_ok(a, a_sm, a_sk, codes, c_sk, c_sn, group_size, chunk_size, std::min<int64_t>(M, 8), N, K)) {
    for (int64_t i0 = 0; i0 < M; i0 += 8) {
      void* o[2] = {reinterpret_cast<f16*>(out1) + i0 * o_sm, reinterpret_cast<f16*>(out2) + i0 * o_sm};
      if (int rc = dual_kn_gemm(reinterpret_cast<const f16*>(a) + i0 * a_sm, a_sm, codes, code_layout, c_sk, bmax,
                                group_size, L, plug_idx, plug_amp, plug_n, elem_base, o, o_sm, o_sn,
                                std::min<int64_t>(8, M - i0), N, K, workspace, workspace_bytes, st))
        return rc;
    }
    return PP_OK;
  }
  const int64_t need = 2 * N * K * (int64_t)sizeof(float);
  PP_REQUIRE(workspace != nullptr && workspace_bytes >= need, "workspace too small: need %lld bytes",
             (long long)need);
  float* w0 = reinterpret_cast<float*>(workspace);
  float* w1 = w0 + N * K;
  if (int rc = pp_dual_dequant(codes, code_layout, c_sk, c_sn, bmax, group_size, chunk_size, amp_lut, amp_lut_n,
                               cos_lut, sin_lut, phase_n, lut_dtype, plug_idx, plug_amp, plug_n, elem_base, w0, w1,
                               N, K, stream))
    return rc;
  DualWsGemmArgs G;
  G.a = reinterpret_cast<const f16*>(a);
  G.a_sm = a_sm;
  G.a_sk = a_sk;
  G.w[0] = w0;
  G.w[1] = w1;
  G.out[0] = reinterpret_cast<f16*>(out1);
  G.out[1] = reinterpret_cast<f16*>(out2);
  G.o_sm = o_sm;
  G.o_sn = o_sn;
  G.M = M;
  G.N = N;
  G.K = K;
  hipLaunchKernelGGL(dual_ws_gemm_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)M), dim3(256), 0, st, G);
  PP_LAUNCH_CHECK();
  return PP_OK;
}
