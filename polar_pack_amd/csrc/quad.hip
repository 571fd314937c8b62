// Quad-pack decode for gfx950: generic layouts, the dequantise export and the
// single-projection operator.
//
// One uint32 word per 4-tuple of weights (one weight per model):
//   [nq 8 | q1 8 | q2 8 | q3 8]  (quad_kernels.py:103-106, quaternion_packer.py:173-176)
// decoded as  r = norm[nq], w0 = r c1, w1 = r s1 c2, w2 = r s1 s2 c3, w3 = r s1 s2 s3
// (quad_kernels.py:108-121, quaternion_packer.py:178-185), times the per-model
// RMS s_m (quad_kernels.py:131-134).
//
// pp_quad_gemm runs the fused row kernel (quad_rows.hip) when the codes are (N,K) rows
// (the container layout) and M <= 8; any other strides go through
//   quad_dequant_kernel / quad_plug_scatter_kernel -- float32 weights in a workspace
//                        (also the parity export pp_quad_dequant), then
//   quad_ws_gemm_kernel -- a plain GEMM on them (correct for any strides, not a
//                        performance path).
#include "dequant_t.h"
#include "pp_common.h"
#include "quad_kn.h"
#include "quad_rows.h"

#include <algorithm>
#include <cmath>

namespace pp {

// Generic path: weights out_m[k*N + n] = s_m * W_m[k, n] (float32 for the workspace GEMM,
// fp16 for a caller's library GEMM), then a GEMM.
struct QuadDequantArgs {
  const uint32_t* codes;
  int64_t c_sk, c_sn;
  QuadLuts luts;
  float s[4];
  void* out[4];   // O[K*N] each
  int64_t N, K;
};

template <typename O>
__device__ __forceinline__ void quad_dequant_at(const QuadLds<1, 1>& T, const QuadDequantArgs& A, int64_t e,
                                                int64_t k, int64_t n) {
  float w[4];
  quad_decode(T, A.codes[k * A.c_sk + n * A.c_sn], 0, 0, w[0], w[1], w[2], w[3]);
#pragma unroll
  for (int m = 0; m < 4; ++m) reinterpret_cast<O*>(A.out[m])[e] = (O)(w[m] * A.s[m]);
}

template <typename O>
__global__ __launch_bounds__(256) void quad_dequant_kernel(const QuadDequantArgs A) {
  __shared__ QuadLds<1, 1> T;
  quad_build_lds(T, A.luts);
  __syncthreads();
  const int64_t total = A.N * A.K;
  if (total < (1ll << 32)) {
    // 32-bit index arithmetic (a 64-bit division per element costs more than the decode)
    const uint32_t N = (uint32_t)A.N, tot = (uint32_t)total;
    for (uint32_t e = blockIdx.x * blockDim.x + threadIdx.x; e < tot; e += gridDim.x * blockDim.x)
      quad_dequant_at<O>(T, A, e, e / N, e % N);
  } else {
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x)
      quad_dequant_at<O>(T, A, e, e / A.N, e % A.N);
  }
}

// Rows contiguous across columns (c_sn == 1, N % 4 == 0, 16-byte aligned rows): a
// thread decodes 4 consecutive columns of one row (one 16-byte code load, one store of 4
// values per model).
template <typename O>
__global__ __launch_bounds__(256) void quad_dequant_vec_kernel(const QuadDequantArgs A) {
  __shared__ QuadLds<1, 1> T;
  quad_build_lds(T, A.luts);
  __syncthreads();
  const uint32_t N4 = (uint32_t)(A.N / 4), tot4 = (uint32_t)(A.N * A.K / 4);
  for (uint32_t v = blockIdx.x * blockDim.x + threadIdx.x; v < tot4; v += gridDim.x * blockDim.x) {
    const uint32_t k = v / N4, n = 4u * (v - k * N4), e = 4u * v;
    const u32x4 q = *reinterpret_cast<const u32x4*>(A.codes + (int64_t)k * A.c_sk + n);
    const uint32_t cw[4] = {q.x, q.y, q.z, q.w};
    float w[4][4];   // [column][model]
#pragma unroll
    for (int c = 0; c < 4; ++c) quad_decode(T, cw[c], 0, 0, w[c][0], w[c][1], w[c][2], w[c][3]);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      O* d = reinterpret_cast<O*>(A.out[m]) + e;
      if constexpr (sizeof(O) == 2) {
        u32x2 h;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const uint32_t a = __builtin_bit_cast(unsigned short, (f16)(w[2 * i][m] * A.s[m]));
          const uint32_t b = __builtin_bit_cast(unsigned short, (f16)(w[2 * i + 1][m] * A.s[m]));
          h[i] = a | (b << 16);
        }
        *reinterpret_cast<u32x2*>(d) = h;
      } else {
        *reinterpret_cast<float4*>(d) =
            make_float4(w[0][m] * A.s[m], w[1][m] * A.s[m], w[2][m] * A.s[m], w[3][m] * A.s[m]);
      }
    }
  }
}

struct QuadPlugScatterArgs {
  const uint32_t* plug_idx;
  const f16* plug_vals;
  int64_t plug_n, elem_base;
  int64_t c_sk, c_sn;
  float s[4];
  void* out[4];
  int64_t N, K;
  int64_t o_k, o_n;   // output element of (k, n): k*o_k + n*o_n
};

// Entries are unique positions, so the scatter has no write conflicts.
template <typename O>
__global__ void quad_plug_scatter_kernel(const QuadPlugScatterArgs A) {
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
  const int64_t e = k * A.o_k + n * A.o_n;
#pragma unroll
  for (int m = 0; m < 4; ++m) reinterpret_cast<O*>(A.out[m])[e] = (O)((float)A.plug_vals[4 * j + m] * A.s[m]);
}

// Transposed decode (dequant_t.h): codes (K,N), row stride c_sk (unit column stride) ->
// out_m (N,K) row-major fp16, s_m applied.
struct QuadDequantTArgs {
  const uint32_t* codes;
  int64_t c_sk;
  QuadLuts luts;
  float s[4];
  f16* out[4];
  int64_t N, K;
};

struct QuadDecT {
  const QuadLds<1, 1>& T;
  const QuadDequantTArgs& A;
  struct Raw {
    u32x4 q0, q1;
  };
  __device__ __forceinline__ Raw load(int64_t k, int64_t n) const {
    const uint32_t* p = A.codes + k * A.c_sk + n;
    return Raw{*reinterpret_cast<const u32x4*>(p), *reinterpret_cast<const u32x4*>(p + 4)};
  }
  __device__ __forceinline__ void decode(const Raw& r, float (&v)[4][8]) const {
    const uint32_t cw[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float w[4];
      quad_decode(T, cw[i], 0, 0, w[0], w[1], w[2], w[3]);
#pragma unroll
      for (int m = 0; m < 4; ++m) v[m][i] = w[m] * A.s[m];
    }
  }
};

__global__ __launch_bounds__(DQT_NT) void quad_dequant_t_kernel(const QuadDequantTArgs A) {
  __shared__ QuadLds<1, 1> T;
  __shared__ __attribute__((aligned(16))) char tile[4 * DQT_T * 128];
  quad_build_lds(T, A.luts);
  __syncthreads();
  f16* const out[4] = {A.out[0], A.out[1], A.out[2], A.out[3]};
  dequant_t_tiles<4>(QuadDecT{T, A}, tile, A.N, A.K, out);
}

struct QuadWsGemmArgs {
  const f16* a;
  int64_t a_sm, a_sk;
  const float* w[4];  // (K, N) row-major, already scaled
  f16* out[4];
  int64_t o_sm, o_sn;
  int64_t M, N, K;
};

// out_m[i, n] = fp16(sum_k a[i,k] * w_m[k,n]); a column per thread, a row of a per block.y.
__global__ __launch_bounds__(256) void quad_ws_gemm_kernel(const QuadWsGemmArgs A) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t i = blockIdx.y;
  if (n >= A.N) return;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const f16* ar = A.a + i * A.a_sm;
  for (int64_t k = 0; k < A.K; ++k) {
    const float av = (float)ar[k * A.a_sk];
#pragma unroll
    for (int m = 0; m < 4; ++m) acc[m] = fmaf(av, A.w[m][k * A.N + n], acc[m]);
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) A.out[m][i * A.o_sm + n * A.o_sn] = (f16)acc[m];
}

// ------------------------------------------------------------------------------------------
// host side

static QuadLuts make_luts(const void* const* luts, int dtype) {
  QuadLuts L;
  for (int i = 0; i < 7; ++i) L.p[i] = luts[i];
  L.dtype = dtype;
  return L;
}

static int check_luts(const void* const* luts, int dtype) {
  PP_REQUIRE(luts != nullptr, "luts is null");
  PP_REQUIRE(dtype == PP_F16 || dtype == PP_F32, "lut_dtype must be PP_F16 or PP_F32");
  for (int i = 0; i < 7; ++i) PP_REQUIRE(luts[i] != nullptr, "lut %d is null", i);
  return PP_OK;
}

}  // namespace pp

using namespace pp;

extern "C" int64_t pp_quad_gemm_workspace_size(const void* a, int64_t a_sm, int64_t a_sk, const uint32_t* codes,
                                               int64_t c_sk, int64_t c_sn, int64_t plug_n, int64_t M, int64_t N,
                                               int64_t K) {
  if (M <= 0 || N <= 0) return 0;
  if (quad_rows_ok(a, a_sm, a_sk, codes, c_sk, c_sn, M, N, K)) return quad_rows_workspace(M, N, plug_n);
  // (K,N) codes: blocks of up to 8 tokens, one after another, sharing the workspace (the
  // last block may have 1..7 tokens: the larger of the 4- and 8-token needs covers it)
  if (quad_kn_ok(a, a_sm, a_sk, codes, c_sk, c_sn, std::min<int64_t>(M, 8), N, K))
    return std::max(quad_kn_workspace(std::min<int64_t>(M, 8), N, K, plug_n),
                    quad_kn_workspace(std::min<int64_t>(M, 4), N, K, plug_n));
  return 4 * N * K * (int64_t)sizeof(float);
}

template <typename O>
static int quad_dequant_to(const uint32_t* codes, int64_t c_sk, int64_t c_sn, const void* const* luts,
                               int lut_dtype, const float* scales, const uint32_t* plug_idx, const void* plug_vals,
                               int64_t plug_n, int64_t elem_base, void* const* out, int64_t N, int64_t K,
                               void* stream) {
  if (int rc = check_luts(luts, lut_dtype)) return rc;
  PP_REQUIRE(N >= 0 && K >= 0, "negative shape");
  PP_REQUIRE(codes != nullptr || N * K == 0, "codes is null");
  PP_REQUIRE(out != nullptr && out[0] && out[1] && out[2] && out[3], "out pointers are null");
  PP_REQUIRE(scales != nullptr, "scales is null");
  PP_REQUIRE(plug_n == 0 || (plug_idx && plug_vals), "plug arrays are null");
  PP_REQUIRE(plug_n == 0 || (c_sk == 1 && c_sn >= K) || (c_sn == 1 && c_sk >= N),
             "plug entries need a unit-stride (K,N) view");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (N * K == 0) return PP_OK;
  QuadDequantArgs A;
  A.codes = codes;
  A.c_sk = c_sk;
  A.c_sn = c_sn;
  A.luts = make_luts(luts, lut_dtype);
  for (int m = 0; m < 4; ++m) {
    A.s[m] = scales[m];
    A.out[m] = out[m];
  }
  A.N = N;
  A.K = K;
  bool vec = c_sn == 1 && c_sk % 4 == 0 && N % 4 == 0 && aligned(codes, 16) && N * K < (1ll << 32);
  for (int m = 0; m < 4; ++m) vec = vec && aligned(out[m], 16);
  if (vec) {
    const int64_t blocks = std::min<int64_t>((N * K / 4 + 255) / 256, (int64_t)device_cu_count() * 8);
    hipLaunchKernelGGL(quad_dequant_vec_kernel<O>, dim3((unsigned)blocks), dim3(256), 0, st, A);
  } else {
    const int64_t blocks = std::min<int64_t>((N * K + 255) / 256, (int64_t)device_cu_count() * 16);
    hipLaunchKernelGGL(quad_dequant_kernel<O>, dim3((unsigned)blocks), dim3(256), 0, st, A);
  }
  PP_LAUNCH_CHECK();
  if (plug_n > 0) {
    QuadPlugScatterArgs P;
    P.plug_idx = plug_idx;
    P.plug_vals = reinterpret_cast<const f16*>(plug_vals);
    P.plug_n = plug_n;
    P.elem_base = elem_base;
    P.c_sk = c_sk;
    P.c_sn = c_sn;
    for (int m = 0; m < 4; ++m) {
      P.s[m] = scales[m];
      P.out[m] = out[m];
    }
    P.N = N;
    P.K = K;
    P.o_k = N;
    P.o_n = 1;
    hipLaunchKernelGGL(quad_plug_scatter_kernel<O>, dim3((unsigned)((plug_n + 255) / 256)), dim3(256), 0, st, P);
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
}

extern "C" int pp_quad_dequant(const uint32_t* codes, int64_t c_sk, int64_t c_sn, const void* const* luts,
                               int lut_dtype, const float* scales, const uint32_t* plug_idx, const void* plug_vals,
                               int64_t plug_n, int64_t elem_base, float* const* out, int64_t N, int64_t K,
                               void* stream) {
  return quad_dequant_to<float>(codes, c_sk, c_sn, luts, lut_dtype, scales, plug_idx, plug_vals, plug_n, elem_base,
                                reinterpret_cast<void* const*>(out), N, K, stream);
}

extern "C" int pp_quad_dequant_f16(const uint32_t* codes, int64_t c_sk, int64_t c_sn, const void* const* luts,
                                   int lut_dtype, const float* scales, const uint32_t* plug_idx,
                                   const void* plug_vals, int64_t plug_n, int64_t elem_base, void* const* out,
                                   int64_t N, int64_t K, void* stream) {
  return quad_dequant_to<f16>(codes, c_sk, c_sn, luts, lut_dtype, scales, plug_idx, plug_vals, plug_n, elem_base,
                              out, N, K, stream);
}

extern "C" int pp_quad_dequant_f16_t(const uint32_t* codes, int64_t c_sk, const void* const* luts, int lut_dtype,
                                     const float* scales, const uint32_t* plug_idx, const void* plug_vals,
                                     int64_t plug_n, int64_t elem_base, void* const* out, int64_t N, int64_t K,
                                     void* stream) {
  if (int rc = check_luts(luts, lut_dtype)) return rc;
  PP_REQUIRE(N >= 0 && K >= 0, "negative shape");
  PP_REQUIRE(out != nullptr && out[0] && out[1] && out[2] && out[3], "out pointers are null");
  PP_REQUIRE(scales != nullptr, "scales is null");
  PP_REQUIRE(plug_n == 0 || (plug_idx && plug_vals), "plug arrays are null");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (N * K == 0) return PP_OK;
  PP_REQUIRE(codes != nullptr, "codes is null");
  PP_REQUIRE(N % 8 == 0 && K % 8 == 0 && c_sk >= N && c_sk % 4 == 0 && aligned(codes, 16),
             "the transposed decode needs N % 8 == 0, K % 8 == 0 and 16-byte aligned code rows "
             "(row stride >= N, a multiple of 4)");
  for (int m = 0; m < 4; ++m) PP_REQUIRE(aligned(out[m], 16), "out[%d] must be 16-byte aligned", m);
  QuadDequantTArgs A;
  A.codes = codes;
  A.c_sk = c_sk;
  A.luts = make_luts(luts, lut_dtype);
  for (int m = 0; m < 4; ++m) {
    A.s[m] = scales[m];
    A.out[m] = reinterpret_cast<f16*>(out[m]);
  }
  A.N = N;
  A.K = K;
  const int64_t tiles = ((N + DQT_T - 1) / DQT_T) * ((K + DQT_T - 1) / DQT_T);
  // 39 KiB of LDS a workgroup: four fit a CU
  const int64_t blocks = std::min<int64_t>(tiles, (int64_t)device_cu_count() * 4);
  hipLaunchKernelGGL(quad_dequant_t_kernel, dim3((unsigned)blocks), dim3(DQT_NT), 0, st, A);
  PP_LAUNCH_CHECK();
  if (plug_n > 0) {
    QuadPlugScatterArgs P;
    P.plug_idx = plug_idx;
    P.plug_vals = reinterpret_cast<const f16*>(plug_vals);
    P.plug_n = plug_n;
    P.elem_base = elem_base;
    P.c_sk = c_sk;
    P.c_sn = 1;
    for (int m = 0; m < 4; ++m) {
      P.s[m] = scales[m];
      P.out[m] = out[m];
    }
    P.N = N;
    P.K = K;
    P.o_k = 1;
    P.o_n = K;
    hipLaunchKernelGGL(quad_plug_scatter_kernel<f16>, dim3((unsigned)((plug_n + 255) / 256)), dim3(256), 0, st, P);
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
}

extern "C" int pp_quad_gemm_kernel(const void* a, int64_t a_sm, int64_t a_sk, const uint32_t* codes, int64_t c_sk,
                                   int64_t c_sn, int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  if (quad_rows_ok(a, a_sm, a_sk, codes, c_sk, c_sn, M, N, K)) return PP_GEMM_ROWS;
  if (quad_kn_ok(a, a_sm, a_sk, codes, c_sk, c_sn, std::min<int64_t>(M, 8), N, K)) return PP_GEMM_KN;
  return PP_GEMM_GENERIC;
}

extern "C" int pp_quad_gemm(const void* a, int64_t a_sm, int64_t a_sk, const uint32_t* codes, int64_t c_sk,
                            int64_t c_sn, const void* const* luts, int lut_dtype, const float* scales,
                            const uint32_t* plug_idx, const void* plug_vals, int64_t plug_n, int64_t elem_base,
                            void* const* out, int64_t o_sm, int64_t o_sn, int64_t M, int64_t N, int64_t K,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  if (int rc = check_luts(luts, lut_dtype)) return rc;
  PP_REQUIRE(M >= 0 && N >= 0 && K >= 0, "negative shape");
  PP_REQUIRE(out != nullptr && out[0] && out[1] && out[2] && out[3], "out pointers are null");
  PP_REQUIRE(scales != nullptr, "scales is null");
  PP_REQUIRE(plug_n >= 0 && (plug_n == 0 || (plug_idx && plug_vals)), "plug arrays are null");
  PP_REQUIRE(plug_n == 0 || (c_sk == 1 && c_sn >= K) || (c_sn == 1 && c_sk >= N),
             "plug entries need a unit-stride (K,N) view");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (M == 0 || N == 0) return PP_OK;
  PP_REQUIRE(a != nullptr && codes != nullptr, "a / codes is null");
  PP_REQUIRE(N < (1ll << 31) && K < (1ll << 31), "N and K must be < 2^31");
  const int64_t need = pp_quad_gemm_workspace_size(a, a_sm, a_sk, codes, c_sk, c_sn, plug_n, M, N, K);
  if (quad_rows_ok(a, a_sm, a_sk, codes, c_sk, c_sn, M, N, K))
    return quad_rows_single(a, a_sm, codes, c_sn, luts, lut_dtype, scales, plug_idx, plug_vals, plug_n, elem_base,
                            out, o_sm, o_sn, M, N, K, workspace, workspace_bytes, st);
  if (quad_kn_ok(a, a_sm, a_sk, codes, c_sk, c_sn, std::min<int64_t>(M, 8), N, K)) {
    for (int64_t i0 = 0; i0 < M; i0 += 8) {
      void* o[4];
      for (int m = 0; m < 4; ++m) o[m] = reinterpret_cast<f16*>(out[m]) + i0 * o_sm;
      if (int rc = quad_kn_gemm(reinterpret_cast<const f16*>(a) + i0 * a_sm, a_sm, codes, c_sk, luts, lut_dtype,
                                scales, plug_idx, plug_vals, plug_n, elem_base, o, o_sm, o_sn,
                                std::min<int64_t>(8, M - i0), N, K, workspace, workspace_bytes, st))
        return rc;
    }
    return PP_OK;
  }
  // generic: dequantise into the workspace, then multiply
  PP_REQUIRE(workspace_bytes >= need && workspace != nullptr, "workspace too small: need %lld bytes",
             (long long)need);
  float* w[4];
  for (int m = 0; m < 4; ++m) w[m] = reinterpret_cast<float*>(workspace) + (int64_t)m * N * K;
  const float one[4] = {scales[0], scales[1], scales[2], scales[3]};
  if (int rc = pp_quad_dequant(codes, c_sk, c_sn, luts, lut_dtype, one, plug_idx, plug_vals, plug_n, elem_base, w,
                               N, K, stream))
    return rc;
  QuadWsGemmArgs G;
  G.a = reinterpret_cast<const f16*>(a);
  G.a_sm = a_sm;
  G.a_sk = a_sk;
  for (int m = 0; m < 4; ++m) {
    G.w[m] = w[m];
    G.out[m] = reinterpret_cast<f16*>(out[m]);
  }
  G.o_sm = o_sm;
  G.o_sn = o_sn;
  G.M = M;
  G.N = N;
  G.K = K;
  hipLaunchKernelGGL(quad_ws_gemm_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)M), dim3(256), 0, st, G);
  PP_LAUNCH_CHECK();
  return PP_OK;
}

