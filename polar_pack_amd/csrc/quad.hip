// Quad-pack fused decode GEMV/GEMM for gfx950.
//
// One uint32 word per 4-tuple of weights (one weight per model):
//   [nq 8 | q1 8 | q2 8 | q3 8]  (quad_kernels.py:103-106, quaternion_packer.py:173-176)
// decoded as  r = norm[nq], w0 = r c1, w1 = r s1 c2, w2 = r s1 s2 c3, w3 = r s1 s2 s3
// (quad_kernels.py:108-121, quaternion_packer.py:178-185), times the per-model
// RMS s_m at the end (quad_kernels.py:131-134).
//
// Kernels:
//   quad_rows_kernel  -- batch <= 8 decode over codes laid out (N,K) row-major (the
//                        container stream layout).  One wavefront owns a task = up to
//                        RG rows x a K slice: it streams the codes once with 16-byte
//                        non-temporal loads (next segment in flight while the current
//                        one decodes), decodes in registers against LDS tables that are
//                        replicated so every lane of an LDS clock reads its own bank,
//                        folds x into the norm (rx = r*x: 3 mul + 4 fma per tuple at
//                        batch 1), reduces across the wave, and applies the plug table
//                        as exact corrections x*(plug - decoded).  Split-K tasks publish
//                        partial sums; the last slice to arrive adds them in slice order
//                        (deterministic) and resets its counter.  Rows that reach FP16
//                        tail positions are one-row tasks on a scalar path.
//   quad_dequant_kernel / quad_plug_scatter_kernel -- float32 weights (parity export
//                        and the generic path); quad_ws_gemm_kernel multiplies them.
#include "pp_common.h"

#include <algorithm>
#include <cmath>

namespace pp {

constexpr int QREPL_R = 32;   // norm table replicas (ds_read_b32 serves 32 lanes per clock)
constexpr int QREPL_C = 16;   // (cos, sin) table replicas (ds_read_b64 serves 16 lanes per clock)
// threads per workgroup: one workgroup per CU (128 KiB LDS); 8 tokens need the
// larger register budget of 8 waves per CU
constexpr int rows_threads(int MT) { return MT >= 8 ? 512 : 1024; }
constexpr int QSEG = 256;     // codes per wave per row per step (64 lanes x 4)
using QLds = QuadLds<QREPL_R, QREPL_C>;

struct QTask {
  const uint32_t* codes;  // code of (row0, k0)
  int64_t ldc;            // row stride of codes
  int64_t pos_row0;       // stream position of (row0, 0)
  const f16* x;           // x(0, 0)
  int64_t x_sm;
  f16* out[4];            // out_m(0, row0)
  int64_t o_sm, o_sn;
  int nrows, K, k0, k1;
  int64_t plug_lo, plug_hi;
  int group, slice, n_slices;
  int tail;
};

struct QuadRowsArgs {
  // single-projection front end (items == nullptr): task ti -> (rowgroup, slice)
  pp_quad_proj proj;
  int64_t o_sn;
  int n_slices, slice_len;
  const int64_t* rg_plug;   // plug range start of each row group (n_rowgroups + 1), or null
  // stream front end
  const pp_quad_proj* projs;
  const pp_quad_item* items;
  // common
  int64_t n_tasks;
  QuadLuts luts;
  float s[4];
  const uint32_t* plug_idx;
  const f16* plug_vals;     // (P, 4)
  int64_t plug_n;
  int M;
  int64_t n_codes;          // positions >= n_codes come from the tails
  const f16* tails[4];
  int64_t tail_len[4];
  float* part;              // split-K partial sums, group g at part + g * part_stride
  int64_t part_stride;      // floats per combine group
  uint32_t* counters;       // [group], zero between launches
};

template <int MT, int RG>
__device__ __forceinline__ void rows_task(const QLds& T, const QuadRowsArgs& A, const QTask& t,
                                          float (&acc)[RG][4][MT]) {
  const int lane = threadIdx.x & 63;
  const int rr = lane % QREPL_R, rc = lane % QREPL_C;
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int j = 0; j < MT; ++j) acc[r][m][j] = 0.f;

  const int len = t.k1 - t.k0;
  const uint32_t* cbase = t.codes + 4 * lane;
  const f16* xbase = t.x + t.k0 + 4 * lane;

  u32x4 q[RG];
#pragma unroll
  for (int r = 0; r < RG; ++r)
    q[r] = (r < t.nrows && 4 * lane < len) ? load_nt(cbase + (int64_t)r * t.ldc) : u32x4{0u, 0u, 0u, 0u};
  for (int kb = 0; kb < len; kb += QSEG) {
    u32x4 qn[RG];
    const int kn = kb + QSEG;
#pragma unroll
    for (int r = 0; r < RG; ++r)
      qn[r] = (r < t.nrows && kn + 4 * lane < len) ? load_nt(cbase + (int64_t)r * t.ldc + kn)
                                                   : u32x4{0u, 0u, 0u, 0u};
    const bool valid = kb + 4 * lane < len;
    float xv[MT][4];
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      if (valid && j < A.M) {
        const f16x4 h = *reinterpret_cast<const f16x4*>(xbase + (int64_t)j * t.x_sm + kb);
        xv[j][0] = (float)h.x;
        xv[j][1] = (float)h.y;
        xv[j][2] = (float)h.z;
        xv[j][3] = (float)h.w;
      } else {
        xv[j][0] = xv[j][1] = xv[j][2] = xv[j][3] = 0.f;
      }
    }
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const uint32_t cw4[4] = {q[r].x, q[r].y, q[r].z, q[r].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t cw = cw4[e];
        const float rv = T.r[(cw >> 24) * QREPL_R + rr];
        const float2 a = T.cs1[((cw >> 16) & 255u) * QREPL_C + rc];
        const float2 b = T.cs2[((cw >> 8) & 255u) * QREPL_C + rc];
        const float2 c = T.cs3[(cw & 255u) * QREPL_C + rc];
        if constexpr (MT == 1) {
          const float rx = rv * xv[0][e];
          acc[r][0][0] = fmaf(rx, a.x, acc[r][0][0]);
          const float t1 = rx * a.y;
          acc[r][1][0] = fmaf(t1, b.x, acc[r][1][0]);
          const float t2 = t1 * b.y;
          acc[r][2][0] = fmaf(t2, c.x, acc[r][2][0]);
          acc[r][3][0] = fmaf(t2, c.y, acc[r][3][0]);
        } else {
          const float rs = rv * a.y;
          const float rss = rs * b.y;
          const float w[4] = {rv * a.x, rs * b.x, rss * c.x, rss * c.y};
#pragma unroll
          for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int j = 0; j < MT; ++j) acc[r][m][j] = fmaf(w[m], xv[j][e], acc[r][m][j]);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RG; ++r) q[r] = qn[r];
  }
}

// Plug corrections for rows [0, nrows) x k in [k0, k1) of the task: lane p takes entry
// plug_lo + p and adds x_k * (plug - decoded) to its own partial sums.
template <int MT, int RG>
__device__ __forceinline__ void rows_plug(const QLds& T, const QuadRowsArgs& A, const QTask& t,
                                          float (&acc)[RG][4][MT]) {
  const int lane = threadIdx.x & 63;
  for (int64_t p0 = t.plug_lo; p0 < t.plug_hi; p0 += 64) {
    const int64_t p = p0 + lane;
    if (p >= t.plug_hi) continue;
    const int64_t off = (int64_t)A.plug_idx[p] - t.pos_row0;
    if (off < 0) continue;
    const int64_t row = off / t.ldc;
    const int k = (int)(off - row * t.ldc);
    if (row >= t.nrows || k < t.k0 || k >= t.k1) continue;
    float wd[4];
    quad_decode(T, t.codes[row * t.ldc + (k - t.k0)], lane % QREPL_R, lane % QREPL_C, wd[0], wd[1], wd[2], wd[3]);
    const f16x4 pv = *reinterpret_cast<const f16x4*>(A.plug_vals + 4 * p);
    const float dlt[4] = {(float)pv.x - wd[0], (float)pv.y - wd[1], (float)pv.z - wd[2], (float)pv.w - wd[3]};
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      if (j >= A.M) break;
      const float xk = (float)t.x[(int64_t)j * t.x_sm + k];
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        if (r == row) {
#pragma unroll
          for (int m = 0; m < 4; ++m) acc[r][m][j] = fmaf(xk, dlt[m], acc[r][m][j]);
        }
      }
    }
  }
}

// A row that reaches FP16 tail positions (>= n_codes), element by element:
// y_m = s_m * sum_{pos < n} x * decoded_m  +  sum_{n <= pos} x * tail_m[pos - n].
template <int MT>
__device__ void rows_tail_task(const QLds& T, const QuadRowsArgs& A, const QTask& t) {
  const int lane = threadIdx.x & 63;
  float accc[4][MT], acct[4][MT];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int j = 0; j < MT; ++j) accc[m][j] = acct[m][j] = 0.f;
  for (int k = lane; k < t.K; k += 64) {
    const int64_t pos = t.pos_row0 + k;
    float xk[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) xk[j] = j < A.M ? (float)t.x[(int64_t)j * t.x_sm + k] : 0.f;
    if (pos < A.n_codes) {
      float w[4];
      quad_decode(T, t.codes[k], lane % QREPL_R, lane % QREPL_C, w[0], w[1], w[2], w[3]);
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int j = 0; j < MT; ++j) accc[m][j] = fmaf(w[m], xk[j], accc[m][j]);
    } else {
      const int64_t ti = pos - A.n_codes;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (ti < A.tail_len[m]) {
          const float w = (float)A.tails[m][ti];
#pragma unroll
          for (int j = 0; j < MT; ++j) acct[m][j] = fmaf(w, xk[j], acct[m][j]);
        }
      }
    }
  }
  for (int64_t p0 = t.plug_lo; p0 < t.plug_hi; p0 += 64) {
    const int64_t p = p0 + lane;
    if (p >= t.plug_hi) continue;
    const int64_t k = (int64_t)A.plug_idx[p] - t.pos_row0;
    if (k < 0 || k >= t.K || t.pos_row0 + k >= A.n_codes) continue;
    float wd[4];
    quad_decode(T, t.codes[k], lane % QREPL_R, lane % QREPL_C, wd[0], wd[1], wd[2], wd[3]);
    const f16x4 pv = *reinterpret_cast<const f16x4*>(A.plug_vals + 4 * p);
    const float dlt[4] = {(float)pv.x - wd[0], (float)pv.y - wd[1], (float)pv.z - wd[2], (float)pv.w - wd[3]};
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      if (j >= A.M) break;
      const float xk = (float)t.x[(int64_t)j * t.x_sm + k];
#pragma unroll
      for (int m = 0; m < 4; ++m) accc[m][j] = fmaf(xk, dlt[m], accc[m][j]);
    }
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    // a model whose stream ends before this row does not have the row: it reads 0
    const bool has = t.pos_row0 < A.n_codes || t.pos_row0 - A.n_codes < A.tail_len[m];
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const float v = wave_sum(accc[m][j]) * A.s[m] + wave_sum(acct[m][j]);
      if (lane == 0 && j < A.M) t.out[m][(int64_t)j * t.o_sm] = (f16)(has ? v : 0.f);
    }
  }
}

template <int MT, int RG>
__device__ __forceinline__ void rows_finish(const QuadRowsArgs& A, const QTask& t, float (&acc)[RG][4][MT]) {
  const int lane = threadIdx.x & 63;
  constexpr int NV = RG * 4 * MT;
  static_assert(NV <= 64, "one lane per output value");
  // butterfly: every lane ends with every sum; lane v then owns value v
  float mine = 0.f;
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const float v = wave_sum(acc[r][m][j]);
        if (lane == (r * 4 + m) * MT + j) mine = v;
      }
  const int r = lane / (4 * MT), m = (lane / MT) % 4, j = lane % MT;
  const bool owner = lane < NV && r < t.nrows && j < A.M;
  if (t.n_slices <= 1) {
    if (owner) t.out[m][(int64_t)j * t.o_sm + (int64_t)r * t.o_sn] = (f16)(mine * A.s[m]);
    return;
  }
  float* grp = A.part + (int64_t)t.group * A.part_stride;
  if (lane < NV) grp[(int64_t)t.slice * NV + lane] = mine;
  __threadfence();
  uint32_t prev = 0;
  if (lane == 0) prev = atomicAdd(A.counters + t.group, 1u);
  prev = __shfl(prev, 0, 64);
  if (prev != (uint32_t)(t.n_slices - 1)) return;
  __threadfence();
  if (lane < NV) {
    float sum = 0.f;
    for (int s = 0; s < t.n_slices; ++s) sum += __builtin_nontemporal_load(grp + (int64_t)s * NV + lane);
    if (owner) t.out[m][(int64_t)j * t.o_sm + (int64_t)r * t.o_sn] = (f16)(sum * A.s[m]);
  }
  if (lane == 0) A.counters[t.group] = 0u;  // ready for the next launch on this stream
}

template <int MT, int RG>
__device__ __forceinline__ void resolve_task(const QuadRowsArgs& A, int64_t ti, QTask& t) {
  if (A.items != nullptr) {
    const pp_quad_item it = A.items[ti];
    const pp_quad_proj& P = A.projs[it.proj];
    t.k0 = it.k0;
    t.k1 = it.k1;
    t.codes = P.codes + (int64_t)it.row0 * P.ldc + it.k0;
    t.ldc = P.ldc;
    t.pos_row0 = P.pos0 + (int64_t)it.row0 * P.ldc;
    t.x = reinterpret_cast<const f16*>(P.x);
    t.x_sm = P.x_sm;
#pragma unroll
    for (int m = 0; m < 4; ++m) t.out[m] = reinterpret_cast<f16*>(P.out[m]) + it.row0;
    t.o_sm = P.o_sm;
    t.o_sn = 1;
    t.nrows = min(it.nrows, RG);
    t.K = P.K;
    t.plug_lo = it.plug_lo;
    t.plug_hi = it.plug_hi;
    t.group = it.group;
    t.slice = it.slice;
    t.n_slices = it.n_slices;
    t.tail = it.flags & PP_ITEM_TAIL;
  } else {
    const pp_quad_proj& P = A.proj;
    const int rg = (int)(ti / A.n_slices);
    const int slice = (int)(ti % A.n_slices);
    const int row0 = rg * RG;
    t.k0 = slice * A.slice_len;
    t.k1 = min(P.K, t.k0 + A.slice_len);
    t.codes = P.codes + (int64_t)row0 * P.ldc + t.k0;
    t.ldc = P.ldc;
    t.pos_row0 = P.pos0 + (int64_t)row0 * P.ldc;
    t.x = reinterpret_cast<const f16*>(P.x);
    t.x_sm = P.x_sm;
#pragma unroll
    for (int m = 0; m < 4; ++m) t.out[m] = reinterpret_cast<f16*>(P.out[m]) + (int64_t)row0 * A.o_sn;
    t.o_sm = P.o_sm;
    t.o_sn = A.o_sn;
    t.nrows = min(RG, P.N - row0);
    t.K = P.K;
    if (A.rg_plug != nullptr) {
      t.plug_lo = A.rg_plug[rg];
      t.plug_hi = A.rg_plug[rg + 1];
    } else {
      t.plug_lo = t.plug_hi = 0;
    }
    t.group = rg;
    t.slice = slice;
    t.n_slices = A.n_slices;
    t.tail = 0;
  }
}

template <int MT, int RG>
__global__ __launch_bounds__(rows_threads(MT)) void quad_rows_kernel(const QuadRowsArgs A) {
  __shared__ QLds T;
  quad_build_lds(T, A.luts);
  __syncthreads();
  constexpr int WAVES = rows_threads(MT) / 64;
  const int64_t gw = (int64_t)blockIdx.x * WAVES + (threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * WAVES;
  const int64_t t_begin = gw * A.n_tasks / nw, t_end = (gw + 1) * A.n_tasks / nw;
  for (int64_t ti = t_begin; ti < t_end; ++ti) {
    QTask t;
    resolve_task<MT, RG>(A, ti, t);
    if (t.tail) {
      rows_tail_task<MT>(T, A, t);
      continue;
    }
    float acc[RG][4][MT];
    rows_task<MT, RG>(T, A, t, acc);
    if (t.plug_hi > t.plug_lo) rows_plug<MT, RG>(T, A, t, acc);
    rows_finish<MT, RG>(A, t, acc);
  }
}

__global__ void zero_u32_kernel(uint32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Plug range start of each row group: first entry with idx >= pos0 + rg*RG*ldc.
__global__ void rowgroup_plug_kernel(const uint32_t* plug_idx, int64_t plug_n, int64_t pos0, int64_t ldc,
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
// Generic path: float32 weights out_m[k*N + n] = s_m * W_m[k, n], then a GEMM.
struct QuadDequantArgs {
  const uint32_t* codes;
  int64_t c_sk, c_sn;
  QuadLuts luts;
  float s[4];
  float* out[4];
  int64_t N, K;
};

__global__ __launch_bounds__(256) void quad_dequant_kernel(const QuadDequantArgs A) {
  __shared__ QuadLds<1, 1> T;
  quad_build_lds(T, A.luts);
  __syncthreads();
  const int64_t total = A.N * A.K;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t k = e / A.N, n = e - k * A.N;
    float w[4];
    quad_decode(T, A.codes[k * A.c_sk + n * A.c_sn], 0, 0, w[0], w[1], w[2], w[3]);
#pragma unroll
    for (int m = 0; m < 4; ++m) A.out[m][e] = w[m] * A.s[m];
  }
}

struct QuadPlugScatterArgs {
  const uint32_t* plug_idx;
  const f16* plug_vals;
  int64_t plug_n, elem_base;
  int64_t c_sk, c_sn;
  float s[4];
  float* out[4];
  int64_t N, K;
};

// Entries are unique positions, so the scatter has no write conflicts.
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
  const int64_t e = k * A.N + n;
#pragma unroll
  for (int m = 0; m < 4; ++m) A.out[m][e] = (float)A.plug_vals[4 * j + m] * A.s[m];
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

// Fast path: codes rows (N,K) row-major, 16-byte aligned rows, contiguous 8-byte aligned x rows.
static bool rows_fast_ok(const void* a, int64_t a_sm, int64_t a_sk, const uint32_t* codes, int64_t c_sk,
                         int64_t c_sn, int64_t M, int64_t K) {
  return c_sk == 1 && c_sn % 4 == 0 && c_sn >= K && K % 4 == 0 && aligned(codes, 16) && M >= 1 && M <= 8 &&
         (a_sk == 1 || K == 1) && (M == 1 || a_sm % 4 == 0) && aligned(a, 8) && K > 0;
}

template <int MT, int RG>
static int launch_rows(QuadRowsArgs& A, hipStream_t st) {
  const int grid = device_cu_count();
  hipLaunchKernelGGL((quad_rows_kernel<MT, RG>), dim3(grid), dim3(rows_threads(MT)), 0, st, A);
  PP_LAUNCH_CHECK();
  return PP_OK;
}

static int dispatch_rows(QuadRowsArgs& A, int mt, hipStream_t st) {
  switch (mt) {
    case 1: return launch_rows<1, 4>(A, st);
    case 2: return launch_rows<2, 2>(A, st);
    case 4: return launch_rows<4, 1>(A, st);
    default: return launch_rows<8, 1>(A, st);
  }
}

static int rows_rg(int mt) { return mt == 1 ? 4 : (mt == 2 ? 2 : 1); }
static int round_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

struct RowsPlan {
  int rg, n_rowgroups, n_slices, slice_len;
  int64_t n_tasks;
  int64_t part_bytes, counter_bytes, plug_bytes;
  int64_t total() const { return part_bytes + counter_bytes + plug_bytes; }
};

static RowsPlan plan_rows(int64_t M, int64_t N, int64_t K, int64_t plug_n) {
  RowsPlan p;
  const int mt = round_mt(M);
  p.rg = rows_rg(mt);
  p.n_rowgroups = (int)((N + p.rg - 1) / p.rg);
  // split K so that the grid has several tasks per wave and a task streams >= 2048 codes per row
  const int64_t waves = (int64_t)device_cu_count() * (rows_threads(mt) / 64);
  const int64_t segs = (K + QSEG - 1) / QSEG;
  int64_t want = (4 * waves + p.n_rowgroups - 1) / p.n_rowgroups;
  want = std::max<int64_t>(1, std::min<int64_t>(want, std::max<int64_t>(1, K / 2048)));
  const int64_t segs_per_slice = (segs + want - 1) / want;
  p.slice_len = (int)(segs_per_slice * QSEG);
  p.n_slices = (int)((K + p.slice_len - 1) / p.slice_len);
  p.n_tasks = (int64_t)p.n_rowgroups * p.n_slices;
  const int nv = p.rg * 4 * mt;
  p.part_bytes = p.n_slices > 1 ? ((int64_t)p.n_rowgroups * p.n_slices * nv * 4 + 255) / 256 * 256 : 0;
  p.counter_bytes = p.n_slices > 1 ? ((int64_t)p.n_rowgroups * 4 + 255) / 256 * 256 : 0;
  p.plug_bytes = plug_n > 0 ? ((int64_t)(p.n_rowgroups + 1) * 8 + 255) / 256 * 256 : 0;
  return p;
}

}  // namespace pp

using namespace pp;

extern "C" int64_t pp_quad_gemm_workspace_size(const void* a, int64_t a_sm, int64_t a_sk, const uint32_t* codes,
                                               int64_t c_sk, int64_t c_sn, int64_t plug_n, int64_t M, int64_t N,
                                               int64_t K) {
  if (M <= 0 || N <= 0) return 0;
  if (rows_fast_ok(a, a_sm, a_sk, codes, c_sk, c_sn, M, K)) return plan_rows(M, N, K, plug_n).total();
  return 4 * N * K * (int64_t)sizeof(float);
}

extern "C" int pp_quad_dequant(const uint32_t* codes, int64_t c_sk, int64_t c_sn, const void* const* luts,
                               int lut_dtype, const float* scales, const uint32_t* plug_idx, const void* plug_vals,
                               int64_t plug_n, int64_t elem_base, float* const* out, int64_t N, int64_t K,
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
  const int64_t blocks = std::min<int64_t>((N * K + 255) / 256, (int64_t)device_cu_count() * 16);
  hipLaunchKernelGGL(quad_dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, st, A);
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
    hipLaunchKernelGGL(quad_plug_scatter_kernel, dim3((unsigned)((plug_n + 255) / 256)), dim3(256), 0, st, P);
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
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
  const bool fast = rows_fast_ok(a, a_sm, a_sk, codes, c_sk, c_sn, M, K);
  if (fast) {
    const RowsPlan p = plan_rows(M, N, K, plug_n);
    PP_REQUIRE(workspace_bytes >= p.total() && (p.total() == 0 || workspace != nullptr),
               "workspace too small: need %lld bytes", (long long)p.total());
    char* ws = reinterpret_cast<char*>(workspace);
    QuadRowsArgs A = {};
    A.proj.codes = codes;
    A.proj.ldc = c_sn;
    A.proj.pos0 = elem_base;
    A.proj.x = a;
    A.proj.x_sm = a_sm;
    for (int m = 0; m < 4; ++m) A.proj.out[m] = out[m];
    A.proj.o_sm = o_sm;
    A.proj.N = (int32_t)N;
    A.proj.K = (int32_t)K;
    A.o_sn = o_sn;
    A.n_slices = p.n_slices;
    A.slice_len = p.slice_len;
    A.n_tasks = p.n_tasks;
    A.luts = make_luts(luts, lut_dtype);
    for (int m = 0; m < 4; ++m) A.s[m] = scales[m];
    A.plug_idx = plug_idx;
    A.plug_vals = reinterpret_cast<const f16*>(plug_vals);
    A.plug_n = plug_n;
    A.M = (int)M;
    A.n_codes = INT64_MAX;
    A.part = p.part_bytes ? reinterpret_cast<float*>(ws) : nullptr;
    A.counters = p.counter_bytes ? reinterpret_cast<uint32_t*>(ws + p.part_bytes) : nullptr;
    A.part_stride = (int64_t)p.n_slices * p.rg * 4 * round_mt(M);
    if (p.counter_bytes) {
      // counters start at zero; a fill kernel rather than a memset node keeps graph capture safe
      const int64_t nc = p.counter_bytes / 4;
      hipLaunchKernelGGL(zero_u32_kernel, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, st, A.counters, nc);
      PP_LAUNCH_CHECK();
    }
    if (plug_n > 0) {
      int64_t* rgp = reinterpret_cast<int64_t*>(ws + p.part_bytes + p.counter_bytes);
      hipLaunchKernelGGL(rowgroup_plug_kernel, dim3((p.n_rowgroups + 1 + 255) / 256), dim3(256), 0, st, plug_idx,
                         plug_n, elem_base, c_sn, p.rg, p.n_rowgroups, (int)N, rgp);
      PP_LAUNCH_CHECK();
      A.rg_plug = rgp;
    }
    return dispatch_rows(A, round_mt(M), st);
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

extern "C" int pp_quad_stream_layout(int64_t M, int* rows_per_item, int* values_per_slice) {
  PP_REQUIRE(M >= 1 && M <= 8, "the stream decode takes 1..8 tokens, got %lld", (long long)M);
  const int mt = round_mt(M);
  if (rows_per_item) *rows_per_item = rows_rg(mt);
  if (values_per_slice) *values_per_slice = rows_rg(mt) * 4 * mt;
  return PP_OK;
}

extern "C" int pp_quad_stream(const pp_quad_proj* projs, const pp_quad_item* items, int64_t n_items,
                              const float* const* luts, const float* scales, const uint32_t* plug_idx,
                              const void* plug_vals, int64_t n_codes, const void* const* tails,
                              const int64_t* tail_len, int64_t M, float* part, int64_t max_slices,
                              uint32_t* counters, void* stream) {
  PP_REQUIRE(projs && items, "projs / items are null");
  PP_REQUIRE(luts != nullptr, "luts is null");
  for (int i = 0; i < 7; ++i) PP_REQUIRE(luts[i] != nullptr, "lut %d is null", i);
  PP_REQUIRE(scales != nullptr, "scales is null");
  PP_REQUIRE(M >= 1 && M <= 8, "the stream decode takes 1..8 tokens, got %lld", (long long)M);
  PP_REQUIRE(max_slices <= 1 || (part != nullptr && counters != nullptr), "split-K items need part / counters");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (n_items == 0) return PP_OK;
  QuadRowsArgs A = {};
  A.projs = projs;
  A.items = items;
  A.n_tasks = n_items;
  A.luts = make_luts(reinterpret_cast<const void* const*>(luts), PP_F32);
  for (int m = 0; m < 4; ++m) A.s[m] = scales[m];
  A.plug_idx = plug_idx;
  A.plug_vals = reinterpret_cast<const f16*>(plug_vals);
  A.M = (int)M;
  A.n_codes = n_codes;
  for (int m = 0; m < 4; ++m) {
    A.tails[m] = tails ? reinterpret_cast<const f16*>(tails[m]) : nullptr;
    A.tail_len[m] = tail_len ? tail_len[m] : 0;
  }
  const int mt = round_mt(M);
  A.part = part;
  A.part_stride = std::max<int64_t>(max_slices, 1) * rows_rg(mt) * 4 * mt;
  A.counters = counters;
  return dispatch_rows(A, mt, st);
}
