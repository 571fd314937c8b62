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
//                        RG full rows.  It walks K in chunks of NSEG x 256 codes and, per
//                        chunk, issues the activations and every 16-byte non-temporal code
//                        load before using any of them (one memory round trip per chunk;
//                        the other waves of the CU hide it).  Codes are decoded in
//                        registers against LDS tables replicated so that every lane of an
//                        LDS clock reads its own bank; x is folded into the norm
//                        (rx = r*x: 3 mul + 4 fma per tuple at batch 1).  Plug entries of
//                        the task are located up front and their dependent loads ride
//                        with the first chunk; each is applied as an exact correction
//                        x*(plug - decoded) before the wave reduction.  Rows that reach
//                        FP16 tail positions are one-row tasks on a scalar path.  No
//                        task spans waves, so no cross-wave combine (and no device-scope
//                        fence, which costs an L2 writeback on this part) is needed.
//   quad_dequant_kernel / quad_plug_scatter_kernel -- float32 weights (parity export
//                        and the generic path); quad_ws_gemm_kernel multiplies them.
#include "pp_common.h"

#include <algorithm>
#include <cmath>

namespace pp {

constexpr int QREPL_R = 32;   // norm table replicas (ds_read_b32 serves 32 lanes per clock)
constexpr int QREPL_C = 16;   // (cos, sin) table replicas (ds_read_b64 serves 16 lanes per clock)
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
  int tail;
};

struct QuadRowsArgs {
  // single-projection front end (items == nullptr): task ti -> rows [ti*rows_per_task, ...)
  pp_quad_proj proj;
  int64_t o_sn;
  int rows_per_task;
  const int64_t* rg_plug;   // plug range start of each task's rows (n_tasks + 1), or null
  // stream front end
  const pp_quad_proj* projs;
  int64_t n_projs;
  const pp_quad_item* items;
  const int64_t* wave_bounds;  // per-wave item ranges (n_waves + 1), or null
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
};

// Per-token-count shape of a task: RG rows x NSEG segments of 256 codes.  Every load
// of a task (x, all codes, the first 64 plug entries) is issued before any of it is
// used, so a task costs one memory round trip; the plug-dependent loads (the plugged
// code word, its fp16 values, x at its column) are issued while the codes stream in.
#ifndef PP_ROWS1_RG
#define PP_ROWS1_RG 4
#endif
#ifndef PP_ROWS1_NSEG
#define PP_ROWS1_NSEG 4
#endif
#ifndef PP_ROWS1_NT
#define PP_ROWS1_NT 1024
#endif
template <int MT> struct RowsCfg;
template <> struct RowsCfg<1> { static constexpr int RG = PP_ROWS1_RG, NSEG = PP_ROWS1_NSEG, NT = PP_ROWS1_NT; };
template <> struct RowsCfg<2> { static constexpr int RG = 2, NSEG = 4, NT = 1024; };
template <> struct RowsCfg<4> { static constexpr int RG = 1, NSEG = 4, NT = 1024; };
template <> struct RowsCfg<8> { static constexpr int RG = 1, NSEG = 4, NT = 512; };

template <int MT, int RG>
__device__ __forceinline__ void plug_apply(const QLds& T, const QuadRowsArgs& A, const QTask& t, int row,
                                           uint32_t cw, f16x4 pv, const float (&xk)[MT], float (&acc)[RG][4][MT]) {
  const int lane = threadIdx.x & 63;
  float wd[4];
  quad_decode(T, cw, lane % QREPL_R, lane % QREPL_C, wd[0], wd[1], wd[2], wd[3]);
  const float dlt[4] = {(float)pv.x - wd[0], (float)pv.y - wd[1], (float)pv.z - wd[2], (float)pv.w - wd[3]};
  // every row is updated with a 0/1 weight: a branch on `row` would be folded into a
  // per-lane index into acc[], which puts the accumulators in scratch memory
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const float on = r == row ? 1.f : 0.f;
#pragma unroll
    for (int j = 0; j < MT; ++j)
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[r][m][j] = fmaf(on * xk[j], dlt[m], acc[r][m][j]);
  }
}

// Locate plug entry p inside the task: row (or -1 when outside its rows) and column.
template <int RG>
__device__ __forceinline__ int plug_locate(const QuadRowsArgs& A, const QTask& t, int64_t p, int& k) {
  const int64_t off = (int64_t)A.plug_idx[p] - t.pos_row0;
  int row = 0;
#pragma unroll
  for (int r = 1; r < RG; ++r)
    if (off >= (int64_t)r * t.ldc) row = r;
  k = (int)(off - (int64_t)row * t.ldc);
  const bool in = off >= 0 && row < t.nrows && k >= t.k0 && k < t.k1;
  return in ? row : -1;
}

template <int MT, int RG, int NSEG>
__device__ __forceinline__ void rows_item(const QLds& T, const QuadRowsArgs& A, const QTask& t,
                                          float (&acc)[RG][4][MT]) {
  const int lane = threadIdx.x & 63;
  const int rr = lane % QREPL_R, rc = lane % QREPL_C;
  constexpr int CHUNK = NSEG * QSEG;
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int j = 0; j < MT; ++j) acc[r][m][j] = 0.f;

  // first 64 plug entries of the task: positions now, dependent loads with the first chunk
  const int64_t n_plug = t.plug_hi - t.plug_lo;
  int prow = -1, pk = 0;
  if (lane < n_plug) prow = plug_locate<RG>(A, t, t.plug_lo + lane, pk);
  uint32_t pcw = 0;
  f16x4 pv = {0, 0, 0, 0};
  float pxk[MT];
#pragma unroll
  for (int j = 0; j < MT; ++j) pxk[j] = 0.f;

  const f16* xbase = t.x + t.k0 + 4 * lane;
  const uint32_t* cbase = t.codes + 4 * lane;
  for (int kc = 0; kc < t.k1 - t.k0; kc += CHUNK) {
    const int len = t.k1 - t.k0 - kc;   // codes of the row left from kc on
    // all activations and codes of the chunk, issued back to back
    f16x4 xh[MT][NSEG];
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
      const bool valid = s * QSEG + 4 * lane < len;
#pragma unroll
      for (int j = 0; j < MT; ++j)
        xh[j][s] = (valid && j < A.M)
                       ? *reinterpret_cast<const f16x4*>(xbase + (int64_t)j * t.x_sm + kc + s * QSEG)
                       : f16x4{0, 0, 0, 0};
    }
    u32x4 q[RG][NSEG];
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
      for (int s = 0; s < NSEG; ++s)
        q[r][s] = (r < t.nrows && s * QSEG + 4 * lane < len)
                      ? load_nt(cbase + (int64_t)r * t.ldc + kc + s * QSEG)
                      : u32x4{0u, 0u, 0u, 0u};
    if (kc == 0 && prow >= 0) {
      pcw = t.codes[(int64_t)prow * t.ldc + (pk - t.k0)];
      pv = *reinterpret_cast<const f16x4*>(A.plug_vals + 4 * (t.plug_lo + lane));
#pragma unroll
      for (int j = 0; j < MT; ++j)
        if (j < A.M) pxk[j] = (float)t.x[(int64_t)j * t.x_sm + pk];
    }
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
      float xv[MT][4];
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        xv[j][0] = (float)xh[j][s].x;
        xv[j][1] = (float)xh[j][s].y;
        xv[j][2] = (float)xh[j][s].z;
        xv[j][3] = (float)xh[j][s].w;
      }
#pragma unroll
      for (int r = 0; r < RG; ++r) {
        const uint32_t cw4[4] = {q[r][s].x, q[r][s].y, q[r][s].z, q[r][s].w};
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
    }
  }
  // plug corrections: x_k * (plug - decoded) on the lane that holds the entry
  if (prow >= 0) plug_apply<MT, RG>(T, A, t, prow, pcw, pv, pxk, acc);
  // tasks with more than 64 entries (dense plug tables): the rest, 64 at a time
  for (int64_t p0 = t.plug_lo + 64; p0 < t.plug_hi; p0 += 64) {
    const int64_t p = p0 + lane;
    if (p >= t.plug_hi) continue;
    int k;
    const int row = plug_locate<RG>(A, t, p, k);
    if (row < 0) continue;
    float xk[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) xk[j] = j < A.M ? (float)t.x[(int64_t)j * t.x_sm + k] : 0.f;
    plug_apply<MT, RG>(T, A, t, row, t.codes[(int64_t)row * t.ldc + (k - t.k0)],
                       *reinterpret_cast<const f16x4*>(A.plug_vals + 4 * p), xk, acc);
  }
}

// A row that reaches FP16 tail positions (>= n_codes), element by element:
// y_m = s_m * sum_{pos < n} x * decoded_m  +  sum_{n <= pos} x * tail_m[pos - n].
template <int MT>
__device__ __forceinline__ void rows_tail_task(const QLds& T, const QuadRowsArgs& A, const QTask& t) {
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
  // butterfly sums; lane r*MT + j keeps the 4 model sums of (row r, token j) and writes
  // them through statically indexed pointers (a per-lane model index would send the
  // pointer array to scratch memory)
  float mine[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const float v = wave_sum(acc[r][m][j]);
        if (lane == r * MT + j) mine[m] = v;
      }
  const int r = lane / MT, j = lane % MT;
  if (lane < RG * MT && r < t.nrows && j < A.M) {
    const int64_t off = (int64_t)j * t.o_sm + (int64_t)r * t.o_sn;
#pragma unroll
    for (int m = 0; m < 4; ++m) t.out[m][off] = (f16)(mine[m] * A.s[m]);
  }
}

constexpr int QPROJ_CACHE = 256;   // projection descriptors staged in LDS (22.5 KiB)

// Task of stream item `it` on projection descriptor P (uniform values).
template <int RG>
__device__ __forceinline__ void task_from_item(const pp_quad_proj& P, int row0, int nrows, int flags, int64_t plo,
                                               int64_t phi, QTask& t) {
  const int64_t ldc = uniform64(P.ldc);
  t.k0 = 0;
  t.K = uniform(P.K);
  t.k1 = t.K;
  t.codes = uniform_ptr(P.codes) + (int64_t)row0 * ldc;
  t.ldc = ldc;
  t.pos_row0 = uniform64(P.pos0) + (int64_t)row0 * ldc;
  t.x = reinterpret_cast<const f16*>(uniform_ptr(P.x));
  t.x_sm = uniform64(P.x_sm);
#pragma unroll
  for (int m = 0; m < 4; ++m) t.out[m] = reinterpret_cast<f16*>(uniform_ptr(P.out[m])) + row0;
  t.o_sm = uniform64(P.o_sm);
  t.o_sn = 1;
  t.nrows = min(nrows, RG);
  t.plug_lo = plo;
  t.plug_hi = phi;
  t.tail = flags & PP_ITEM_TAIL;
}

template <int MT, int RG>
__device__ __forceinline__ void single_task(const QuadRowsArgs& A, int64_t ti, QTask& t) {
  const pp_quad_proj& P = A.proj;
  const int row0 = (int)ti * A.rows_per_task;
  t.k0 = 0;
  t.k1 = P.K;
  t.codes = P.codes + (int64_t)row0 * P.ldc;
  t.ldc = P.ldc;
  t.pos_row0 = P.pos0 + (int64_t)row0 * P.ldc;
  t.x = reinterpret_cast<const f16*>(P.x);
  t.x_sm = P.x_sm;
#pragma unroll
  for (int m = 0; m < 4; ++m) t.out[m] = reinterpret_cast<f16*>(P.out[m]) + (int64_t)row0 * A.o_sn;
  t.o_sm = P.o_sm;
  t.o_sn = A.o_sn;
  t.nrows = min(A.rows_per_task, P.N - row0);
  t.K = P.K;
  if (A.rg_plug != nullptr) {
    t.plug_lo = uniform64(A.rg_plug[ti]);
    t.plug_hi = uniform64(A.rg_plug[ti + 1]);
  } else {
    t.plug_lo = t.plug_hi = 0;
  }
  t.tail = 0;
}

template <int MT, int RG, int NSEG>
__device__ __forceinline__ void run_task(const QLds& T, const QuadRowsArgs& A, const QTask& t) {
  if (t.tail) {
    rows_tail_task<MT>(T, A, t);
    return;
  }
  float acc[RG][4][MT];
  rows_item<MT, RG, NSEG>(T, A, t, acc);
  rows_finish<MT, RG>(A, t, acc);
}

template <int MT>
__global__ __launch_bounds__(RowsCfg<MT>::NT) void quad_rows_kernel(const QuadRowsArgs A) {
  constexpr int RG = RowsCfg<MT>::RG, NSEG = RowsCfg<MT>::NSEG;
  constexpr int WAVES = RowsCfg<MT>::NT / 64;
  __shared__ QLds T;
  __shared__ pp_quad_proj Pc[QPROJ_CACHE];
  quad_build_lds(T, A.luts);
  if (A.items != nullptr) {
    const int np = (int)min<int64_t>(A.n_projs, QPROJ_CACHE);
    constexpr int W = sizeof(pp_quad_proj) / 4;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(A.projs);
    uint32_t* dst = reinterpret_cast<uint32_t*>(Pc);
    for (int i = threadIdx.x; i < np * W; i += blockDim.x) dst[i] = src[i];
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int64_t gw = (int64_t)blockIdx.x * WAVES + uniform(threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * WAVES;
  if (A.items == nullptr) {
    const int64_t t_begin = gw * A.n_tasks / nw, t_end = (gw + 1) * A.n_tasks / nw;
    for (int64_t ti = t_begin; ti < t_end; ++ti) {
      QTask t;
      single_task<MT, RG>(A, ti, t);
      run_task<MT, RG, NSEG>(T, A, t);
    }
    return;
  }
  // Stream items: with wave_bounds, wave gw runs the contiguous range [bounds[gw], bounds[gw+1]);
  // without, items are dealt round robin (item i to wave i % nw), which keeps the pages all
  // waves touch at one time inside a window of nw items.
  int64_t first, count, stride;
  if (A.wave_bounds != nullptr) {
    first = uniform64(A.wave_bounds[gw]);
    count = uniform64(A.wave_bounds[gw + 1]) - first;
    stride = 1;
  } else {
    first = gw;
    count = gw < A.n_tasks ? (A.n_tasks - gw + nw - 1) / nw : 0;
    stride = nw;
  }
  // item records 64 at a time, one per lane; task j of the batch is read out of lane j
  for (int64_t b = 0; b < count; b += 64) {
    const int nb = (int)min<int64_t>(64, count - b);
    pp_quad_item mine = {};
    if (lane < nb) mine = A.items[first + (b + lane) * stride];
    for (int j = 0; j < nb; ++j) {
      const int proj = __builtin_amdgcn_readlane(mine.proj, j);
      const int row0 = __builtin_amdgcn_readlane(mine.row0, j);
      const int nrows = __builtin_amdgcn_readlane(mine.nrows, j);
      const int flags = __builtin_amdgcn_readlane(mine.flags, j);
      const int64_t plo = lane_read64(mine.plug_lo, j), phi = lane_read64(mine.plug_hi, j);
      QTask t;
      if (proj < QPROJ_CACHE) task_from_item<RG>(Pc[proj], row0, nrows, flags, plo, phi, t);
      else task_from_item<RG>(A.projs[proj], row0, nrows, flags, plo, phi, t);
      run_task<MT, RG, NSEG>(T, A, t);
    }
  }
}

// Plug range start of each task: first entry with idx >= pos0 + task*rows_per_task*ldc.
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

template <int MT>
static int launch_rows(QuadRowsArgs& A, int64_t grid, hipStream_t st) {
  hipLaunchKernelGGL((quad_rows_kernel<MT>), dim3((unsigned)grid), dim3(RowsCfg<MT>::NT), 0, st, A);
  PP_LAUNCH_CHECK();
  return PP_OK;
}

static int round_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

struct RowsShape {
  int rg, chunk, waves_per_wg;
};

static RowsShape rows_shape(int mt) {
  switch (mt) {
    case 1: return {RowsCfg<1>::RG, RowsCfg<1>::NSEG * QSEG, RowsCfg<1>::NT / 64};
    case 2: return {RowsCfg<2>::RG, RowsCfg<2>::NSEG * QSEG, RowsCfg<2>::NT / 64};
    case 4: return {RowsCfg<4>::RG, RowsCfg<4>::NSEG * QSEG, RowsCfg<4>::NT / 64};
    default: return {RowsCfg<8>::RG, RowsCfg<8>::NSEG * QSEG, RowsCfg<8>::NT / 64};
  }
}

static int dispatch_rows(QuadRowsArgs& A, int mt, int64_t grid, hipStream_t st) {
  switch (mt) {
    case 1: return launch_rows<1>(A, grid, st);
    case 2: return launch_rows<2>(A, grid, st);
    case 4: return launch_rows<4>(A, grid, st);
    default: return launch_rows<8>(A, grid, st);
  }
}

struct RowsPlan {
  int rows_per_task;
  int64_t n_tasks, grid, plug_bytes;
  int64_t total() const { return plug_bytes; }
};

// Single-projection tasks: full rows, RG per task, or 1 per task when that keeps more
// waves busy; as many workgroups (one per CU at most: the LDS tables fill it) as tasks need.
static RowsPlan plan_rows(int64_t M, int64_t N, int64_t plug_n) {
  RowsPlan p;
  const int mt = round_mt(M);
  const RowsShape sh = rows_shape(mt);
  const int64_t waves = (int64_t)device_cu_count() * sh.waves_per_wg;
  p.rows_per_task = ((N + sh.rg - 1) / sh.rg >= waves) ? sh.rg : 1;
  p.n_tasks = (N + p.rows_per_task - 1) / p.rows_per_task;
  p.grid = std::max<int64_t>(1, std::min<int64_t>(device_cu_count(), (p.n_tasks + sh.waves_per_wg - 1) / sh.waves_per_wg));
  p.plug_bytes = plug_n > 0 ? ((p.n_tasks + 1) * 8 + 255) / 256 * 256 : 0;
  return p;
}

}  // namespace pp

using namespace pp;

extern "C" int64_t pp_quad_gemm_workspace_size(const void* a, int64_t a_sm, int64_t a_sk, const uint32_t* codes,
                                               int64_t c_sk, int64_t c_sn, int64_t plug_n, int64_t M, int64_t N,
                                               int64_t K) {
  if (M <= 0 || N <= 0) return 0;
  if (rows_fast_ok(a, a_sm, a_sk, codes, c_sk, c_sn, M, K)) return plan_rows(M, N, plug_n).total();
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
    const RowsPlan p = plan_rows(M, N, plug_n);
    PP_REQUIRE(workspace_bytes >= p.total() && (p.total() == 0 || workspace != nullptr),
               "workspace too small: need %lld bytes", (long long)p.total());
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
    A.rows_per_task = p.rows_per_task;
    A.n_tasks = p.n_tasks;
    A.luts = make_luts(luts, lut_dtype);
    for (int m = 0; m < 4; ++m) A.s[m] = scales[m];
    A.plug_idx = plug_idx;
    A.plug_vals = reinterpret_cast<const f16*>(plug_vals);
    A.plug_n = plug_n;
    A.M = (int)M;
    A.n_codes = INT64_MAX;
    if (plug_n > 0) {
      int64_t* rgp = reinterpret_cast<int64_t*>(workspace);
      hipLaunchKernelGGL(rowgroup_plug_kernel, dim3((unsigned)((p.n_tasks + 1 + 255) / 256)), dim3(256), 0, st,
                         plug_idx, plug_n, elem_base, c_sn, p.rows_per_task, (int)p.n_tasks, (int)N, rgp);
      PP_LAUNCH_CHECK();
      A.rg_plug = rgp;
    }
    return dispatch_rows(A, round_mt(M), p.grid, st);
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

extern "C" int pp_quad_stream_rows(int64_t M) {
  if (M < 1 || M > 8) {
    set_error("the stream decode takes 1..8 tokens, got %lld", (long long)M);
    return 0;
  }
  return rows_shape(round_mt(M)).rg;
}

extern "C" int64_t pp_quad_stream_waves(int64_t M) {
  if (M < 1 || M > 8) return 0;
  return (int64_t)device_cu_count() * rows_shape(round_mt(M)).waves_per_wg;
}

extern "C" int pp_quad_stream(const pp_quad_proj* projs, int64_t n_projs, const pp_quad_item* items, int64_t n_items,
                              const int64_t* wave_bounds, int64_t n_waves,
                              const float* const* luts, const float* scales, const uint32_t* plug_idx,
                              const void* plug_vals, int64_t n_codes, const void* const* tails,
                              const int64_t* tail_len, int64_t M, void* stream) {
  PP_REQUIRE(projs && items, "projs / items are null");
  PP_REQUIRE(luts != nullptr, "luts is null");
  for (int i = 0; i < 7; ++i) PP_REQUIRE(luts[i] != nullptr, "lut %d is null", i);
  PP_REQUIRE(scales != nullptr, "scales is null");
  PP_REQUIRE(M >= 1 && M <= 8, "the stream decode takes 1..8 tokens, got %lld", (long long)M);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (n_items == 0) return PP_OK;
  PP_REQUIRE(wave_bounds == nullptr || n_waves == pp_quad_stream_waves(M),
             "wave_bounds were built for %lld waves, this device launches %lld", (long long)n_waves,
             (long long)pp_quad_stream_waves(M));
  PP_REQUIRE(n_projs >= 1, "no projections");
  QuadRowsArgs A = {};
  A.projs = projs;
  A.n_projs = n_projs;
  A.items = items;
  A.wave_bounds = wave_bounds;
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
  return dispatch_rows(A, round_mt(M), device_cu_count(), st);
}
