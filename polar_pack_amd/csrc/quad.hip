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
//                        x*(plug - decoded) before the wave reduction.  No task spans
//                        waves, so no cross-wave combine (and no device-scope fence,
//                        which costs an L2 writeback on this part) is needed.
//   quad_tail_kernel  -- rows that reach FP16 tail positions, one row per wavefront on
//                        a scalar path (a handful of rows per stream).
//   quad_dequant_kernel / quad_plug_scatter_kernel -- float32 weights (parity export
//                        and the generic path); quad_ws_gemm_kernel multiplies them.
#include "pp_common.h"

#include <algorithm>
#include <cmath>

namespace pp {

constexpr int QSEG = 256;     // codes per wave per row per step (64 lanes x 4)
constexpr int QPROJ_CACHE = 256;   // projection descriptors staged in LDS (22.5 KiB)
using QLds = QuadLdsP;

// Uniform (scalar-register) state of a task; kept small, the pipeline holds one.
struct QTask {
  const uint32_t* codes;  // code of (row0, 0)
  const f16* x;           // x(0, 0)
  int64_t pos_row0;       // stream position of (row0, 0)
  int64_t plug_lo, plug_hi;
  int ldc;                // row stride of codes
  int x_sm;               // row stride of x
  int nrows, K, tail;
  int proj, row0;         // for the output pointers, read when the task finishes
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
#define PP_ROWS1_NSEG 2
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
  quad_decode_p(T, cw, quad_lane_offsets(lane), wd[0], wd[1], wd[2], wd[3]);
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
  const bool in = off >= 0 && row < t.nrows && k < t.K;
  return in ? row : -1;
}

// One chunk of a task: RG rows x NSEG segments of 256 codes, plus the activations.
template <int MT, int RG, int NSEG>
struct Chunk {
  u32x4 q[RG][NSEG];
  f16x4 xh[MT][NSEG];
};

// Issue every load of chunk [kc, kc + NSEG*256) of task t (codes past the row, rows past
// nrows and tokens past M read as zero).
template <int MT, int RG, int NSEG>
__device__ __forceinline__ void chunk_issue(const QuadRowsArgs& A, const QTask& t, int kc, Chunk<MT, RG, NSEG>& c) {
  const int lane = threadIdx.x & 63;
  const int len = t.K - kc;
  const f16* xb = t.x + kc + 4 * lane;
#pragma unroll
  for (int s = 0; s < NSEG; ++s) {
    const bool valid = s * QSEG + 4 * lane < len;
#pragma unroll
    for (int j = 0; j < MT; ++j)
      c.xh[j][s] = (valid && j < A.M) ? *reinterpret_cast<const f16x4*>(xb + (int64_t)j * t.x_sm + s * QSEG)
                                      : f16x4{0, 0, 0, 0};
  }
  const uint32_t* cb = t.codes + kc + 4 * lane;
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int s = 0; s < NSEG; ++s)
      c.q[r][s] = (r < t.nrows && s * QSEG + 4 * lane < len) ? load_nt(cb + (int64_t)r * t.ldc + s * QSEG)
                                                            : u32x4{0u, 0u, 0u, 0u};
}

// Decode a chunk and accumulate: LDS lookups addressed with one v_perm each, x folded
// into the norm at batch 1 (3 mul + 4 fma per tuple).
template <int MT, int RG, int NSEG>
__device__ __forceinline__ void chunk_compute(const QLds& T, const QuadRowsArgs& A, const Chunk<MT, RG, NSEG>& c,
                                              float (&acc)[RG][4][MT]) {
  const QuadLaneOff lo = quad_lane_offsets(threadIdx.x & 63);
  const char* lds = reinterpret_cast<const char*>(T.w);
#pragma unroll
  for (int s = 0; s < NSEG; ++s) {
    float xv[MT][4];
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      xv[j][0] = (float)c.xh[j][s].x;
      xv[j][1] = (float)c.xh[j][s].y;
      xv[j][2] = (float)c.xh[j][s].z;
      xv[j][3] = (float)c.xh[j][s].w;
    }
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const uint32_t cw4[4] = {c.q[r][s].x, c.q[r][s].y, c.q[r][s].z, c.q[r][s].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t cw = cw4[e];
        const float rv = *reinterpret_cast<const float*>(lds + quad_lds_addr<3>(cw, lo.r));
        const float2 a = *reinterpret_cast<const float2*>(lds + quad_lds_addr<2>(cw, lo.c1));
        const float2 b = *reinterpret_cast<const float2*>(lds + quad_lds_addr<1>(cw, lo.c2));
        const float2 d = *reinterpret_cast<const float2*>(lds + quad_lds_addr<0>(cw, lo.c3));
        if constexpr (MT == 1) {
          const float rx = rv * xv[0][e];
          acc[r][0][0] = fmaf(rx, a.x, acc[r][0][0]);
          const float t1 = rx * a.y;
          acc[r][1][0] = fmaf(t1, b.x, acc[r][1][0]);
          const float t2 = t1 * b.y;
          acc[r][2][0] = fmaf(t2, d.x, acc[r][2][0]);
          acc[r][3][0] = fmaf(t2, d.y, acc[r][3][0]);
        } else {
          const float rs = rv * a.y;
          const float rss = rs * b.y;
          const float w[4] = {rv * a.x, rs * b.x, rss * d.x, rss * d.y};
#pragma unroll
          for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int j = 0; j < MT; ++j) acc[r][m][j] = fmaf(w[m], xv[j][e], acc[r][m][j]);
        }
      }
    }
  }
}

// Plug entries of a task: the first 64 are located when the task starts (one load of
// their positions), their dependent loads (plugged code, fp16 values, x at the column)
// are issued a chunk later, and all of them are applied when the task ends.
template <int MT>
struct PlugPre {
  int prow, pk;
  uint32_t pcw;
  f16x4 pv;
  float pxk[MT];
};

template <int MT, int RG>
__device__ __forceinline__ void plug_locate_first(const QuadRowsArgs& A, const QTask& t, PlugPre<MT>& p) {
  const int lane = threadIdx.x & 63;
  p.prow = -1;
  p.pk = 0;
  if (lane < t.plug_hi - t.plug_lo) p.prow = plug_locate<RG>(A, t, t.plug_lo + lane, p.pk);
}

template <int MT>
__device__ __forceinline__ void plug_issue_deps(const QuadRowsArgs& A, const QTask& t, PlugPre<MT>& p) {
  const int lane = threadIdx.x & 63;
  p.pcw = 0;
  p.pv = f16x4{0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < MT; ++j) p.pxk[j] = 0.f;
  if (p.prow >= 0) {
    p.pcw = t.codes[(int64_t)p.prow * t.ldc + p.pk];
    p.pv = *reinterpret_cast<const f16x4*>(A.plug_vals + 4 * (t.plug_lo + lane));
#pragma unroll
    for (int j = 0; j < MT; ++j)
      if (j < A.M) p.pxk[j] = (float)t.x[(int64_t)j * t.x_sm + p.pk];
  }
}

template <int MT, int RG>
__device__ __forceinline__ void plug_finish(const QLds& T, const QuadRowsArgs& A, const QTask& t,
                                            const PlugPre<MT>& p, float (&acc)[RG][4][MT]) {
  const int lane = threadIdx.x & 63;
  if (p.prow >= 0) plug_apply<MT, RG>(T, A, t, p.prow, p.pcw, p.pv, p.pxk, acc);
  // tasks with more than 64 entries (dense plug tables): the rest, 64 at a time
  for (int64_t p0 = t.plug_lo + 64; p0 < t.plug_hi; p0 += 64) {
    const int64_t q = p0 + lane;
    if (q >= t.plug_hi) continue;
    int k;
    const int row = plug_locate<RG>(A, t, q, k);
    if (row < 0) continue;
    float xk[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) xk[j] = j < A.M ? (float)t.x[(int64_t)j * t.x_sm + k] : 0.f;
    plug_apply<MT, RG>(T, A, t, row, t.codes[(int64_t)row * t.ldc + k],
                       *reinterpret_cast<const f16x4*>(A.plug_vals + 4 * q), xk, acc);
  }
}

// Output pointers of a task (read from the projection descriptor when the task writes).
struct OutPtrs {
  f16* p[4];
  int64_t o_sm, o_sn;
};

__device__ __forceinline__ OutPtrs task_outputs(const QuadRowsArgs& A, const pp_quad_proj* Pc, const QTask& t) {
  OutPtrs o;
  if (t.proj < 0) {
#pragma unroll
    for (int m = 0; m < 4; ++m) o.p[m] = reinterpret_cast<f16*>(A.proj.out[m]) + (int64_t)t.row0 * A.o_sn;
    o.o_sm = A.proj.o_sm;
    o.o_sn = A.o_sn;
  } else if (Pc != nullptr && t.proj < QPROJ_CACHE) {
#pragma unroll
    for (int m = 0; m < 4; ++m) o.p[m] = reinterpret_cast<f16*>(uniform_ptr(Pc[t.proj].out[m])) + t.row0;
    o.o_sm = uniform64(Pc[t.proj].o_sm);
    o.o_sn = 1;
  } else {
#pragma unroll
    for (int m = 0; m < 4; ++m) o.p[m] = reinterpret_cast<f16*>(A.projs[t.proj].out[m]) + t.row0;
    o.o_sm = A.projs[t.proj].o_sm;
    o.o_sn = 1;
  }
  return o;
}

// A row that reaches FP16 tail positions (>= n_codes), element by element:
// y_m = s_m * sum_{pos < n} x * decoded_m  +  sum_{n <= pos} x * tail_m[pos - n].
template <int MT>
__device__ __forceinline__ void rows_tail_task(const QuadLds<1, 1>& T, const QuadRowsArgs& A,
                                               const pp_quad_proj* Pc, const QTask& t) {
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
      quad_decode(T, t.codes[k], 0, 0, w[0], w[1], w[2], w[3]);
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
    quad_decode(T, t.codes[k], 0, 0, wd[0], wd[1], wd[2], wd[3]);
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
  const OutPtrs o = task_outputs(A, Pc, t);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    // a model whose stream ends before this row does not have the row: it reads 0
    const bool has = t.pos_row0 < A.n_codes || t.pos_row0 - A.n_codes < A.tail_len[m];
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const float v = wave_sum(accc[m][j]) * A.s[m] + wave_sum(acct[m][j]);
      if (lane == 0 && j < A.M) o.p[m][(int64_t)j * o.o_sm] = (f16)(has ? v : 0.f);
    }
  }
}

template <int MT, int RG>
__device__ __forceinline__ void rows_finish(const QuadRowsArgs& A, const pp_quad_proj* Pc, const QTask& t,
                                            float (&acc)[RG][4][MT]) {
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
  const OutPtrs o = task_outputs(A, Pc, t);
  if (lane < RG * MT && r < t.nrows && j < A.M) {
    const int64_t off = (int64_t)j * o.o_sm + (int64_t)r * o.o_sn;
#pragma unroll
    for (int m = 0; m < 4; ++m) o.p[m][off] = (f16)(mine[m] * A.s[m]);
  }
}


// Task of stream item `it` on projection descriptor P (uniform values).
template <int RG>
__device__ __forceinline__ void task_from_item(const pp_quad_proj& P, int proj, int row0, int nrows, int flags,
                                               int64_t plo, int64_t phi, QTask& t) {
  const int ldc = uniform((int)P.ldc);
  t.K = uniform(P.K);
  t.codes = uniform_ptr(P.codes) + (int64_t)row0 * ldc;
  t.ldc = ldc;
  t.pos_row0 = uniform64(P.pos0) + (int64_t)row0 * ldc;
  t.x = reinterpret_cast<const f16*>(uniform_ptr(P.x));
  t.x_sm = uniform((int)P.x_sm);
  t.nrows = min(nrows, RG);
  t.plug_lo = plo;
  t.plug_hi = phi;
  t.tail = flags & PP_ITEM_TAIL;
  t.proj = proj;
  t.row0 = row0;
}

template <int MT, int RG>
__device__ __forceinline__ void single_task(const QuadRowsArgs& A, int64_t ti, QTask& t) {
  const pp_quad_proj& P = A.proj;
  const int row0 = (int)ti * A.rows_per_task;
  t.K = P.K;
  t.codes = P.codes + (int64_t)row0 * P.ldc;
  t.ldc = (int)P.ldc;
  t.pos_row0 = P.pos0 + (int64_t)row0 * P.ldc;
  t.x = reinterpret_cast<const f16*>(P.x);
  t.x_sm = (int)P.x_sm;
  t.nrows = min(A.rows_per_task, P.N - row0);
  if (A.rg_plug != nullptr) {
    t.plug_lo = uniform64(A.rg_plug[ti]);
    t.plug_hi = uniform64(A.rg_plug[ti + 1]);
  } else {
    t.plug_lo = t.plug_hi = 0;
  }
  t.tail = 0;
  t.proj = -1;
  t.row0 = row0;
}

// The tasks of one wavefront, in order: contiguous stream items (wave_bounds), items
// dealt round robin, or row groups of the single-projection front end.  Stream item
// records are read 64 at a time, one per lane, and handed out with readlane.
struct TaskSource {
  int64_t first, count, stride;
  int64_t batch;       // batch of 64 records held in `rec`, -1 before the first
  pp_quad_item rec;
};

template <int RG>
__device__ __forceinline__ bool fetch_task(const QuadRowsArgs& A, const pp_quad_proj* Pc, TaskSource& S, int64_t i,
                                           QTask& t) {
  if (i >= S.count) return false;
  if (A.items == nullptr) {
    single_task<1, RG>(A, S.first + i, t);
    return true;
  }
  const int lane = threadIdx.x & 63;
  const int64_t b = i >> 6;
  if (b != S.batch) {
    S.batch = b;
    const int64_t k = (b << 6) + lane;
    S.rec = pp_quad_item{};
    if (k < S.count) S.rec = A.items[S.first + k * S.stride];
  }
  const int j = (int)(i & 63);
  const int proj = __builtin_amdgcn_readlane(S.rec.proj, j);
  const int row0 = __builtin_amdgcn_readlane(S.rec.row0, j);
  const int nrows = __builtin_amdgcn_readlane(S.rec.nrows, j);
  const int flags = __builtin_amdgcn_readlane(S.rec.flags, j);
  const int64_t plo = lane_read64(S.rec.plug_lo, j), phi = lane_read64(S.rec.plug_hi, j);
  if (proj < QPROJ_CACHE) task_from_item<RG>(Pc[proj], proj, row0, nrows, flags, plo, phi, t);
  else task_from_item<RG>(A.projs[proj], proj, row0, nrows, flags, plo, phi, t);
  return true;
}

template <int MT, int RG>
__device__ __forceinline__ void zero_acc(float (&acc)[RG][4][MT]) {
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int j = 0; j < MT; ++j) acc[r][m][j] = 0.f;
}

template <int MT>
__global__ __launch_bounds__(RowsCfg<MT>::NT) void quad_rows_kernel(const QuadRowsArgs A) {
  constexpr int RG = RowsCfg<MT>::RG, NSEG = RowsCfg<MT>::NSEG;
  constexpr int WAVES = RowsCfg<MT>::NT / 64;
  constexpr int CHUNK = NSEG * QSEG;
  __shared__ QLds T;
  __shared__ pp_quad_proj Pc[QPROJ_CACHE];
  quad_build_lds_p(T, A.luts);
  if (A.items != nullptr) {
    const int np = (int)min<int64_t>(A.n_projs, QPROJ_CACHE);
    constexpr int W = sizeof(pp_quad_proj) / 4;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(A.projs);
    uint32_t* dst = reinterpret_cast<uint32_t*>(Pc);
    for (int i = threadIdx.x; i < np * W; i += blockDim.x) dst[i] = src[i];
  }
  __syncthreads();
  const int64_t gw = (int64_t)blockIdx.x * WAVES + uniform(threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * WAVES;
  TaskSource S;
  S.batch = -1;
  if (A.items != nullptr && A.wave_bounds != nullptr) {
    S.first = uniform64(A.wave_bounds[gw]);
    S.count = uniform64(A.wave_bounds[gw + 1]) - S.first;
    S.stride = 1;
  } else if (A.items != nullptr) {
    // round robin: item i to wave i % nw
    S.first = gw;
    S.count = gw < A.n_tasks ? (A.n_tasks - gw + nw - 1) / nw : 0;
    S.stride = nw;
  } else {
    S.first = gw * A.n_tasks / nw;
    S.count = (gw + 1) * A.n_tasks / nw - S.first;
    S.stride = 1;
  }
  QTask t;
  for (int64_t i = 0; fetch_task<RG>(A, Pc, S, i, t); ++i) {
    float acc[RG][4][MT];
    zero_acc<MT, RG>(acc);
    PlugPre<MT> pp;
    plug_locate_first<MT, RG>(A, t, pp);
    for (int kc = 0; kc < t.K; kc += CHUNK) {
      Chunk<MT, RG, NSEG> c;
      chunk_issue<MT, RG, NSEG>(A, t, kc, c);
      if (kc == 0) plug_issue_deps<MT>(A, t, pp);
      chunk_compute<MT, RG, NSEG>(T, A, c, acc);
    }
    plug_finish<MT, RG>(T, A, t, pp, acc);
    rows_finish<MT, RG>(A, Pc, t, acc);
  }
}

// Rows that reach the FP16 tails: one wavefront per tail item, compact tables.
template <int MT>
__global__ __launch_bounds__(256) void quad_tail_kernel(const QuadRowsArgs A) {
  __shared__ QuadLds<1, 1> T;
  quad_build_lds(T, A.luts);
  __syncthreads();
  const int64_t ti = (int64_t)blockIdx.x * 4 + uniform(threadIdx.x >> 6);
  if (ti >= A.n_tasks) return;
  const int lane = threadIdx.x & 63;
  pp_quad_item rec = {};
  if (lane == 0) rec = A.items[ti];
  const int proj = __builtin_amdgcn_readlane(rec.proj, 0);
  QTask t;
  task_from_item<1>(A.projs[proj], proj, __builtin_amdgcn_readlane(rec.row0, 0), 1, PP_ITEM_TAIL,
                    lane_read64(rec.plug_lo, 0), lane_read64(rec.plug_hi, 0), t);
  rows_tail_task<MT>(T, A, nullptr, t);   // outputs from the global descriptor table
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
                              const pp_quad_item* tail_items, int64_t n_tail, const int64_t* wave_bounds,
                              int64_t n_waves, const float* const* luts, const float* scales,
                              const uint32_t* plug_idx, const void* plug_vals, int64_t n_codes,
                              const void* const* tails, const int64_t* tail_len, int64_t M, void* stream) {
  PP_REQUIRE(projs != nullptr && n_projs >= 1, "no projections");
  PP_REQUIRE(n_items == 0 || items != nullptr, "items is null");
  PP_REQUIRE(n_tail == 0 || tail_items != nullptr, "tail_items is null");
  PP_REQUIRE(luts != nullptr, "luts is null");
  for (int i = 0; i < 7; ++i) PP_REQUIRE(luts[i] != nullptr, "lut %d is null", i);
  PP_REQUIRE(scales != nullptr, "scales is null");
  PP_REQUIRE(M >= 1 && M <= 8, "the stream decode takes 1..8 tokens, got %lld", (long long)M);
  PP_REQUIRE(wave_bounds == nullptr || n_waves == pp_quad_stream_waves(M),
             "wave_bounds were built for %lld waves, this device launches %lld", (long long)n_waves,
             (long long)pp_quad_stream_waves(M));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  QuadRowsArgs A = {};
  A.projs = projs;
  A.n_projs = n_projs;
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
  if (n_items > 0) {
    A.items = items;
    A.wave_bounds = wave_bounds;
    A.n_tasks = n_items;
    if (int rc = dispatch_rows(A, mt, device_cu_count(), st)) return rc;
  }
  if (n_tail > 0) {
    A.items = tail_items;
    A.wave_bounds = nullptr;
    A.n_tasks = n_tail;
    const unsigned grid = (unsigned)((n_tail + 3) / 4);
    switch (mt) {
      case 1: hipLaunchKernelGGL(quad_tail_kernel<1>, dim3(grid), dim3(256), 0, st, A); break;
      case 2: hipLaunchKernelGGL(quad_tail_kernel<2>, dim3(grid), dim3(256), 0, st, A); break;
      case 4: hipLaunchKernelGGL(quad_tail_kernel<4>, dim3(grid), dim3(256), 0, st, A); break;
      default: hipLaunchKernelGGL(quad_tail_kernel<8>, dim3(grid), dim3(256), 0, st, A); break;
    }
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
}
