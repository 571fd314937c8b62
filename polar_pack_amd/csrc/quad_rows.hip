// Fused quad-pack decode GEMV (batch <= 8) over codes laid out (N,K) row-major, the
// container stream layout.  Serves the whole-stream launch (pp_quad_stream) and the
// single-projection fast path of pp_quad_gemm.
//
// Word [nq 8 | q1 8 | q2 8 | q3 8] (quad_kernels.py:103-106, quaternion_packer.py:173-176)
// decodes to  w0 = r c1, w1 = r s1 c2, w2 = r s1 s2 c3, w3 = r s1 s2 s3
// (quad_kernels.py:108-121, quaternion_packer.py:178-185); the per-model RMS s_m is
// applied to the float32 sum at the end (quad_kernels.py:131-134).
//
// Structure (one workgroup per CU, persistent):
//  * LDS tables.  gfx950's LDS serves 256 B/clk; a b64 read runs at that rate only when
//    each 32-lane half covers all 64 banks, a b32 read when the lanes' replicas differ.
//    When the t1 and t2 tables are equal (they always are for the reference's packers:
//    both are cos/sin(pi i/255), quad_kernels.py:41-44), the 160 KiB layout holds
//    32 replicas of every entry: (cos,sin)(pi i/255) and (cos,sin)(2 pi i/255) as
//    256-byte rows, the norm as 128-byte rows.  Lane l reads replica l % 32, so every
//    lookup is conflict-free whatever the codes are.  Otherwise a 128 KiB layout with
//    16 replicas of four tables is used.
//  * Work.  Each wavefront owns a list of segments: runs of full rows of one
//    projection.  It walks a segment in tasks of RG rows and chunks of NSEG x 256
//    columns, software-pipelined: the codes and activations of the next chunk (also
//    across task boundaries) are in flight while the current one is decoded.  Loads are
//    bounds-checked buffer loads, so rows past the segment, columns past K and absent
//    plug entries read zero without branches.
//  * Plug table.  Entries are consumed in order: a task's entries are the next ones in
//    the sorted list whose position falls before the task's end.  Their positions are
//    loaded one task ahead; the plugged code (from the side table plug_code when the
//    caller built one, else from the code stream), its fp16 values and x at its column
//    are loaded with the task's first chunk, and each entry is applied as the exact
//    correction x*(plug - decoded) before the reduction (quaternion_packer.py:187-193
//    replaces the decoded tuple by the plug tuple; the sum is the same).
//  * Reduction.  The RG*4*MT partial sums of a lane are reduced across the wavefront by
//    a transposing butterfly (permlane32/16 swaps, then DPP): each step halves the
//    number of values a lane holds, so 16 sums cost ~35 instructions instead of 96
//    shuffles; lane groups end up holding distinct (row, model, token) sums and write them.
//  * Tails.  Rows that reach FP16 tail positions run in quad_tail_kernel, one row per
//    wavefront (quaternion_packer.py:201-210).
#include "quad_rows.h"
#include "quad_lds.h"
#include "rows_common.h"

#include <algorithm>

namespace pp {

constexpr int QSEG = 256;                 // columns per wave per row per segment (64 lanes x 4)
// ------------------------------------------------------------------ configuration
// Batch 1 (the decode step): 8 rows per task and 8 waves per CU measured fastest on
// the 3B-shaped stream (vs 4 rows / 16 waves: fewer per-task reductions and stores, and
// the lookups of 8 independent rows fill the LDS latency); 2 chunks in flight per wave.
#ifndef PP_ROWS1_RG
#define PP_ROWS1_RG 8
#endif
#ifndef PP_ROWS1_NSEG
#define PP_ROWS1_NSEG 1
#endif
#ifndef PP_ROWS1_NT
#define PP_ROWS1_NT 512
#endif
// RG rows per task, NSEG x 256 columns per chunk, NT threads per workgroup; one chunk
// is prefetched ahead of the one being decoded.
template <int MT> struct RowsCfg;
template <> struct RowsCfg<1> {
  static constexpr int RG = PP_ROWS1_RG, NSEG = PP_ROWS1_NSEG, NT = PP_ROWS1_NT;
};
#ifndef PP_ROWS4_RG
#define PP_ROWS4_RG 1
#endif
#ifndef PP_ROWS4_NSEG
#define PP_ROWS4_NSEG 2
#endif
template <> struct RowsCfg<2> { static constexpr int RG = 2, NSEG = 2, NT = 512; };
template <> struct RowsCfg<4> { static constexpr int RG = PP_ROWS4_RG, NSEG = PP_ROWS4_NSEG, NT = 512; };
template <> struct RowsCfg<8> { static constexpr int RG = 1, NSEG = 2, NT = 512; };

struct QuadRowsArgs {
  // one-Linear front end (segs == nullptr): the tasks of `proj`, cut into `parts` column
  // slices of whole chunks, dealt to the waves by direct_item
  pp_quad_proj proj;
  int64_t o_sn;
  int64_t n_tasks;
  int parts, n_chunks;       // column slices; chunks of the K columns
  int wg_parts;              // 1: a task's slices are waves of one workgroup, summed in LDS
  float* acc;                // parts > 1: accumulators [4][M][N] (zero on entry, left zero)
  uint32_t* cnt;             // parts > 1: one arrival counter per task (zero on entry, left zero)
  const int64_t* wave_plug;  // plug start of each wave's first row (n_waves + 1), or null
  // stream front end
  const pp_quad_proj* projs;
  const pp_quad_seg* segs;
  const int64_t* seg_bounds;  // wave w owns segs [seg_bounds[w], seg_bounds[w+1])
  // common
  QuadLuts luts;
  float s[4];
  const uint32_t* plug_idx;
  const f16* plug_vals;  // (P, 4)
  const uint32_t* plug_code;  // per entry: the code word at its position, or null (gathered)
  int64_t plug_n;
  int M;
  void* ws;              // split segments: uint32 task counters, float32 accumulators
};

// Uniform state of the segment a wave is working on.
struct SegCtx {
  rsrc_t rc;          // codes of the segment's rows (row r at byte r*ldc*4)
  rsrc_t rx;          // activations (token j, column k at byte (j*x_sm + k)*2)
  const uint32_t* codes;  // the same two, as pointers
  const f16* x;
  int64_t pos0;       // stream position of the segment's first row
  int ldc, K, nrows, x_sm;
  int row0;           // projection row of the segment's first row
  f16* out[4];        // outputs of the segment's first row
  int64_t o_sm, o_sn;
  int kbeg, kend;     // the columns decoded: [kbeg, kend)
  int parts;          // > 1: one of `parts` column slices, sums go through the workspace
  int N;              // rows of the projection (accumulator stride)
  float* acc;         // parts > 1: the projection's accumulators
  uint32_t* cnt;      // parts > 1: counter of the segment's first task
  bool park;          // slices meeting in LDS: the runner keeps its reduced sum (SegRunner::parked)
};

template <int MT, int RG, int NSEG>
struct Chunk {
  u32x4 q[RG][NSEG];
  u32x2 xr[MT][NSEG];   // fp16 x 4 per lane per segment, raw
  static constexpr int LOADS = RG * NSEG + MT * NSEG;
};

// Issue every load of one chunk (Chunk::LOADS instructions): RG rows x NSEG segments of
// codes starting at row `row` (of the segment) and column kc, plus the activations
// (read as 0 from the segment's column end on, which also cancels the codes read there).
// The buffer resources are rebased to the chunk in scalar registers, so each lane's
// offsets are fixed for the whole segment (no per-step vector address arithmetic):
// codes resource = rows [row, nrows) from column kc, num_records ends at column K of
// the segment's last row, so rows past the segment and columns past K of the last row
// read 0; columns past K of other rows read the next row's codes, which meet a zero x.
// live = false: the same instructions, every load reading nothing (a buffer filled past the
// wave's last chunk; kc must still name a chunk of the segment).
template <int MT, int RG, int NSEG>
__device__ __forceinline__ void chunk_issue(const SegCtx& S, int row, int kc, const uint32_t (&voff)[RG], int lane,
                                            Chunk<MT, RG, NSEG>& c, bool live = true) {
  const int64_t first = (int64_t)row * S.ldc + kc;
  const int64_t end = (int64_t)(S.nrows - 1) * S.ldc + S.K;   // one past the last code
  // not live: empty resources (a scalar choice, no per-lane offsets to select)
  const rsrc_t rc = make_rsrc(S.codes + first, live ? 4u * (uint32_t)(end - first) : 0u);
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int s = 0; s < NSEG; ++s) vload128(c.q[r][s], voff[r] + 1024u * s, rc);
  if constexpr (MT == 1) {
    const rsrc_t rx = make_rsrc(S.x + kc, live ? 2u * (uint32_t)(S.kend - kc) : 0u);   // past kend: reads 0
#pragma unroll
    for (int s = 0; s < NSEG; ++s) vload64(c.xr[0][s], 8u * lane + 512u * s, rx);
  } else {
#pragma unroll
    for (int s = 0; s < NSEG; ++s) {
      const int k = kc + s * QSEG + 4 * lane;
      const bool valid = live && k < S.kend;
#pragma unroll
      for (int j = 0; j < MT; ++j) vload64(c.xr[j][s], valid ? 2u * (uint32_t)(j * S.x_sm + k) : OOB, S.rx);
    }
  }
}

// Table values of one code word.
struct Tup {
  float r;
  float2 a, b, c;
};

// Decode a chunk and accumulate the normalised products.  At batch 1 x is folded
// into the norm: rx = r*x, acc0 += rx*c1, t1 = rx*s1, acc1 += t1*c2, t2 = t1*s2,
// acc2 += t2*c3, acc3 += t2*s3 (3 mul + 4 fma per tuple).
// The lookups run one group of GT tuples ahead of the arithmetic (the scheduler would
// otherwise wait for each tuple's four reads before issuing the next tuple's), with
// at most 2*4*GT LDS reads in flight (the LDS counter holds 15).  GT = 2 measured 0.4%
// faster than 4 on the 3B-shaped stream (1.796 vs 1.802 ms, means of 4-6 runs on three
// boxes); 8 spills.
template <int MT, int RG, int NSEG, class L>
__device__ __forceinline__ void chunk_compute(const char* lds, const LaneOff& lo, const Chunk<MT, RG, NSEG>& c,
                                              float (&acc)[RG][4][MT]) {
#ifndef PP_LOOKUP_GROUP
#define PP_LOOKUP_GROUP 2
#endif
  constexpr int GT = PP_LOOKUP_GROUP;       // tuples per group
  constexpr int NT = RG * NSEG * 4;         // tuples per lane in the chunk
  constexpr int NG = NT / GT;
  static_assert(NT % GT == 0, "the lookup group must divide the tuples of a chunk");
  float xv[MT][NSEG][4];
#pragma unroll
  for (int s = 0; s < NSEG; ++s)
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const f16x4 xh = __builtin_bit_cast(f16x4, c.xr[j][s]);
      xv[j][s][0] = (float)xh.x;
      xv[j][s][1] = (float)xh.y;
      xv[j][s][2] = (float)xh.z;
      xv[j][s][3] = (float)xh.w;
    }
  // tuple t: row r = t / (4*NSEG), segment s = (t / 4) % NSEG, element e = t % 4
  auto word = [&](int t) -> uint32_t {
    const u32x4 q = c.q[t / (4 * NSEG)][(t / 4) % NSEG];
    const int e = t % 4;
    return e == 0 ? q.x : e == 1 ? q.y : e == 2 ? q.z : q.w;
  };
  Tup buf[2][GT];
#pragma unroll
  for (int u = 0; u < GT; ++u) lookup<L>(lds, word(u), lo, buf[0][u].r, buf[0][u].a, buf[0][u].b, buf[0][u].c);
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (g + 1 < NG) {
#pragma unroll
      for (int u = 0; u < GT; ++u) {
        Tup& T = buf[(g + 1) & 1][u];
        lookup<L>(lds, word((g + 1) * GT + u), lo, T.r, T.a, T.b, T.c);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < GT; ++u) {
      const int t = g * GT + u;
      const int r = t / (4 * NSEG), s = (t / 4) % NSEG, e = t % 4;
      const Tup& T = buf[g & 1][u];
      if constexpr (MT == 1) {
        const float rx = T.r * xv[0][s][e];
        acc[r][0][0] = fmaf(rx, T.a.x, acc[r][0][0]);
        const float t1 = rx * T.a.y;
        acc[r][1][0] = fmaf(t1, T.b.x, acc[r][1][0]);
        const float t2 = t1 * T.b.y;
        acc[r][2][0] = fmaf(t2, T.c.x, acc[r][2][0]);
        acc[r][3][0] = fmaf(t2, T.c.y, acc[r][3][0]);
      } else {
        const float rs = T.r * T.a.y;
        const float rss = rs * T.b.y;
        const float w[4] = {T.r * T.a.x, rs * T.b.x, rss * T.c.x, rss * T.c.y};
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int j = 0; j < MT; ++j) acc[r][m][j] = fmaf(w[m], xv[j][s][e], acc[r][m][j]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// ------------------------------------------------------------------ plug entries
template <int MT>
struct PlugSt {
  uint32_t idx;     // stream position of entry pc + lane (loaded a task ahead)
  int row;          // row in the task of this lane's entry, -1 when none
  uint32_t cw;      // plugged code word
  u32x2 pv;         // plug values (normalised tuple, fp16 x 4)
  uint32_t xk[MT];  // x at the entry's column (fp16 bits)
  bool dense;       // the task has >= 64 entries: the rest are applied when it ends
  static constexpr int LOADS = 3 + MT;   // cw, pv, xk[MT], next idx
};

__device__ __forceinline__ rsrc_t plug_idx_rsrc(const QuadRowsArgs& A, int64_t pc) {
  const int64_t left = A.plug_n - pc;
  const uint32_t bytes = left <= 0 ? 0u : (uint32_t)std::min<int64_t>(left * 4, 0x7FFFFFF0);
  return make_rsrc(A.plug_idx + (left > 0 ? pc : 0), bytes);
}
__device__ __forceinline__ rsrc_t plug_code_rsrc(const QuadRowsArgs& A, int64_t pc) {
  const int64_t left = A.plug_n - pc;
  const uint32_t bytes = left <= 0 ? 0u : (uint32_t)std::min<int64_t>(left * 4, 0x7FFFFFF0);
  return make_rsrc(A.plug_code + (left > 0 ? pc : 0), bytes);
}
__device__ __forceinline__ rsrc_t plug_val_rsrc(const QuadRowsArgs& A, int64_t pc) {
  const int64_t left = A.plug_n - pc;
  const uint32_t bytes = left <= 0 ? 0u : (uint32_t)std::min<int64_t>(left * 8, 0x7FFFFFF0);
  return make_rsrc(A.plug_vals + 4 * (left > 0 ? pc : 0), bytes);
}

// Row (or -1) and column of stream position `pos` inside the task starting at tpos0.
template <int RG>
__device__ __forceinline__ int plug_locate(int64_t pos, int64_t tpos0, int ldc, int K, int nr, int& k) {
  const int64_t off = pos - tpos0;
  int row = 0;
#pragma unroll
  for (int r = 1; r < RG; ++r)
    if (off >= (int64_t)r * ldc) row = r;
  k = (int)(off - (int64_t)row * ldc);
  return (off >= 0 && row < nr && k < K) ? row : -1;
}

// Start of task ti (P.idx has arrived): find its entries among the 64 loaded, issue
// their dependent loads and the next task's positions (PlugSt::LOADS instructions,
// all lanes, out of range where there is nothing to load), advance the cursor pc.
template <int MT, int RG>
__device__ __forceinline__ void plug_begin(const QuadRowsArgs& A, const SegCtx& S, int ti, int lane, int64_t& pc,
                                           PlugSt<MT>& P) {
  const int64_t tpos0 = S.pos0 + (int64_t)ti * RG * S.ldc;
  const int nr = min(RG, S.nrows - ti * RG);
  const int64_t tend = tpos0 + (int64_t)nr * S.ldc;
  const bool in = (pc + lane < A.plug_n) && ((int64_t)P.idx < tend);
  const int cnt = __popcll(__ballot(in));
  int k = 0;
  int row = in ? plug_locate<RG>((int64_t)P.idx, tpos0, S.ldc, S.K, nr, k) : -1;
  if (k < S.kbeg || k >= S.kend) row = -1;   // consumed with the task's rows, applied by its slice
  P.row = row;
  const bool v = row >= 0;
  // the plugged word from the side table (entry pc + lane) or, without one, from the codes
  const bool tab = A.plug_code != nullptr;
  vload32(P.cw, v ? (tab ? 4u * lane : 4u * (uint32_t)((ti * RG + row) * S.ldc + k)) : OOB,
          tab ? plug_code_rsrc(A, pc) : S.rc);
  vload64(P.pv, in ? 8u * lane : OOB, plug_val_rsrc(A, pc));
#pragma unroll
  for (int j = 0; j < MT; ++j) vload16(P.xk[j], (v && j < A.M) ? 2u * (uint32_t)(j * S.x_sm + k) : OOB, S.rx);
  P.dense = cnt == 64;
  pc += cnt;
  vload32(P.idx, 4u * lane, plug_idx_rsrc(A, pc));
}

template <int MT, int RG, class L>
__device__ __forceinline__ void plug_correct(const char* lds, const LaneOff& lo, int row, uint32_t cw, f16x4 pv,
                                             const float (&xk)[MT], float (&acc)[RG][4][MT]) {
  // the decoded tuple is rebuilt from the same tables as the chunk, so the correction
  // cancels its contribution exactly up to float32 rounding
  float r;
  float2 a, b, c;
  lookup<L>(lds, cw, lo, r, a, b, c);
  const float rs = r * a.y, rss = rs * b.y;
  const float dlt[4] = {(float)pv.x - r * a.x, (float)pv.y - rs * b.x, (float)pv.z - rss * c.x,
                        (float)pv.w - rss * c.y};
  // every row is updated with a 0/1 weight: indexing acc by a per-lane row would put
  // the accumulators in scratch memory
#pragma unroll
  for (int q = 0; q < RG; ++q) {
    const float on = q == row ? 1.f : 0.f;
#pragma unroll
    for (int j = 0; j < MT; ++j)
#pragma unroll
      for (int m = 0; m < 4; ++m) acc[q][m][j] = fmaf(on * xk[j], dlt[m], acc[q][m][j]);
  }
}

// Finish the plug entries of task ti: apply the ones located when it began; for a dense
// task (>= 64 entries), the rest too (loaded and used at once: rare), then reload the
// next task's positions at the advanced cursor.  Returns 1 when it took the dense path.
template <int MT, int RG, class L>
__device__ __forceinline__ int plug_end(const char* lds, const LaneOff& lo, const QuadRowsArgs& A, const SegCtx& S,
                                        int ti, int lane, int64_t& pc, PlugSt<MT>& P, float (&acc)[RG][4][MT]) {
  if (P.row >= 0) {
    float xk[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) xk[j] = h2f(P.xk[j]);
    plug_correct<MT, RG, L>(lds, lo, P.row, P.cw, __builtin_bit_cast(f16x4, P.pv), xk, acc);
  }
  if (!P.dense) return 0;
  const int64_t tpos0 = S.pos0 + (int64_t)ti * RG * S.ldc;
  const int nr = min(RG, S.nrows - ti * RG);
  const int64_t tend = tpos0 + (int64_t)nr * S.ldc;
  const uint32_t* codes = S.codes;
  const f16* x = S.x;
  for (;;) {
    const int64_t q = pc + lane;
    const bool has = q < A.plug_n;
    const int64_t pos = has ? (int64_t)A.plug_idx[q] : tend;
    const bool in = pos < tend;
    const int cnt = __popcll(__ballot(in));
    int k = 0;
    int row = in ? plug_locate<RG>(pos, tpos0, S.ldc, S.K, nr, k) : -1;
    if (k < S.kbeg || k >= S.kend) row = -1;
    if (row >= 0) {
      float xk[MT];
#pragma unroll
      for (int j = 0; j < MT; ++j) xk[j] = j < A.M ? (float)x[(int64_t)j * S.x_sm + k] : 0.f;
      const uint32_t cw = A.plug_code ? A.plug_code[q] : codes[(int64_t)(ti * RG + row) * S.ldc + k];
      const f16x4 pv = *reinterpret_cast<const f16x4*>(A.plug_vals + 4 * q);
      plug_correct<MT, RG, L>(lds, lo, row, cw, pv, xk, acc);
    }
    pc += cnt;
    if (cnt < 64) break;
  }
  vload32(P.idx, 4u * lane, plug_idx_rsrc(A, pc));
  // wait for it here: a load still in flight on this rare path would make the compiler
  // assume it may be in flight at every next use, and wait for the prefetch there
  asm volatile("" : : "v"(P.idx));
  return 1;
}

// The reduced sum a lane holds after the transposing reduction, and where it goes.
template <int MT, int RG>
struct Reduced {
  float y;       // normalised sum of (row r, model m, token j)
  int r, m, j;
  bool wr;       // this lane writes it
};

// The (row, model, token) lane `lane` holds after the reduction below, and whether it writes.
template <int MT, int RG>
__device__ __forceinline__ Reduced<MT, RG> task_slot(const QuadRowsArgs& A, const SegCtx& S, int ti, int lane) {
  constexpr int LNV = Log2<RG * 4 * MT>::v;
  Reduced<MT, RG> o;
  o.y = 0.f;
  const int idx = lane >> (6 - LNV);
  o.r = idx / (4 * MT);
  o.m = (idx / MT) & 3;
  o.j = idx % MT;
  const int nr = min(RG, S.nrows - ti * RG);
  o.wr = (lane & ((1 << (6 - LNV)) - 1)) == 0 && o.r < nr && o.j < A.M;
  return o;
}

template <int MT, int RG>
__device__ __forceinline__ Reduced<MT, RG> task_reduce(const QuadRowsArgs& A, const SegCtx& S, int ti, int lane,
                                                       float (&acc)[RG][4][MT]) {
  constexpr int NV = RG * 4 * MT;
  constexpr int LNV = Log2<NV>::v;
  static_assert((1 << LNV) == NV, "RG*4*MT must be a power of two");
  float v[NV];
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int j = 0; j < MT; ++j) v[(r * 4 + m) * MT + j] = acc[r][m][j];
  Reduced<MT, RG> o = task_slot<MT, RG>(A, S, ti, lane);
  o.y = wave_transpose_reduce<LNV>(v, lane);
  return o;
}

// Store value h (fp16 bits) of (row r of task ti, model m, token j) from the lanes with wr.
template <int MT, int RG>
__device__ __forceinline__ void task_store(const QuadRowsArgs& A, const SegCtx& S, int ti, const Reduced<MT, RG>& o,
                                           const float (&val)[4]) {
  const uint32_t off = 2u * (uint32_t)((int64_t)o.j * S.o_sm + (int64_t)(ti * RG + o.r) * S.o_sn);
  // one store per model (4 counted stores), each lane writing only its own model:
  // selecting the pointer per lane would index the pointer array in scratch memory
  const uint32_t obytes = 2u * (uint32_t)((int64_t)(A.M - 1) * S.o_sm + (int64_t)(S.nrows - 1) * S.o_sn + 1);
#pragma unroll
  for (int mm = 0; mm < 4; ++mm) {
    const f16 h = (f16)val[mm];
    vstore16((uint32_t)__builtin_bit_cast(unsigned short, h), (o.wr && o.m == mm) ? off : OOB,
             make_rsrc(S.out[mm], obytes));
  }
}

template <int MT, int RG>
__device__ __forceinline__ void task_write(const QuadRowsArgs& A, const SegCtx& S, int ti, int lane,
                                           float (&acc)[RG][4][MT]) {
  const Reduced<MT, RG> o = task_reduce<MT, RG>(A, S, ti, lane, acc);
  const float val[4] = {o.y * A.s[0], o.y * A.s[1], o.y * A.s[2], o.y * A.s[3]};
  task_store<MT, RG>(A, S, ti, o, val);
}

// A column slice of task ti: add the scaled sums to the projection's accumulators and
// count the part in the task's counter; the last part to arrive takes the totals
// (swapping in zeros, so the workspace is clean for the next launch), writes the
// outputs and clears the counter.  Every access to the workspace is a device-scope
// atomic, performed where all CUs see it, so no cache maintenance is needed; the order
// "sums before count" comes from a data dependence: the count added is 1 + 0 * (the
// values the sum atomics returned), so it cannot be issued before they completed.
template <int MT, int RG>
__device__ __forceinline__ void task_accumulate(const QuadRowsArgs& A, const SegCtx& S, int ti, int lane,
                                                float (&acc)[RG][4][MT]) {
  const Reduced<MT, RG> o = task_reduce<MT, RG>(A, S, ti, lane, acc);
  // the scale of the lane's model, selected among values: a select among the loads
  // A.s[0..3] would become an indexed load, which puts the kernel arguments in scratch
  float sc[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) sc[m] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(A.s[m])));
  const float sm = o.m == 0 ? sc[0] : o.m == 1 ? sc[1] : o.m == 2 ? sc[2] : sc[3];
  float* a = S.acc + ((int64_t)(o.m * A.M + o.j) * S.N + S.row0 + ti * RG + o.r);
  float before = 0.f;
  if (o.wr) before = __hip_atomic_fetch_add(a, o.y * sm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // a zero the compiler cannot see through, computed from the returned sums
  uint32_t z;
  asm volatile("v_and_b32 %0, 0, %1" : "=v"(z) : "v"(before));
  uint32_t old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(S.cnt + ti, 1u + z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __builtin_amdgcn_readfirstlane(old);
  if (old + 1 == (uint32_t)S.parts) {
    const float t = o.wr ? __hip_atomic_exchange(a, 0.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
    const float val[4] = {t, t, t, t};
    task_store<MT, RG>(A, S, ti, o, val);
    if (lane == 0) __hip_atomic_exchange(S.cnt + ti, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
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

// ------------------------------------------------------------------ segment walk

template <int MT, int RG, int NSEG, class L, bool SPLIT>
struct SegRunner {
  static constexpr int CHUNK = NSEG * QSEG;
  const char* lds;
  LaneOff lo;
  const QuadRowsArgs& A;
  const SegCtx& S;
  int lane, nck, ntask;
  uint32_t voff[RG];
  float acc[RG][4][MT];    // the task being decoded
  float pend[RG][4][MT];   // the previous task, finished one step late
  int pend_ti;             // its index, -1 when none
  PlugSt<MT> P;            // plug entries of the pending task (then of the current one)
  int64_t pc;
  Cursor lc;               // next chunk to load
  float parked;            // S.park: the last task's reduced (unscaled) sum of this lane

  __device__ __forceinline__ SegRunner(const char* l, const QuadRowsArgs& a, const SegCtx& s, int64_t plug_lo)
      : lds(l), A(a), S(s), pend_ti(-1), pc(plug_lo), parked(0.f) {
    lane = threadIdx.x & 63;
    lo = L::lane(lane);
    nck = (S.kend - S.kbeg + CHUNK - 1) / CHUNK;
    ntask = (S.nrows + RG - 1) / RG;
    lc = {0, 0};
#pragma unroll
    for (int r = 0; r < RG; ++r) voff[r] = 4u * (uint32_t)(r * S.ldc) + 16u * lane;
    zero_acc<MT, RG>(acc);
  }

  __device__ __forceinline__ void advance(Cursor& c) const {
    if (++c.ck == nck) {
      c.ck = 0;
      ++c.ti;
    }
  }

  // Issue the next chunk's loads (past the last chunk: reload the last one, so every
  // step issues the same loads).
  __device__ __forceinline__ void prefetch(Chunk<MT, RG, NSEG>& c) {
    chunk_issue<MT, RG, NSEG>(S, lc.ti * RG, S.kbeg + lc.ck * CHUNK, voff, lane, c);
    Cursor nx = lc;
    advance(nx);
    if (nx.ti < ntask) lc = nx;
  }

  // Finish the pending task: plug corrections, wave reduction, stores.
  __device__ __forceinline__ void finish_pending() {
    plug_end<MT, RG, L>(lds, lo, A, S, pend_ti, lane, pc, P, pend);
    if constexpr (SPLIT) {
      if (S.park) parked = task_reduce<MT, RG>(A, S, pend_ti, lane, pend).y;
      else if (S.parts > 1) task_accumulate<MT, RG>(A, S, pend_ti, lane, pend);
      else task_write<MT, RG>(A, S, pend_ti, lane, pend);
    } else {
      task_write<MT, RG>(A, S, pend_ti, lane, pend);
    }
    pend_ti = -1;
  }

  // One step.  Memory operations are placed so that each is consumed at least one
  // step after it was issued, and every conditional one right after the prefetch:
  //   prefetch the next chunk | [first chunk of a task] finish the previous task (its
  //   plug loads arrived during the previous step; its stores) and issue this task's
  //   plug loads | decode the current chunk | [last chunk] park the sums for the next step.
  // The compiler waits for each register before its first use; since nothing is used
  // in the step that loaded it, no wait has to cover the prefetch just issued.
  __device__ __forceinline__ bool step(Cursor& cur, Chunk<MT, RG, NSEG>& comp, Chunk<MT, RG, NSEG>& pref) {
    prefetch(pref);
    if (cur.ck == 0) {
      if (pend_ti >= 0) finish_pending();
      plug_begin<MT, RG>(A, S, cur.ti, lane, pc, P);
    }
    chunk_compute<MT, RG, NSEG, L>(lds, lo, comp, acc);
    if (cur.ck == nck - 1) {
#pragma unroll
      for (int r = 0; r < RG; ++r)
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int j = 0; j < MT; ++j) pend[r][m][j] = acc[r][m][j];
      zero_acc<MT, RG>(acc);
      pend_ti = cur.ti;
    }
    advance(cur);
    return cur.ti < ntask;
  }

  __device__ __forceinline__ void run() {
    if (ntask <= 0 || S.kend <= S.kbeg) return;
    Chunk<MT, RG, NSEG> c0, c1;
    Cursor cur = {0, 0};
    vload32(P.idx, 4u * lane, plug_idx_rsrc(A, pc));
    prefetch(c0);
    for (;;) {
      if (!step(cur, c0, c1)) break;
      if (!step(cur, c1, c0)) break;
    }
    finish_pending();
  }

  // Chunk ck of the wave's only task into c (past the last chunk: the last chunk's
  // addresses, nothing read).
  __device__ __forceinline__ void issue_one(Chunk<MT, RG, NSEG>& c, int ck) const {
    chunk_issue<MT, RG, NSEG>(S, 0, S.kbeg + min(ck, nck - 1) * CHUNK, voff, lane, c, ck < nck);
  }

  // A wave with one task (one-Linear launches with no more tasks per column slice than
  // waves): the caller issued chunks 0 and 1 into c0, c1 and the plug positions (idx)
  // before the table build; three buffers deep, so two chunks are in flight while one is
  // decoded (no pending task, whose sums would take the third buffer's registers).
  __device__ __forceinline__ void run_one(Chunk<MT, RG, NSEG>& c0, Chunk<MT, RG, NSEG>& c1, uint32_t idx) {
    Chunk<MT, RG, NSEG> c2;
    P.idx = idx;
    plug_begin<MT, RG>(A, S, 0, lane, pc, P);
    // whole rounds of three chunks with no exit between them (an exit inside the round
    // makes the compiler wait for both chunks in flight at the round's first decode), then
    // the 0-2 chunks left, already in c0 and c1
    int ck = 0;
    for (; ck + 3 <= nck; ck += 3) {
      issue_one(c2, ck + 2);
      chunk_compute<MT, RG, NSEG, L>(lds, lo, c0, acc);
      issue_one(c0, ck + 3);
      chunk_compute<MT, RG, NSEG, L>(lds, lo, c1, acc);
      issue_one(c1, ck + 4);
      chunk_compute<MT, RG, NSEG, L>(lds, lo, c2, acc);
    }
    if (ck < nck) {
      chunk_compute<MT, RG, NSEG, L>(lds, lo, c0, acc);
      if (ck + 1 < nck) chunk_compute<MT, RG, NSEG, L>(lds, lo, c1, acc);
    }
    plug_end<MT, RG, L>(lds, lo, A, S, 0, lane, pc, P, acc);
    if constexpr (SPLIT) {
      if (S.park) parked = task_reduce<MT, RG>(A, S, 0, lane, acc).y;
      else if (S.parts > 1) task_accumulate<MT, RG>(A, S, 0, lane, acc);
      else task_write<MT, RG>(A, S, 0, lane, acc);
    } else {
      task_write<MT, RG>(A, S, 0, lane, acc);
    }
  }

  // The same walk when the caller has already issued the first chunk into c0 (with this
  // runner's lane offsets): the first task's plug positions are requested, then the loop.
  __device__ __forceinline__ void run_issued(Chunk<MT, RG, NSEG>& c0) {
    Chunk<MT, RG, NSEG> c1;
    Cursor cur = {0, 0};
    vload32(P.idx, 4u * lane, plug_idx_rsrc(A, pc));
    Cursor nx = lc;                    // the load cursor past the first chunk, as prefetch(c0) leaves it
    advance(nx);
    if (nx.ti < ntask) lc = nx;
    for (;;) {
      if (!step(cur, c0, c1)) break;
      if (!step(cur, c1, c0)) break;
    }
    finish_pending();
  }
};

// Segment context of rows [row0, row1) of projection P.  Every field goes through
// readfirstlane: the descriptors are read from memory the kernel also writes, so the
// compiler cannot prove them uniform, and a buffer resource in vector registers would
// turn each load into a loop over lanes.
__device__ __forceinline__ void seg_ctx(const pp_quad_proj& P, int64_t o_sn, int row0, int row1, int M, SegCtx& S) {
  const int ldc = uniform((int)P.ldc), K = uniform(P.K);
  row0 = uniform(row0);
  row1 = uniform(row1);
  S.ldc = ldc;
  S.K = K;
  S.nrows = row1 - row0;
  S.row0 = row0;
  S.x_sm = uniform((int)P.x_sm);
  S.pos0 = uniform64(P.pos0) + (int64_t)row0 * ldc;
  const uint32_t cbytes = S.nrows > 0 ? 4u * (uint32_t)((S.nrows - 1) * ldc + K) : 0u;
  S.codes = uniform_ptr(P.codes) + (int64_t)row0 * ldc;
  S.x = reinterpret_cast<const f16*>(uniform_ptr(P.x));
  S.rc = make_rsrc(S.codes, cbytes);
  S.rx = make_rsrc(S.x, 2u * (uint32_t)((M - 1) * S.x_sm + K));
#pragma unroll
  for (int m = 0; m < 4; ++m) S.out[m] = reinterpret_cast<f16*>(uniform_ptr(P.out[m])) + (int64_t)row0 * o_sn;
  S.o_sm = uniform64(P.o_sm);
  S.o_sn = o_sn;
  S.kbeg = 0;
  S.kend = K;
  S.parts = 1;
  S.N = uniform(P.N);
  S.acc = nullptr;
  S.cnt = nullptr;
  S.park = false;
}

// Wave gw of the launch; [s0, s1) its segments (stream front end).
template <int MT, class L, bool SPLIT>
__device__ __forceinline__ void rows_body(const char* lds, const QuadRowsArgs& A, int64_t gw, int64_t s0, int64_t s1) {
  constexpr int RG = RowsCfg<MT>::RG, NSEG = RowsCfg<MT>::NSEG;
  for (int64_t si = s0; si < s1; ++si) {
    const pp_quad_seg g = A.segs[si];
    SegCtx S;
    seg_ctx(A.projs[uniform(g.proj)], 1, g.row0, g.row1, A.M, S);
    const int parts = uniform(g.parts);
    if (parts > 1) {
      if (!SPLIT) continue;   // split segments run in the kernel that has the workspace
      // one column slice of its rows (clamped to the projection)
      S.kbeg = max(0, min(S.K, uniform(g.k0)));
      S.kend = max(S.kbeg, min(S.K, uniform(g.k1)));
      S.parts = parts;
      S.acc = reinterpret_cast<float*>(A.ws) + uniform64(g.acc_off);
      S.cnt = reinterpret_cast<uint32_t*>(A.ws) + uniform(g.task0);
    }
    SegRunner<MT, RG, NSEG, L, SPLIT> R(lds, A, S, uniform64(g.plug_lo));
    R.run();
  }
}

// The one-Linear front end.  Its first chunk needs no descriptor, so the wave issues it
// before the table build and the round trip to HBM runs under the build: first the plug
// start of its first row (so that waiting for it waits for nothing else), then the LUT
// loads, then the first chunk; the build waits for the LUT values only.
// PARTS: 0 whole rows; 1 column slices meeting through the workspace; 2 a task's slices are
// consecutive waves of one workgroup (wg_item): each keeps its reduced sums, and after every
// wave of the workgroup is done with the tables (a barrier) they go into the table memory,
// where after a second barrier the slice-0 wave adds them and writes the outputs.
// ONE: every wave has at most one task (SegRunner::run_one): its first two chunks and its
// plug positions are requested before the build.
template <int MT, typename E, int PARTS, bool ONE>
__device__ __forceinline__ void direct_body(uint32_t* T, const QuadRowsArgs& A, int64_t gw) {
  constexpr int RG = RowsCfg<MT>::RG, NSEG = RowsCfg<MT>::NSEG, NT = RowsCfg<MT>::NT, WAVES = NT / 64;
  constexpr bool SPLIT = PARTS != 0, WG = PARTS == 2;
  const int lane = threadIdx.x & 63;
  const int64_t W = (int64_t)gridDim.x * WAVES;
  u32x2 wp = {0u, 0u};
  if (A.wave_plug != nullptr) vload64(wp, 8u * (uint32_t)gw, make_rsrc(A.wave_plug, 8u * (uint32_t)(W + 1)));
  QuadTableBuild<NT, E> tb;
  tb.load(A.luts);
  const int K = uniform(A.proj.K), N = uniform(A.proj.N);
  const uint32_t parts = (uint32_t)uniform(A.parts);
  const int wave = (int)(gw - (int64_t)blockIdx.x * WAVES);
  const DirectItem d = WG ? wg_item<WAVES>(blockIdx.x, gridDim.x, (uint32_t)wave, (uint32_t)uniform64(A.n_tasks), parts,
                                           (uint32_t)uniform(A.n_chunks), NSEG * QSEG, (uint32_t)K)
                          : direct_item<WAVES>((uint32_t)gw, (uint32_t)W, (uint32_t)uniform64(A.n_tasks), parts,
                                               (uint32_t)uniform(A.n_chunks), NSEG * QSEG, (uint32_t)K);
  SegCtx S;
  seg_ctx(A.proj, A.o_sn, min(d.t0 * RG, N), min(d.t1 * RG, N), A.M, S);
  S.kbeg = uniform(d.kbeg);
  S.kend = uniform(d.kend);
  if (SPLIT && parts > 1) {
    S.parts = (int)parts;
    if (WG) {
      S.park = true;
    } else {
      S.acc = uniform_ptr(A.acc);
      S.cnt = uniform_ptr(A.cnt) + d.t0;
    }
  }
  const bool busy = S.nrows > 0 && S.kend > S.kbeg;
  uint32_t voff[RG];
#pragma unroll
  for (int r = 0; r < RG; ++r) voff[r] = 4u * (uint32_t)(r * S.ldc) + 16u * lane;
  Chunk<MT, RG, NSEG> c0, c1;
  if (busy) chunk_issue<MT, RG, NSEG>(S, 0, S.kbeg, voff, lane, c0);   // 1 us faster than after the build
  // the caller's plan, kept inside the table whatever it holds (a stale plan must not send
  // the plug loads outside it)
  const int64_t pc = std::min<int64_t>(std::max<int64_t>(uniform64((int64_t)(((uint64_t)wp[1] << 32) | wp[0])), 0),
                                       A.plug_n);
  uint32_t idx0 = 0;
  if (ONE && busy) vload32(idx0, 4u * lane, plug_idx_rsrc(A, pc));
  const bool same = tb.same();
  if (ONE && busy) {
    // the second chunk once the first LUT values are back (issued with the first, gate
    // 11008x2048 built its tables 4.9 us after entry; 4.7 this way, both 25.1-26.2 us)
    const int k1 = S.kbeg + NSEG * QSEG;
    chunk_issue<MT, RG, NSEG>(S, 0, k1 < S.kend ? k1 : S.kbeg, voff, lane, c1, k1 < S.kend);
  }
  const bool shared = tb.finish(T, A.luts, same);
  if (!WG && !busy) return;
  const char* lds = reinterpret_cast<const char*>(T);
  float y = 0.f;
  if (busy) {
    if (shared) {
      SegRunner<MT, RG, NSEG, LayShared, SPLIT> R(lds, A, S, pc);
      if constexpr (ONE) R.run_one(c0, c1, idx0);
      else R.run_issued(c0);
      y = R.parked;
    } else {
      SegRunner<MT, RG, NSEG, LaySplit, SPLIT> R(lds, A, S, pc);
      if constexpr (ONE) R.run_one(c0, c1, idx0);
      else R.run_issued(c0);
      y = R.parked;
    }
  }
  if constexpr (WG) {
    float* red = reinterpret_cast<float*>(T);
    __syncthreads();   // every wave of the workgroup is done with the tables
    red[64 * wave + lane] = y;
    __syncthreads();
    if (busy && wave % (int)parts == 0) {
      Reduced<MT, RG> o = task_slot<MT, RG>(A, S, 0, lane);
      float t = 0.f;
      for (int p = 0; p < (int)parts; ++p) t += red[64 * (wave + p) + lane];
      const float val[4] = {t * A.s[0], t * A.s[1], t * A.s[2], t * A.s[3]};
      task_store<MT, RG>(A, S, 0, o, val);
    }
  }
}

// The whole-stream launch (segments from the planner's tables).
template <int MT, bool SPLIT>
__global__ __launch_bounds__(RowsCfg<MT>::NT) void quad_rows_kernel(const QuadRowsArgs A) {
  __shared__ __attribute__((aligned(16))) uint32_t T[QLDS_BYTES / 4];
  const char* lds = reinterpret_cast<const char*>(T);
  const int64_t gw = (int64_t)blockIdx.x * (RowsCfg<MT>::NT / 64) + uniform(threadIdx.x >> 6);
  SegRange sr;
  sr.issue(A.seg_bounds, gw, (int64_t)gridDim.x * (RowsCfg<MT>::NT / 64));
  if (quad_tables<RowsCfg<MT>::NT>(T, A.luts)) rows_body<MT, LayShared, SPLIT>(lds, A, gw, sr.lo(), sr.hi());
  else rows_body<MT, LaySplit, SPLIT>(lds, A, gw, sr.lo(), sr.hi());
}

// One Linear (segs == nullptr): a kernel of its own, so that the whole-stream kernel keeps
// its register allocation.  PARTS as direct_body.
template <int MT, int PARTS, bool ONE = false>
__global__ __launch_bounds__(RowsCfg<MT>::NT) void quad_direct_kernel(const QuadRowsArgs A) {
  __shared__ __attribute__((aligned(16))) uint32_t T[QLDS_BYTES / 4];
  const int64_t gw = (int64_t)blockIdx.x * (RowsCfg<MT>::NT / 64) + uniform(threadIdx.x >> 6);
  if (A.luts.dtype == PP_F16) direct_body<MT, f16, PARTS, ONE>(T, A, gw);
  else direct_body<MT, float, PARTS, ONE>(T, A, gw);
}

// ------------------------------------------------------------------ tail rows
struct QuadTailArgs {
  const pp_quad_proj* projs;
  const pp_quad_item* items;
  int64_t n_items;
  QuadLuts luts;
  float s[4];
  const uint32_t* plug_idx;
  const f16* plug_vals;
  int M;
  int64_t n_codes;  // positions >= n_codes come from the tails
  const f16* tails[4];
  int64_t tail_len[4];
};

// A row that reaches FP16 tail positions, element by element:
// y_m = s_m * sum_{pos < n} x * decoded_m  +  sum_{n <= pos} x * tail_m[pos - n].
template <int MT>
__global__ __launch_bounds__(256) void quad_tail_kernel(const QuadTailArgs A) {
  __shared__ QuadLds<1, 1> T;
  quad_build_lds(T, A.luts);
  __syncthreads();
  const int64_t ti = (int64_t)blockIdx.x * 4 + uniform(threadIdx.x >> 6);
  if (ti >= A.n_items) return;
  const int lane = threadIdx.x & 63;
  const pp_quad_item it = A.items[ti];
  const pp_quad_proj& P = A.projs[it.proj];
  const int K = P.K;
  const int64_t pos_row = P.pos0 + (int64_t)it.row0 * P.ldc;
  const uint32_t* codes = P.codes + (int64_t)it.row0 * P.ldc;
  const f16* x = reinterpret_cast<const f16*>(P.x);
  float accc[4][MT], acct[4][MT];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int j = 0; j < MT; ++j) accc[m][j] = acct[m][j] = 0.f;
  for (int k = lane; k < K; k += 64) {
    const int64_t pos = pos_row + k;
    float xk[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) xk[j] = j < A.M ? (float)x[(int64_t)j * P.x_sm + k] : 0.f;
    if (pos < A.n_codes) {
      float w[4];
      quad_decode(T, codes[k], 0, 0, w[0], w[1], w[2], w[3]);
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int j = 0; j < MT; ++j) accc[m][j] = fmaf(w[m], xk[j], accc[m][j]);
    } else {
      const int64_t t = pos - A.n_codes;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (t < A.tail_len[m]) {
          const float w = (float)A.tails[m][t];
#pragma unroll
          for (int j = 0; j < MT; ++j) acct[m][j] = fmaf(w, xk[j], acct[m][j]);
        }
      }
    }
  }
  for (int64_t p0 = it.plug_lo; p0 < it.plug_hi; p0 += 64) {
    const int64_t p = p0 + lane;
    if (p >= it.plug_hi) continue;
    const int64_t k = (int64_t)A.plug_idx[p] - pos_row;
    if (k < 0 || k >= K || pos_row + k >= A.n_codes) continue;
    float wd[4];
    quad_decode(T, codes[k], 0, 0, wd[0], wd[1], wd[2], wd[3]);
    const f16x4 pv = *reinterpret_cast<const f16x4*>(A.plug_vals + 4 * p);
    const float dlt[4] = {(float)pv.x - wd[0], (float)pv.y - wd[1], (float)pv.z - wd[2], (float)pv.w - wd[3]};
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      if (j >= A.M) break;
      const float xk = (float)x[(int64_t)j * P.x_sm + k];
#pragma unroll
      for (int m = 0; m < 4; ++m) accc[m][j] = fmaf(xk, dlt[m], accc[m][j]);
    }
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    // a model whose stream ends before this row does not have the row: it reads 0
    const bool has = pos_row < A.n_codes || pos_row - A.n_codes < A.tail_len[m];
    f16* o = reinterpret_cast<f16*>(P.out[m]) + it.row0;
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const float v = wave_sum(accc[m][j]) * A.s[m] + wave_sum(acct[m][j]);
      if (lane == 0 && j < A.M) o[(int64_t)j * P.o_sm] = (f16)(has ? v : 0.f);
    }
  }
}

// Plug start of each wave's first row (one-Linear front end): the first entry with
// idx >= pos0 + row*ldc, row the first row of direct_item(g); entry n_waves: the end of the
// rows.  One thread per wave, a binary search over the ascending positions.
template <int G>
__global__ void wave_plug_kernel(const uint32_t* plug_idx, int64_t plug_n, int64_t pos0, int64_t ldc,
                                 int rows_per_task, int64_t n_tasks, int parts, int n_chunks, int chunk, int K,
                                 int64_t n_waves, int N, int wg, int64_t* wave_plug) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g > n_waves) return;
  int64_t row = N;
  if (g < n_waves) {
    const DirectItem d = wg ? wg_item<G>((uint32_t)(g / G), (uint32_t)(n_waves / G), (uint32_t)(g % G),
                                         (uint32_t)n_tasks, (uint32_t)parts, (uint32_t)n_chunks, (uint32_t)chunk,
                                         (uint32_t)K)
                            : direct_item<G>((uint32_t)g, (uint32_t)n_waves, (uint32_t)n_tasks, (uint32_t)parts,
                                             (uint32_t)n_chunks, (uint32_t)chunk, (uint32_t)K);
    row = std::min<int64_t>((int64_t)d.t0 * rows_per_task, N);
  }
  const int64_t key = pos0 + row * ldc;
  int64_t lo = 0, hi = plug_n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)plug_idx[mid] < key) lo = mid + 1;
    else hi = mid;
  }
  wave_plug[g] = lo;
}

// ------------------------------------------------------------------ host side
static int round_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

static int cfg_rg(int mt) {
  switch (mt) {
    case 1: return RowsCfg<1>::RG;
    case 2: return RowsCfg<2>::RG;
    case 4: return RowsCfg<4>::RG;
    default: return RowsCfg<8>::RG;
  }
}
static int cfg_waves(int mt) {
  switch (mt) {
    case 1: return RowsCfg<1>::NT / 64;
    case 2: return RowsCfg<2>::NT / 64;
    case 4: return RowsCfg<4>::NT / 64;
    default: return RowsCfg<8>::NT / 64;
  }
}

template <int PARTS>
static void launch_direct_t(const QuadRowsArgs& A, int mt, hipStream_t st) {
  const unsigned grid = (unsigned)device_cu_count();
  // at most one task per wave: a task per column slice per wave at most (direct_item deals
  // each slice's tasks over its >= W / parts waves; wg_item gives a wave one task)
  const int64_t W = (int64_t)grid * (RowsCfg<1>::NT / 64);
  const bool one = PARTS == 2 || A.n_tasks <= W / std::max(1, A.parts);
  switch (mt) {
    case 1:
      if (one) hipLaunchKernelGGL((quad_direct_kernel<1, PARTS, true>), dim3(grid), dim3(RowsCfg<1>::NT), 0, st, A);
      else hipLaunchKernelGGL((quad_direct_kernel<1, PARTS>), dim3(grid), dim3(RowsCfg<1>::NT), 0, st, A);
      break;
    case 2: hipLaunchKernelGGL((quad_direct_kernel<2, PARTS>), dim3(grid), dim3(RowsCfg<2>::NT), 0, st, A); break;
    case 4: hipLaunchKernelGGL((quad_direct_kernel<4, PARTS>), dim3(grid), dim3(RowsCfg<4>::NT), 0, st, A); break;
    default: hipLaunchKernelGGL((quad_direct_kernel<8, PARTS>), dim3(grid), dim3(RowsCfg<8>::NT), 0, st, A); break;
  }
}

template <bool SPLIT>
static void launch_rows_t(const QuadRowsArgs& A, int mt, hipStream_t st) {
  const unsigned grid = (unsigned)device_cu_count();
  if (A.segs == nullptr) {
    if (SPLIT && A.wg_parts) launch_direct_t<2>(A, mt, st);
    else launch_direct_t<SPLIT ? 1 : 0>(A, mt, st);
    return;
  }
  switch (mt) {
    case 1: hipLaunchKernelGGL((quad_rows_kernel<1, SPLIT>), dim3(grid), dim3(RowsCfg<1>::NT), 0, st, A); break;
    case 2: hipLaunchKernelGGL((quad_rows_kernel<2, SPLIT>), dim3(grid), dim3(RowsCfg<2>::NT), 0, st, A); break;
    case 4: hipLaunchKernelGGL((quad_rows_kernel<4, SPLIT>), dim3(grid), dim3(RowsCfg<4>::NT), 0, st, A); break;
    default: hipLaunchKernelGGL((quad_rows_kernel<8, SPLIT>), dim3(grid), dim3(RowsCfg<8>::NT), 0, st, A); break;
  }
}

// The stream launch with a workspace, and a one-Linear launch cut into column slices, run
// the kernel that also takes split segments.
static int launch_rows(const QuadRowsArgs& A, int mt, hipStream_t st) {
  if (A.segs != nullptr ? A.ws != nullptr : A.parts > 1) launch_rows_t<true>(A, mt, st);
  else launch_rows_t<false>(A, mt, st);
  PP_LAUNCH_CHECK();
  return PP_OK;
}

static QuadLuts make_luts(const void* const* luts, int dtype) {
  QuadLuts L;
  for (int i = 0; i < 7; ++i) L.p[i] = luts[i];
  L.dtype = dtype;
  return L;
}

bool quad_rows_ok(const void* a, int64_t a_sm, int64_t a_sk, const uint32_t* codes, int64_t c_sk, int64_t c_sn,
                  int64_t M, int64_t N, int64_t K) {
  // buffer offsets are 32-bit: a projection's codes and activations must stay below 2 GiB
  return c_sk == 1 && c_sn % 4 == 0 && c_sn >= K && K % 4 == 0 && K > 0 && aligned(codes, 16) && M >= 1 &&
         M <= 8 && (a_sk == 1 || K == 1) && (M == 1 || (a_sm % 4 == 0 && a_sm >= K)) && aligned(a, 8) &&
         N * c_sn < (1ll << 29) && (M - 1) * a_sm + K < (1ll << 30);
}

static int cfg_chunk(int mt) {
  switch (mt) {
    case 1: return RowsCfg<1>::NSEG * QSEG;
    case 2: return RowsCfg<2>::NSEG * QSEG;
    case 4: return RowsCfg<4>::NSEG * QSEG;
    default: return RowsCfg<8>::NSEG * QSEG;
  }
}

// How one Linear runs on the row kernel: T tasks of rg rows, cut into `parts` column slices
// of whole chunks when the tasks are too few for the launch's W wavefronts (direct_parts:
// gate 11008x2048 at one token, 1,376 tasks, runs whole rows; down 2048x11008 in 4 slices).
// The split workspace holds one arrival counter per task (256-byte aligned), then float32
// accumulators [4][M][N].
struct DirectPlan {
  int mt, rg, chunk, parts, n_chunks;
  bool wg;                 // the slices meet in LDS (no workspace)
  int64_t n_tasks, waves, cnt_bytes, split_bytes;
};
// Slices of a Linear with at least 4 waves per task: as many as fill the waves, a power of
// two up to a workgroup's waves so that they meet in LDS (down 2048x11008 at one token:
// 8 slices of 1,376 columns, 26.4 us, against 4 slices, 28.3); otherwise direct_parts.
static int quad_direct_parts(int64_t T, int64_t W, int64_t C, int waves_per_wg) {
  if (T > 0 && W >= 4 * T) {
    int p = 1;
    while (2 * p <= waves_per_wg && 2 * p * T <= W && 2 * p <= C) p *= 2;
    if (p > 1) return p;
  }
  return direct_parts(T, W, C);
}

static DirectPlan direct_plan(int64_t M, int64_t N, int64_t K, bool split) {
  DirectPlan p;
  p.mt = round_mt(M);
  p.rg = cfg_rg(p.mt);
  p.chunk = cfg_chunk(p.mt);
  p.waves = (int64_t)device_cu_count() * cfg_waves(p.mt);
  p.n_tasks = (N + p.rg - 1) / p.rg;
  p.n_chunks = (int)std::max<int64_t>(1, (K + p.chunk - 1) / p.chunk);
  p.parts = split ? quad_direct_parts(p.n_tasks, p.waves, p.n_chunks, cfg_waves(p.mt)) : 1;
  p.wg = wg_parts_ok(p.n_tasks, p.waves, p.parts, cfg_waves(p.mt));
  p.cnt_bytes = p.parts > 1 && !p.wg ? (p.n_tasks * 4 + 255) / 256 * 256 : 0;
  p.split_bytes = p.parts > 1 && !p.wg ? p.cnt_bytes + 4 * 4 * M * N : 0;
  return p;
}

static void direct_args(QuadRowsArgs& A, const DirectPlan& p, const void* a, int64_t a_sm, const uint32_t* codes,
                        int64_t ldc, const void* const* luts, int lut_dtype, const float* scales,
                        const uint32_t* plug_idx, const void* plug_vals, const uint32_t* plug_code, int64_t plug_n,
                        int64_t elem_base, void* const* out, int64_t o_sm, int64_t o_sn, int64_t M, int64_t N,
                        int64_t K) {
  A.proj.codes = codes;
  A.proj.ldc = ldc;
  A.proj.pos0 = elem_base;
  A.proj.x = a;
  A.proj.x_sm = M > 1 ? a_sm : K;
  for (int m = 0; m < 4; ++m) A.proj.out[m] = out[m];
  A.proj.o_sm = o_sm;
  A.proj.N = (int32_t)N;
  A.proj.K = (int32_t)K;
  A.o_sn = o_sn;
  A.n_tasks = p.n_tasks;
  A.parts = p.parts;
  A.n_chunks = p.n_chunks;
  A.wg_parts = p.wg ? 1 : 0;
  A.luts = make_luts(luts, lut_dtype);
  for (int m = 0; m < 4; ++m) A.s[m] = scales[m];
  A.plug_idx = plug_idx;
  A.plug_vals = reinterpret_cast<const f16*>(plug_vals);
  A.plug_code = plug_code;
  A.plug_n = plug_n;
  A.M = (int)M;
}

static int launch_wave_plug(const DirectPlan& p, const uint32_t* plug_idx, int64_t plug_n, int64_t elem_base,
                            int64_t ldc, int64_t N, int64_t K, int64_t* wave_plug, hipStream_t st) {
  static_assert(RowsCfg<1>::NT == RowsCfg<2>::NT && RowsCfg<1>::NT == RowsCfg<4>::NT && RowsCfg<1>::NT == RowsCfg<8>::NT,
                "one workgroup size for the one-Linear launches");
  hipLaunchKernelGGL(wave_plug_kernel<RowsCfg<1>::NT / 64>, dim3((unsigned)((p.waves + 1 + 255) / 256)), dim3(256), 0,
                     st, plug_idx, plug_n, elem_base, ldc, p.rg, p.n_tasks, p.parts, p.n_chunks, p.chunk, (int)K,
                     p.waves, (int)N, p.wg ? 1 : 0, wave_plug);
  PP_LAUNCH_CHECK();
  return PP_OK;
}

int64_t quad_rows_workspace(int64_t M, int64_t N, int64_t plug_n) {
  if (plug_n <= 0) return 0;
  const int mt = round_mt(M);
  const int64_t waves = (int64_t)device_cu_count() * cfg_waves(mt);
  return ((waves + 1) * 8 + 255) / 256 * 256;
}

// pp_quad_gemm's route: whole rows (any workspace content; the plug starts are found in
// the workspace by a first launch).
int quad_rows_single(const void* a, int64_t a_sm, const uint32_t* codes, int64_t ldc, const void* const* luts,
                     int lut_dtype, const float* scales, const uint32_t* plug_idx, const void* plug_vals,
                     int64_t plug_n, int64_t elem_base, void* const* out, int64_t o_sm, int64_t o_sn, int64_t M,
                     int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, hipStream_t st) {
  const DirectPlan p = direct_plan(M, N, K, false);
  PP_REQUIRE(p.waves < (1 << 16), "the one-Linear launch deals at most 65,535 wavefronts");
  const int64_t need = quad_rows_workspace(M, N, plug_n);
  PP_REQUIRE(workspace_bytes >= need && (need == 0 || workspace != nullptr), "workspace too small: need %lld bytes",
             (long long)need);
  QuadRowsArgs A = {};
  direct_args(A, p, a, a_sm, codes, ldc, luts, lut_dtype, scales, plug_idx, plug_vals, nullptr, plug_n, elem_base,
              out, o_sm, o_sn, M, N, K);
  if (plug_n > 0) {
    int64_t* wp = reinterpret_cast<int64_t*>(workspace);
    if (int rc = launch_wave_plug(p, plug_idx, plug_n, elem_base, ldc, N, K, wp, st)) return rc;
    A.wave_plug = wp;
  }
  return launch_rows(A, p.mt, st);
}

}  // namespace pp

using namespace pp;

extern "C" int pp_quad_stream_rows(int64_t M) {
  if (M < 1 || M > 8) {
    set_error("the stream decode takes 1..8 tokens, got %lld", (long long)M);
    return 0;
  }
  return cfg_rg(round_mt(M));
}

extern "C" int pp_quad_stream_chunk(int64_t M) {
  if (M < 1 || M > 8) return 0;
  switch (round_mt(M)) {
    case 1: return RowsCfg<1>::NSEG * QSEG;
    case 2: return RowsCfg<2>::NSEG * QSEG;
    case 4: return RowsCfg<4>::NSEG * QSEG;
    default: return RowsCfg<8>::NSEG * QSEG;
  }
}

extern "C" int64_t pp_quad_stream_waves(int64_t M) {
  if (M < 1 || M > 8) return 0;
  return (int64_t)device_cu_count() * cfg_waves(round_mt(M));
}

extern "C" int64_t pp_quad_rows_plan_size(int64_t M) {
  if (M < 1 || M > 8) return 0;
  return (int64_t)device_cu_count() * cfg_waves(round_mt(M)) + 1;
}

extern "C" int64_t pp_quad_rows_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > 8 || N < 1 || K < 1) return 0;
  return direct_plan(M, N, K, true).split_bytes;
}

extern "C" int pp_quad_rows_parts(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > 8 || N < 1 || K < 1) return 0;
  return direct_plan(M, N, K, true).parts;
}

extern "C" int pp_quad_rows_plan(const uint32_t* plug_idx, int64_t plug_n, int64_t elem_base, int64_t ldc, int64_t M,
                                 int64_t N, int64_t K, int64_t* wave_plug, void* stream) {
  PP_REQUIRE(M >= 1 && M <= 8, "the row kernel takes 1..8 tokens, got %lld", (long long)M);
  PP_REQUIRE(N >= 1 && K >= 1 && ldc >= K && N < (1ll << 31) && K < (1ll << 31), "bad shape");
  PP_REQUIRE(plug_n >= 0 && (plug_n == 0 || plug_idx != nullptr) && wave_plug != nullptr, "null pointer argument");
  const DirectPlan p = direct_plan(M, N, K, true);
  PP_REQUIRE(p.waves < (1 << 16), "the one-Linear launch deals at most 65,535 wavefronts");
  return launch_wave_plug(p, plug_idx, plug_n, elem_base, ldc, N, K, wave_plug, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pp_quad_rows(const void* a, int64_t a_sm, const uint32_t* codes, int64_t ldc, const void* const* luts,
                            int lut_dtype, const float* scales, const uint32_t* plug_idx, const void* plug_vals,
                            const uint32_t* plug_code, int64_t plug_n, const int64_t* wave_plug, int64_t elem_base,
                            void* const* out, int64_t o_sm, int64_t o_sn, int64_t M, int64_t N, int64_t K,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  PP_REQUIRE(luts != nullptr && scales != nullptr && out != nullptr, "null pointer argument");
  for (int i = 0; i < 7; ++i) PP_REQUIRE(luts[i] != nullptr, "lut %d is null", i);
  for (int m = 0; m < 4; ++m) PP_REQUIRE(out[m] != nullptr, "out[%d] is null", m);
  PP_REQUIRE(lut_dtype == PP_F16 || lut_dtype == PP_F32, "bad lut_dtype");
  PP_REQUIRE(quad_rows_ok(a, a_sm, 1, codes, 1, ldc, M, N, K),
             "the row kernel needs 1..8 tokens of contiguous fp16 activations (8-byte aligned, row stride a "
             "multiple of 4) and 16-byte aligned (N,K) rows of ldc >= K words (a multiple of 4)");
  PP_REQUIRE(N < (1ll << 31) && o_sn >= 1 && (M == 1 || o_sm >= 1), "bad output strides");
  PP_REQUIRE(plug_n >= 0 && (plug_n == 0 || (plug_idx && plug_vals && wave_plug)),
             "plug entries need plug_idx, plug_vals and a wave_plug plan (pp_quad_rows_plan)");
  const DirectPlan p = direct_plan(M, N, K, true);
  PP_REQUIRE(p.waves < (1 << 16), "the one-Linear launch deals at most 65,535 wavefronts");
  PP_REQUIRE(p.split_bytes == 0 || (workspace != nullptr && workspace_bytes >= p.split_bytes),
             "workspace too small: need %lld bytes (pp_quad_rows_workspace_size), zero on entry",
             (long long)p.split_bytes);
  QuadRowsArgs A = {};
  direct_args(A, p, a, a_sm, codes, ldc, luts, lut_dtype, scales, plug_idx, plug_vals, plug_code, plug_n, elem_base,
              out, o_sm, o_sn, M, N, K);
  A.wave_plug = plug_n > 0 ? wave_plug : nullptr;
  if (p.parts > 1) {
    A.cnt = reinterpret_cast<uint32_t*>(workspace);
    A.acc = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + p.cnt_bytes);
  }
  return launch_rows(A, p.mt, reinterpret_cast<hipStream_t>(stream));
}

// Side table of the plug entries: code[j] = the code word at stream position plug_idx[j]
// (0 for an entry at or past n_codes).
__global__ __launch_bounds__(256) void quad_plug_code_kernel(const uint32_t* codes, int64_t n_codes,
                                                             const uint32_t* plug_idx, int64_t plug_n, uint32_t* code) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= plug_n) return;
  const int64_t p = plug_idx[j];
  code[j] = p < n_codes ? codes[p] : 0u;
}

// row_plug[r*slices + s] = first j with plug_idx[j] >= pos0 + r*pld + s*cols, and
// row_plug[rows*slices] = first j with plug_idx[j] >= pos0 + rows*pld: one thread per key,
// a binary search over the ascending uint32 positions.
__global__ __launch_bounds__(256) void plug_search_kernel(const uint32_t* idx, int64_t n, int64_t pos0, int64_t pld,
                                                          int64_t rows, int64_t slices, int64_t cols,
                                                          int64_t* row_plug) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nk = rows * slices;
  if (i > nk) return;
  const int64_t key = i == nk ? pos0 + rows * pld : pos0 + (i / slices) * pld + (i % slices) * cols;
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if ((int64_t)idx[mid] < key) lo = mid + 1;
    else hi = mid;
  }
  row_plug[i] = lo;
}

extern "C" int pp_plug_search(const uint32_t* plug_idx, int64_t plug_n, int64_t pos0, int64_t pld, int64_t rows,
                              int64_t slices, int64_t cols, int64_t* row_plug, void* stream) {
  PP_REQUIRE(plug_n >= 0 && rows >= 0 && slices >= 1 && cols >= 0 && pld >= 0 && pos0 >= 0,
             "bad sizes (plug_n=%lld rows=%lld slices=%lld)", (long long)plug_n, (long long)rows,
             (long long)slices);
  PP_REQUIRE(row_plug != nullptr && (plug_n == 0 || plug_idx != nullptr), "null pointer");
  PP_REQUIRE(rows * slices < (1ll << 40), "too many keys");
  const int64_t keys = rows * slices + 1;
  hipLaunchKernelGGL(plug_search_kernel, dim3((unsigned)((keys + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), plug_idx, plug_n, pos0, pld, rows, slices, cols,
                     row_plug);
  PP_LAUNCH_CHECK();
  return PP_OK;
}

extern "C" int pp_quad_plug_codes(const uint32_t* codes, int64_t n_codes, const uint32_t* plug_idx, int64_t plug_n,
                                  uint32_t* code, void* stream) {
  PP_REQUIRE(plug_n >= 0 && plug_n < (1ll << 31), "plug_n out of range");
  if (plug_n == 0) return PP_OK;
  PP_REQUIRE(codes != nullptr && plug_idx != nullptr && code != nullptr && n_codes >= 0, "null pointer or bad n_codes");
  hipLaunchKernelGGL(quad_plug_code_kernel, dim3((unsigned)((plug_n + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), codes, n_codes, plug_idx, plug_n, code);
  PP_LAUNCH_CHECK();
  return PP_OK;
}

extern "C" int pp_quad_stream(const pp_quad_proj* projs, int64_t n_projs, const pp_quad_seg* segs, int64_t n_segs,
                              const int64_t* seg_bounds, int64_t n_waves, void* workspace,
                              const pp_quad_item* tail_items,
                              int64_t n_tail, const float* const* luts, const float* scales,
                              const uint32_t* plug_idx, const void* plug_vals, const uint32_t* plug_code,
                              int64_t plug_n, int64_t n_codes, const void* const* tails, const int64_t* tail_len,
                              int64_t M, void* stream) {
  PP_REQUIRE(projs != nullptr && n_projs >= 1, "no projections");
  PP_REQUIRE(n_segs >= 0 && (n_segs == 0 || (segs != nullptr && seg_bounds != nullptr)), "segs / seg_bounds is null");
  PP_REQUIRE(n_tail == 0 || tail_items != nullptr, "tail_items is null");
  PP_REQUIRE(luts != nullptr, "luts is null");
  for (int i = 0; i < 7; ++i) PP_REQUIRE(luts[i] != nullptr, "lut %d is null", i);
  PP_REQUIRE(scales != nullptr, "scales is null");
  PP_REQUIRE(plug_n >= 0 && (plug_n == 0 || (plug_idx != nullptr && plug_vals != nullptr)), "plug arrays are null");
  PP_REQUIRE(M >= 1 && M <= 8, "the stream decode takes 1..8 tokens, got %lld", (long long)M);
  PP_REQUIRE(n_segs == 0 || n_waves == pp_quad_stream_waves(M),
             "seg_bounds were built for %lld waves, this device launches %lld", (long long)n_waves,
             (long long)pp_quad_stream_waves(M));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int mt = round_mt(M);
  const QuadLuts L = make_luts(reinterpret_cast<const void* const*>(luts), PP_F32);
  if (n_segs > 0) {
    QuadRowsArgs A = {};
    A.projs = projs;
    A.segs = segs;
    A.seg_bounds = seg_bounds;
    A.luts = L;
    for (int m = 0; m < 4; ++m) A.s[m] = scales[m];
    A.plug_idx = plug_idx;
    A.plug_vals = reinterpret_cast<const f16*>(plug_vals);
    A.plug_code = plug_code;
    A.plug_n = plug_n;
    A.M = (int)M;
    A.ws = workspace;
    if (int rc = launch_rows(A, mt, st)) return rc;
  }
  if (n_tail > 0) {
    QuadTailArgs T = {};
    T.projs = projs;
    T.items = tail_items;
    T.n_items = n_tail;
    T.luts = L;
    for (int m = 0; m < 4; ++m) T.s[m] = scales[m];
    T.plug_idx = plug_idx;
    T.plug_vals = reinterpret_cast<const f16*>(plug_vals);
    T.M = (int)M;
    T.n_codes = n_codes;
    for (int m = 0; m < 4; ++m) {
      T.tails[m] = tails ? reinterpret_cast<const f16*>(tails[m]) : nullptr;
      T.tail_len[m] = tail_len ? tail_len[m] : 0;
    }
    const unsigned grid = (unsigned)((n_tail + 3) / 4);
    switch (mt) {
      case 1: hipLaunchKernelGGL(quad_tail_kernel<1>, dim3(grid), dim3(256), 0, st, T); break;
      case 2: hipLaunchKernelGGL(quad_tail_kernel<2>, dim3(grid), dim3(256), 0, st, T); break;
      case 4: hipLaunchKernelGGL(quad_tail_kernel<4>, dim3(grid), dim3(256), 0, st, T); break;
      default: hipLaunchKernelGGL(quad_tail_kernel<8>, dim3(grid), dim3(256), 0, st, T); break;
    }
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
}
