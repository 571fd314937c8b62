// Fused dual-pack decode GEMV (batch <= 4) over a whole .dualpack stream: every
// projection of a decode step in one launch (pp_dual_stream).
//
// One 16-bit code per pair of weights: (amp_q << 10) | phase (polar_bitpack.py:130),
// stored big-endian in the file (polar_bitpack.py:81-85) or as native int16 = code - 32768
// (polar_kernels.py:9-11).  Decode (polar_bitpack.py:228-247):
//   amp = amp_lut[amp_q] * scale[group(pos)],  w1 = amp cos_lut[phase],  w2 = amp sin_lut[phase],
// with group(pos) = (pos / chunk) * ceil(chunk / gs) + (pos % chunk) / gs (groups restart
// every chunk, polar_bitpack.py:201-203); plug entries replace amp by an exact fp16
// amplitude (polar_bitpack.py:240-243).
//
// Same structure as quad_rows.hip: one workgroup per CU, wavefronts walk segments (runs of
// full rows of one projection) in tasks of RG rows and chunks of 512 pairs, the next chunk
// (at one token the next two) in flight while one is decoded, reduction / stores of a task
// done in the first step of the next.  Plug corrections go through a three-stage window
// pipeline (below).  Per lane and row a chunk is one 16-byte load (8 pairs that share one
// group scale, so the scale multiplies a per-lane partial sum once per 8 pairs) and one
// 2-byte scale load; with the scale table (SM = 2, pp_dual_scale_table) one load brings
// the scales of all RG rows of the task (16 bytes at one token; measured on the 3B-shaped
// stream: 1.12 -> 1.03 ms per step, the per-row scale loads and their group arithmetic
// having cost more than the decode's table lookups).
//
// LDS tables (129 KiB, dual_lds.h): (cos, sin) of the 1024 phases in 128-byte rows of 16
// replicas, the 64 amplitudes one per bank.
#include "dual_lds.h"
#include "rows_common.h"

namespace pp {

constexpr int DPAIRS = 512;                    // pairs per wave per row per chunk (64 lanes x 8)

template <int MT> struct DualCfg;
#ifndef PP_DUAL1_RG
#define PP_DUAL1_RG 8
#endif
#ifndef PP_DUAL1_NT
#define PP_DUAL1_NT 512
#endif
template <> struct DualCfg<1> { static constexpr int RG = PP_DUAL1_RG, NT = PP_DUAL1_NT; };
template <> struct DualCfg<2> { static constexpr int RG = 4, NT = 512; };
template <> struct DualCfg<4> { static constexpr int RG = 2, NT = 512; };

struct DualStreamArgs {
  const pp_dual_proj* projs;
  const pp_quad_seg* segs;
  const int64_t* seg_bounds;
  const float* amp_lut;   // [64], float32
  const float* cos_lut;   // [1024]
  const float* sin_lut;   // [1024]
  const f16* scales;
  int64_t n_groups;
  const f16* scale_tab;       // SM = 2: the group scales regrouped per task (pp_dual_scale_table)
  int64_t n_tab;
  int64_t gs, chunk, per_chunk;
  int log2gs;
  const uint32_t* plug_idx;
  const f16* plug_amp;
  const uint32_t* plug_ent;   // per entry 2 words: column | row in its task << 19 | phase << 22;
                              // the amplitude correction (float32 bits)
  int64_t plug_n;
  const int64_t* task_plug;   // per task: first plug entry in its rows, first entry past them
  int64_t n_tasks;
  int64_t task_cap;           // > 0: plug_ent holds task_cap records per task (task t's entries
                              // from t * task_cap, null records after them) and plug_n is its
                              // length; task_plug is not read (one-Linear launch)
  int M;
  void* ws;                   // split launches: per-task counters, then float32 accumulators
  // one-Linear launch (dual_direct_kernel): the projection, its column slices and chunks,
  // the accumulators [2][M][N] and per-task counters of a sliced launch
  pp_dual_proj proj;
  int parts, n_chunks;
  float* acc;
  uint32_t* cnt;
  int wg_parts;               // 1: a task's parts are waves of one workgroup, summed in LDS
};

// (cos, sin) rows as 16-byte units (two replicas) in address order, so that a wavefront's
// stores fill consecutive banks; every LUT load of a thread is issued before its stores.
// In two steps, so that a kernel can issue other loads between the LUT loads and the stores.
template <int LAYOUT, int NT>
struct DualTableBuild {
  static constexpr int KU = (8192 + NT - 1) / NT;
  float c[KU], s[KU], amp;
  __device__ __forceinline__ void load(const DualStreamArgs& A) {
#pragma unroll
    for (int k = 0; k < KU; ++k) {
      const int u = threadIdx.x + k * NT;
      if (u < 8192) {
        c[k] = A.cos_lut[u >> 3];
        s[k] = A.sin_lut[u >> 3];
      }
    }
    // the int16 layout stores code ^ 0x8000: entry a holds amplitude a ^ 32
    if (threadIdx.x < 64) amp = A.amp_lut[LAYOUT == PP_DUAL_I16_OFFSET ? (threadIdx.x ^ 32) : threadIdx.x];
  }
  __device__ __forceinline__ void store(char* lds) const {
    if (threadIdx.x < 64) *reinterpret_cast<float*>(lds + DLDS_AMP + 4 * threadIdx.x) = amp;
#pragma unroll
    for (int k = 0; k < KU; ++k) {
      const int u = threadIdx.x + k * NT;
      if (u < 8192) *reinterpret_cast<float4*>(lds + DLDS_CS + 16 * u) = make_float4(c[k], s[k], c[k], s[k]);
    }
  }
};

template <int LAYOUT, int NT>
__device__ __forceinline__ void dual_build_lds(char* lds, const DualStreamArgs& A) {
  DualTableBuild<LAYOUT, NT> b;
  b.load(A);
  b.store(lds);
}

// Uniform state of a segment.
struct DualSeg {
  rsrc_t rx, rcs;      // activations; the segment's codes
  const uint16_t* codes;
  const f16* x;
  int64_t pos0;        // stream position of the segment's first row
  int ldc, K, nrows, x_sm;
  f16* out[2];
  int64_t o_sm;
  int kbeg, kend;      // the column slice the segment covers
  int parts, N, row0;  // slices of its rows; the projection's rows; the first row
  float* acc;          // parts > 1: the projection's accumulators [2][M][N]
  uint32_t* cnt;       // parts > 1: the counters of the segment's tasks
  float* red;          // parts meeting in LDS: the wave's 64 reduced sums
};

// Group (scale index) of stream position p.  SM = 0 and 2: chunk is a multiple of gs, so
// groups never restart mid-group and group = p / gs; SM = 1: the general rule.
template <int SM>
__device__ __forceinline__ uint32_t dual_group(const DualStreamArgs& A, int64_t p) {
  if constexpr (SM != 1) {
    return (uint32_t)(p >> A.log2gs);
  } else {
    const uint32_t pp = (uint32_t)p, ch = (uint32_t)A.chunk;
    const uint32_t c = pp / ch, rem = pp - c * ch;
    return c * (uint32_t)A.per_chunk + (rem >> A.log2gs);
  }
}

template <int MT, int RG>
struct DChunk {
  u32x4 q[RG];          // 8 pairs per lane per row
  uint32_t sc[RG];      // their group scale (fp16 bits); SM = 2: in sq
  u32x4 sq;             // SM = 2: the RG rows' scales of the lane's group, one fp16 each
  u32x4 xr[MT];         // 8 fp16 activations per lane
};

// Scale of row r of a chunk (fp16 bits in the low half).
template <int RG, int SM, int MT>
__device__ __forceinline__ uint32_t dchunk_scale(const DChunk<MT, RG>& c, int r) {
  if constexpr (SM == 2) {
    const uint32_t w = r < 2 ? c.sq.x : r < 4 ? c.sq.y : r < 6 ? c.sq.z : c.sq.w;
    return (r & 1) ? w >> 16 : w;
  } else {
    return c.sc[r];
  }
}

// live = false (a buffer filled past the wave's last chunk): every load reads nothing.
template <int MT, int RG, int SM>
__device__ __forceinline__ void dchunk_issue(const DualStreamArgs& A, const DualSeg& S, int row, int kc,
                                             const uint32_t (&voff)[RG], int lane, bool live, DChunk<MT, RG>& c) {
  const int64_t first = (int64_t)row * S.ldc + kc;
  const int64_t end = (int64_t)(S.nrows - 1) * S.ldc + S.K;
  const rsrc_t rc = make_rsrc(S.codes + first, 2u * (uint32_t)(end - first));
  const rsrc_t rs = make_rsrc(A.scales, 2u * (uint32_t)A.n_groups);
  // lanes past the row end read nothing: those codes start the next row, whose own first
  // chunk reads them (38 MB of the 3B-shaped stream's 11008-pair rows, read twice otherwise)
  const bool in_row = live && 8 * lane < S.K - kc;
#pragma unroll
  for (int r = 0; r < RG; ++r) vload128(c.q[r], in_row ? voff[r] : OOB, rc);
  const int k = kc + 8 * lane;
  const int64_t base = S.pos0 + first;   // stream position of (row, kc): uniform
  if constexpr (SM == 2) {
    // the task's RG rows start at a multiple of RG gs positions: their scales of group j
    // (columns j gs .. j gs + gs - 1 of each row) are the 2 RG bytes at entry
    // task start / gs + RG j of the table
    static_assert(RG == 8 || RG == 4 || RG == 2, "scale table cells hold 8, 4 or 2 rows");
    const int64_t t0 = (S.pos0 + (int64_t)row * S.ldc) >> A.log2gs;
    const rsrc_t rt = make_rsrc(A.scale_tab + t0, 2u * (uint32_t)(A.n_tab - t0));
    const uint32_t off = live ? 2u * RG * ((uint32_t)k >> A.log2gs) : OOB;
    if constexpr (RG == 8) {
      vload128(c.sq, off, rt);
    } else if constexpr (RG == 4) {
      u32x2 v;
      vload64(v, off, rt);
      c.sq = u32x4{v.x, v.y, 0u, 0u};
    } else {
      uint32_t v;
      vload32(v, off, rt);
      c.sq = u32x4{v, 0u, 0u, 0u};
    }
  } else {
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const bool in = live && (row + r) < S.nrows && k < S.kend;
      const int64_t br = base + (int64_t)r * S.ldc;
      uint32_t g;
      if constexpr (SM == 0) {
        // group = (br + 8 lane) / gs, split into a uniform part and a small per-lane one
        const uint32_t U = (uint32_t)(br >> A.log2gs), R = (uint32_t)br & (uint32_t)(A.gs - 1);
        g = U + ((R + 8u * lane) >> A.log2gs);
      } else {
        g = dual_group<1>(A, br + 8 * lane);
      }
      vload16(c.sc[r], in ? 2u * g : OOB, rs);
    }
  }
  if constexpr (MT == 1) {
    // columns past the slice read x = 0, so the codes loaded there add nothing
    const rsrc_t rx = make_rsrc(S.x + kc, 2u * (uint32_t)(S.kend - kc));
    vload128c(c.xr[0], live ? 16u * lane : OOB, rx);
  } else {
#pragma unroll
    for (int j = 0; j < MT; ++j)
      vload128c(c.xr[j], live && k < S.kend ? 2u * (uint32_t)(j * S.x_sm + k) : OOB, S.rx);
  }
}

template <int MT, int RG, int LAYOUT, int SM>
__device__ __forceinline__ void dchunk_compute(const char* lds, const DualLane& lo, const DChunk<MT, RG>& c,
                                               float (&acc)[RG][2][MT]) {
  float xv[MT][8];
#pragma unroll
  for (int j = 0; j < MT; ++j) {
    const f16x4 h0 = __builtin_bit_cast(f16x4, u32x2{c.xr[j].x, c.xr[j].y});
    const f16x4 h1 = __builtin_bit_cast(f16x4, u32x2{c.xr[j].z, c.xr[j].w});
    xv[j][0] = (float)h0.x; xv[j][1] = (float)h0.y; xv[j][2] = (float)h0.z; xv[j][3] = (float)h0.w;
    xv[j][4] = (float)h1.x; xv[j][5] = (float)h1.y; xv[j][6] = (float)h1.z; xv[j][7] = (float)h1.w;
  }
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const uint32_t w4[4] = {c.q[r].x, c.q[r].y, c.q[r].z, c.q[r].w};
    float an[8];
    float2 cs[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float a2[2];
      float2 c2[2];
      dual_lookup2<LAYOUT>(lds, w4[e], lo, a2, c2);
      an[2 * e] = a2[0];
      an[2 * e + 1] = a2[1];
      cs[2 * e] = c2[0];
      cs[2 * e + 1] = c2[1];
    }
    float l1[MT], l2[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) l1[j] = l2[j] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const float xa = an[e] * xv[j][e];
        l1[j] = fmaf(xa, cs[e].x, l1[j]);
        l2[j] = fmaf(xa, cs[e].y, l2[j]);
      }
    const float sc = h2f(dchunk_scale<RG, SM>(c, r));
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      acc[r][0][j] = fmaf(sc, l1[j], acc[r][0][j]);
      acc[r][1][j] = fmaf(sc, l2[j], acc[r][1][j]);
    }
  }
}

// Plug entries.  The host gives every task its plug range [tlo, thi): the entries whose
// positions lie in the task's rows, and every entry its 8-byte record plug_ent (column,
// row in its task and phase of its pair; the amplitude correction d = plug amplitude -
// amp_lut[aq] * scale, computed once per plan), so a window needs one contiguous load and
// the x gather, and no position arithmetic.  Step ck of a task takes the window of entries
// tlo + 64*PW*ck .. +64*PW (one entry per lane and window, filled from the front); a
// task with more entries than its steps can take corrects the rest when it finishes.
// A window passes through three stages, one step apart, so that every load is issued a
// step before the step that reads it and the number of loads per step is fixed:
//   step s-2: the entries' records;
//   step s-1: x at each entry's column;
//   step s:   acc[row] += d * x * (cos, sin)(phase).
// Lanes without an entry load nothing (reads of 0 make their correction 0).

// Uniform description of the window of one step: its task, its first entry and the
// number of the task's entries from there on (the window takes up to 64*PW of them).
struct DSlot {
  int ti;
  int rem;
  int64_t lo;
};

template <int PW>
__device__ __forceinline__ int dslot_cnt(const DSlot& s) {
  return s.rem < 64 * PW ? s.rem : 64 * PW;
}

template <int MT, int PW>
struct DWin {
  uint32_t ph[PW], d[PW];              // phase, amplitude correction (float32 bits)
  uint32_t xk[PW][MT];                 // x at the entry's column (fp16 bits)
  int q[PW];                           // row of the entry in its task, -1 for none
};

// Stage 1: the records of the window's entries.
template <int PW>
__device__ __forceinline__ void dwin_positions(const DualStreamArgs& A, const DSlot& t, int lane, u32x2 (&ent)[PW]) {
  const int cnt = dslot_cnt<PW>(t);
  const uint32_t base = 8u * (uint32_t)t.lo;
  const rsrc_t r = make_rsrc(A.plug_ent, 8u * (uint32_t)A.plug_n);
#pragma unroll
  for (int w = 0; w < PW; ++w)
    vload64(ent[w], 64 * w + lane < cnt ? base + 8u * (uint32_t)(64 * w + lane) : OOB, r);
}

// Stage 2: per entry its row in the task, and x at its column.
template <int MT, int RG, int PW, int SM>
__device__ __forceinline__ void dwin_data(const DualStreamArgs& A, const DualSeg& S, const DSlot& t,
                                          const u32x2 (&ent)[PW], int lane, DWin<MT, PW>& W) {
  const int cnt = dslot_cnt<PW>(t);
#pragma unroll
  for (int w = 0; w < PW; ++w) {
    const int e = 64 * w + lane;
    const int row = (int)((ent[w].x >> 19) & 7u), k = (int)(ent[w].x & 0x7FFFFu);
    // entries of the task's other column slices are theirs
    const bool v = e < cnt && k >= S.kbeg && k < S.kend;
    W.q[w] = v ? row : -1;
    W.ph[w] = ent[w].x >> 22;
    W.d[w] = ent[w].y;
#pragma unroll
    for (int j = 0; j < MT; ++j)
      vload16(W.xk[w][j], (v && j < A.M) ? 2u * (uint32_t)(j * S.x_sm + k) : OOB, S.rx);
  }
}

// Stage 3: the corrections.
template <int MT, int RG, int PW>
__device__ __forceinline__ void dwin_apply(const char* lds, const DualLane& lo, const DWin<MT, PW>& W,
                                           float (&acc)[RG][2][MT]) {
#pragma unroll
  for (int w = 0; w < PW; ++w) {
    const float2 cs = *reinterpret_cast<const float2*>(lds + DLDS_CS + ((W.ph[w] << 7) | lo.cs));
    const float d = __uint_as_float(W.d[w]);
    float dx[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) dx[j] = d * h2f(W.xk[w][j]);
#pragma unroll
    for (int q = 0; q < RG; ++q) {
      const bool on = q == W.q[w];
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const float t = on ? dx[j] : 0.f;
        acc[q][0][j] = fmaf(t, cs.x, acc[q][0][j]);
        acc[q][1][j] = fmaf(t, cs.y, acc[q][1][j]);
      }
    }
  }
}

// The task's sums reduced over the wave: lane `wr` holds (row r, model m, token j).
struct DReduced {
  float y;
  int r, m, j;
  bool wr;
};

// The (row, model, token) lane `lane` holds after the reduction below, and whether it writes.
template <int MT, int RG>
__device__ __forceinline__ DReduced dred_slot(const DualStreamArgs& A, const DualSeg& S, int ti, int lane) {
  constexpr int LNV = Log2<RG * 2 * MT>::v;
  DReduced o;
  o.y = 0.f;
  const int idx = lane >> (6 - LNV);
  o.r = idx / (2 * MT);
  o.m = (idx / MT) & 1;
  o.j = idx % MT;
  const int nr = min(RG, S.nrows - ti * RG);
  o.wr = (lane & ((1 << (6 - LNV)) - 1)) == 0 && o.r < nr && o.j < A.M;
  return o;
}

template <int MT, int RG>
__device__ __forceinline__ DReduced dtask_reduce(const DualStreamArgs& A, const DualSeg& S, int ti, int lane,
                                                 float (&acc)[RG][2][MT]) {
  constexpr int NV = RG * 2 * MT;
  constexpr int LNV = Log2<NV>::v;
  static_assert((1 << LNV) == NV, "RG*2*MT must be a power of two");
  float v[NV];
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int j = 0; j < MT; ++j) v[(r * 2 + m) * MT + j] = acc[r][m][j];
  DReduced o = dred_slot<MT, RG>(A, S, ti, lane);
  o.y = wave_transpose_reduce<LNV>(v, lane);
  return o;
}

template <int RG>
__device__ __forceinline__ void dtask_store(const DualStreamArgs& A, const DualSeg& S, int ti, const DReduced& o,
                                            float y) {
  const uint32_t off = 2u * (uint32_t)((int64_t)o.j * S.o_sm + (int64_t)(ti * RG + o.r));
  const uint32_t obytes = 2u * (uint32_t)((int64_t)(A.M - 1) * S.o_sm + (int64_t)S.nrows);
  const f16 h = (f16)y;
#pragma unroll
  for (int mm = 0; mm < 2; ++mm)
    vstore16((uint32_t)__builtin_bit_cast(unsigned short, h), (o.wr && o.m == mm) ? off : OOB,
             make_rsrc(S.out[mm], obytes));
}

template <int MT, int RG>
__device__ __forceinline__ void dtask_write(const DualStreamArgs& A, const DualSeg& S, int ti, int lane,
                                            float (&acc)[RG][2][MT]) {
  const DReduced o = dtask_reduce<MT, RG>(A, S, ti, lane, acc);
  dtask_store<RG>(A, S, ti, o, o.y);
}

// A column slice of task ti: add the sums to the projection's accumulators and count the
// part in the task's counter; the last part to arrive takes the totals (swapping in
// zeros, so the workspace is clean for the next launch), writes the outputs and clears
// the counter.  Every workspace access is a device-scope atomic, performed where all CUs
// see it; "sums before count" comes from a data dependence (the count added is
// 1 + 0 * the values the sum atomics returned).
template <int MT, int RG>
__device__ __forceinline__ void dtask_accumulate(const DualStreamArgs& A, const DualSeg& S, int ti, int lane,
                                                 float (&acc)[RG][2][MT]) {
  const DReduced o = dtask_reduce<MT, RG>(A, S, ti, lane, acc);
  float* a = S.acc + ((int64_t)(o.m * A.M + o.j) * S.N + S.row0 + ti * RG + o.r);
  float before = 0.f;
  if (o.wr) before = __hip_atomic_fetch_add(a, o.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // a zero the compiler cannot see through, computed from the returned sums
  uint32_t z;
  asm volatile("v_and_b32 %0, 0, %1" : "=v"(z) : "v"(before));
  uint32_t old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(S.cnt + ti, 1u + z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __builtin_amdgcn_readfirstlane(old);
  if (old + 1 == (uint32_t)S.parts) {
    const float t = o.wr ? __hip_atomic_exchange(a, 0.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
    dtask_store<RG>(A, S, ti, o, t);
    if (lane == 0) __hip_atomic_exchange(S.cnt + ti, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <int MT, int RG>
__device__ __forceinline__ void dzero(float (&acc)[RG][2][MT]) {
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[r][0][j] = acc[r][1][j] = 0.f;
}

template <int MT, int RG, int PW, int LAYOUT, int SM, bool SPLIT>
struct DualRunner {
  const char* lds;
  DualLane lo;
  const DualStreamArgs& A;
  const DualSeg& S;
  int lane, nck, ntask, task0;
  uint32_t voff[RG];
  float acc[RG][2][MT];
  float pend[RG][2][MT];
  int pend_ti;
  DSlot pend_left;           // entries of the parked task left after its last step
  Cursor lc;                 // chunk to prefetch
  bool lc_live;              // false once every chunk of the wave is issued
  DSlot s0, s1, s2;          // windows of steps s, s+1, s+2 (s = the step being computed)
  Cursor c3;                 // step s+3, whose task plug range is in flight
  u32x4 T;                   // that range: {tlo lo, tlo hi, thi lo, thi hi}
  u32x2 I[PW];               // records of the entries of step s+1's window
  DWin<MT, PW> D;            // data of step s's window

  __device__ __forceinline__ DualRunner(const char* l, const DualStreamArgs& a, const DualSeg& s, int t0)
      : lds(l), A(a), S(s), task0(t0), pend_ti(-1) {
    lane = threadIdx.x & 63;
    lo = dual_lane(lane);
    nck = (S.kend - S.kbeg + DPAIRS - 1) / DPAIRS;
    ntask = (S.nrows + RG - 1) / RG;
    lc = {0, 0};
    lc_live = true;
#pragma unroll
    for (int r = 0; r < RG; ++r) voff[r] = 2u * (uint32_t)(r * S.ldc) + 16u * lane;
    dzero<MT, RG>(acc);
  }

  __device__ __forceinline__ void advance(Cursor& c) const {
    if (++c.ck == nck) {
      c.ck = 0;
      ++c.ti;
    }
  }
  // Cursor for the plug windows: stops one task past the end (empty windows).
  __device__ __forceinline__ void advance_slot(Cursor& c) const {
    if (c.ti < ntask) advance(c);
  }

  // Ranges come from task_plug, one load per task; with per-task records (task_cap > 0) a
  // task's range is its block of the array, known without a load.
  __device__ __forceinline__ void load_range(const Cursor& c, u32x4& t) const {
    if (uniform64(A.task_cap) > 0) {
      t = u32x4{0u, 0u, 0u, 0u};
      return;
    }
    vload128(t, c.ti < ntask ? 16u * (uint32_t)(task0 + c.ti) : OOB,
             make_rsrc(A.task_plug, 16u * (uint32_t)A.n_tasks));
  }
  __device__ __forceinline__ DSlot slot_of(const Cursor& c, const u32x4& t) const {
    const int64_t cap = uniform64(A.task_cap);
    int64_t tlo, thi;
    if (cap > 0) {
      tlo = (int64_t)(task0 + c.ti) * cap;
      thi = c.ti < ntask ? min(tlo + cap, (int64_t)A.plug_n) : tlo;
    } else {
      tlo = (int64_t)(((uint64_t)__builtin_amdgcn_readfirstlane(t.y) << 32) | __builtin_amdgcn_readfirstlane(t.x));
      thi = (int64_t)(((uint64_t)__builtin_amdgcn_readfirstlane(t.w) << 32) | __builtin_amdgcn_readfirstlane(t.z));
    }
    DSlot s;
    s.ti = c.ti;
    s.lo = tlo + (int64_t)(64 * PW) * c.ck;
    const int64_t r = thi - s.lo;
    s.rem = r <= 0 ? 0 : r >= 0x7FFFFFFF ? 0x7FFFFFFF : (int)r;
    return s;
  }

  __device__ __forceinline__ void prefetch(DChunk<MT, RG>& c) {
    dchunk_issue<MT, RG, SM>(A, S, lc.ti * RG, S.kbeg + lc.ck * DPAIRS, voff, lane, lc_live, c);
    Cursor nx = lc;
    advance(nx);
    if (nx.ti < ntask) lc = nx;
    else lc_live = false;
  }

  // Entries of the finished task that its steps could not take, then its outputs.
  __device__ __forceinline__ void finish_pending() {
    for (DSlot t = pend_left; t.rem > 0; t.lo += 64 * PW, t.rem -= 64 * PW) {
      u32x2 idx[PW];
      DWin<MT, PW> W;
      dwin_positions<PW>(A, t, lane, idx);
      dwin_data<MT, RG, PW, SM>(A, S, t, idx, lane, W);
      dwin_apply<MT, RG, PW>(lds, lo, W, pend);
    }
    if (SPLIT && S.red != nullptr) S.red[lane] = dtask_reduce<MT, RG>(A, S, pend_ti, lane, pend).y;
    else if (SPLIT && S.parts > 1) dtask_accumulate<MT, RG>(A, S, pend_ti, lane, pend);
    else dtask_write<MT, RG>(A, S, pend_ti, lane, pend);
    pend_ti = -1;
  }

  // range of step s+2, range load for s+3 | corrections of step s | data loads for s+1 |
  // positions for s+2 | [first chunk] finish the previous task | prefetch | decode | [last
  // chunk] park the sums.  The prefetch is the step's last load: every load the next step
  // waits for (range, data, positions) was issued before it, so with three buffers the
  // chunk it requests is first waited for two steps later (the buffer counter is in order).
  __device__ __forceinline__ void step(Cursor& cur, DChunk<MT, RG>& comp, DChunk<MT, RG>& pref) {
    s2 = slot_of(c3, T);
    advance_slot(c3);
    load_range(c3, T);
    if (dslot_cnt<PW>(s0) > 0) dwin_apply<MT, RG, PW>(lds, lo, D, acc);
    dwin_data<MT, RG, PW, SM>(A, S, s1, I, lane, D);
    dwin_positions<PW>(A, s2, lane, I);
    if (cur.ck == 0 && pend_ti >= 0) finish_pending();
    prefetch(pref);
    dchunk_compute<MT, RG, LAYOUT, SM>(lds, lo, comp, acc);
    if (cur.ck == nck - 1) {
#pragma unroll
      for (int r = 0; r < RG; ++r)
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int j = 0; j < MT; ++j) pend[r][m][j] = acc[r][m][j];
      dzero<MT, RG>(acc);
      pend_ti = cur.ti;
      pend_left = s0;
      pend_left.lo += 64 * PW;
      pend_left.rem = s0.rem > 64 * PW ? s0.rem - 64 * PW : 0;
    }
    s0 = s1;
    s1 = s2;
    advance(cur);
  }

  // The walk's ntask * nck steps over NB rotating buffers (cb[0 .. NB-2] already issued):
  // whole rounds of NB steps with no exit inside a round (an exit inside makes the
  // compiler's count of loads in flight at the round's first decode conservative, so it
  // waits for the chunks the round has in flight), then the steps left.
  template <int NB>
  __device__ __forceinline__ void walk(DChunk<MT, RG> (&cb)[NB]) {
    const int n = ntask * nck;
    Cursor cur = {0, 0};
    int i = 0;
    if constexpr (NB == 3) {
      for (; i + 3 <= n; i += 3) {
        step(cur, cb[0], cb[2]);
        step(cur, cb[1], cb[0]);
        step(cur, cb[2], cb[1]);
      }
      if (i < n) step(cur, cb[0], cb[2]);
      if (i + 1 < n) step(cur, cb[1], cb[0]);
    } else {
      for (; i + 2 <= n; i += 2) {
        step(cur, cb[0], cb[1]);
        step(cur, cb[1], cb[0]);
      }
      if (i < n) step(cur, cb[0], cb[1]);
    }
  }

  // One-Linear launch, in three parts around the table build: start_ranges() requests the
  // plug ranges of steps 0-2 (the first thing a wave loads), start_chunks() waits for the
  // first two, requests the entries of step 0's window and issues the first chunks,
  // run_started() (after the build) completes the window stages and runs the walk.
  u32x4 Tr[2];
  __device__ __forceinline__ void start_ranges() {
    Cursor c = {0, 0};
    load_range(c, Tr[0]);
    advance_slot(c);
    load_range(c, Tr[1]);
    advance_slot(c);
    load_range(c, T);
    c3 = c;
  }
  template <int NPRE, int NB>
  __device__ __forceinline__ void start_chunks(DChunk<MT, RG> (&cb)[NB]) {
    s0 = slot_of(Cursor{0, 0}, Tr[0]);
    Cursor c = {0, 0};
    advance_slot(c);
    s1 = slot_of(c, Tr[1]);
    dwin_positions<PW>(A, s0, lane, I);
#pragma unroll
    for (int b = 0; b < NPRE; ++b) prefetch(cb[b]);
  }
  // A wave of one task and one chunk (the usual one-Linear shape) in straight-line code:
  // the activations of its corrections are requested, the chunk decoded while they are in
  // flight (its codes arrived before the table barrier), then the corrections applied;
  // entries past the first window are taken when the task finishes.
  __device__ __forceinline__ void run_started_single(const DChunk<MT, RG>& c) {
    dwin_data<MT, RG, PW, SM>(A, S, s0, I, lane, D);
    dchunk_compute<MT, RG, LAYOUT, SM>(lds, lo, c, acc);
    // unconditional (an empty window adds zeros), so that the activation loads are not
    // moved into a branch after the decode
    dwin_apply<MT, RG, PW>(lds, lo, D, acc);
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int j = 0; j < MT; ++j) pend[r][m][j] = acc[r][m][j];
    pend_ti = 0;
    pend_left = s0;
    pend_left.lo += 64 * PW;
    pend_left.rem = s0.rem > 64 * PW ? s0.rem - 64 * PW : 0;
    finish_pending();
  }
  __device__ __forceinline__ void run_started_one(DChunk<MT, RG> (&cb)[3]) {
    dwin_data<MT, RG, PW, SM>(A, S, s0, I, lane, D);
    dwin_positions<PW>(A, s1, lane, I);
    walk<3>(cb);
    finish_pending();
  }
  __device__ __forceinline__ void run_started_two(DChunk<MT, RG> (&cb)[2]) {
    dwin_data<MT, RG, PW, SM>(A, S, s0, I, lane, D);
    dwin_positions<PW>(A, s1, lane, I);
    walk<2>(cb);
    finish_pending();
  }

  __device__ __forceinline__ void run() {
    if (ntask <= 0 || S.kend <= S.kbeg) return;
    // fill the window stages for steps 0 and 1, the range of step 2 in flight
    Cursor c = {0, 0};
    load_range(c, T);
    s0 = slot_of(c, T);
    advance_slot(c);
    load_range(c, T);
    s1 = slot_of(c, T);
    dwin_positions<PW>(A, s0, lane, I);
    dwin_data<MT, RG, PW, SM>(A, S, s0, I, lane, D);
    dwin_positions<PW>(A, s1, lane, I);
    c3 = c;
    advance_slot(c3);
    load_range(c3, T);
    // c3 now names step 2; step() turns T into s2 and moves c3 to step 3
    if constexpr (MT == 1) {
      // one token: two chunks in flight while one is decoded (measured 1-2 % faster on
      // the 3B stream than one; the registers of more tokens leave room for one)
      DChunk<MT, RG> cb[3];
      prefetch(cb[0]);
      prefetch(cb[1]);
      walk<3>(cb);
    } else {
      DChunk<MT, RG> cb[2];
      prefetch(cb[0]);
      walk<2>(cb);
    }
    finish_pending();
  }
};

__device__ __forceinline__ void dual_seg(const pp_dual_proj& P, int row0, int row1, int M, DualSeg& S) {
  const int ldc = uniform((int)P.ldc), K = uniform(P.K);
  row0 = uniform(row0);
  row1 = uniform(row1);
  S.ldc = ldc;
  S.K = K;
  S.nrows = row1 - row0;
  S.x_sm = uniform((int)P.x_sm);
  S.pos0 = uniform64(P.pos0) + (int64_t)row0 * ldc;
  S.codes = reinterpret_cast<const uint16_t*>(uniform_ptr(P.codes)) + (int64_t)row0 * ldc;
  S.x = reinterpret_cast<const f16*>(uniform_ptr(P.x));
  S.rx = make_rsrc(S.x, 2u * (uint32_t)((M - 1) * S.x_sm + K));
  S.rcs = make_rsrc(S.codes, 2u * (uint32_t)((int64_t)(S.nrows - 1) * ldc + K));
#pragma unroll
  for (int m = 0; m < 2; ++m) S.out[m] = reinterpret_cast<f16*>(uniform_ptr(P.out[m])) + row0;
  S.o_sm = uniform64(P.o_sm);
  S.kbeg = 0;
  S.kend = K;
  S.parts = 1;
  S.N = uniform(P.N);
  S.row0 = row0;
  S.acc = nullptr;
  S.cnt = nullptr;
  S.red = nullptr;
}

template <int MT, int PW, int LAYOUT, int SM, bool SPLIT>
__global__ __launch_bounds__(DualCfg<MT>::NT) void dual_stream_kernel(const DualStreamArgs A) {
  constexpr int RG = DualCfg<MT>::RG, WAVES = DualCfg<MT>::NT / 64;
  __shared__ __attribute__((aligned(16))) uint32_t T[DLDS_BYTES / 4];
  char* lds = reinterpret_cast<char*>(T);
  const int64_t gw = (int64_t)blockIdx.x * WAVES + uniform(threadIdx.x >> 6);
  SegRange sr;
  sr.issue(A.seg_bounds, gw, (int64_t)gridDim.x * WAVES);
  dual_build_lds<LAYOUT, DualCfg<MT>::NT>(lds, A);
  __syncthreads();
  const int64_t s0 = sr.lo(), s1 = sr.hi();
  for (int64_t si = s0; si < s1; ++si) {
    const pp_quad_seg g = A.segs[si];
    DualSeg S;
    dual_seg(A.projs[uniform(g.proj)], g.row0, g.row1, A.M, S);
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
    DualRunner<MT, RG, PW, LAYOUT, SM, SPLIT> R(lds, A, S, uniform(g.task0));
    R.run();
  }
}

// One Linear: wave gw's column slice and task run from the launch shape (direct_item, as
// the quad row kernel deals them), no segment table.  The wave requests its first plug
// ranges, then the LUTs, its first window's entries and first chunks, so their round trips
// run under the table build.
// PARTS: 0 whole rows; 1 K parts meeting through the workspace; 2 a task's parts are
// consecutive waves of one workgroup (wg_item), each parks its reduced sums in LDS and, after a
// barrier every wave of the workgroup reaches, the part-0 wave adds them and writes the outputs
// (no workspace, no atomics); 3 as 2 with one chunk per part (parts == chunks), run in
// straight-line code (run_started_single).
template <int MT, int PW, int LAYOUT, int SM, int PARTS>
__global__ __launch_bounds__(DualCfg<MT>::NT) void dual_direct_kernel(const DualStreamArgs A) {
  constexpr int RG = DualCfg<MT>::RG, NT = DualCfg<MT>::NT, WAVES = NT / 64;
  constexpr bool SPLIT = PARTS != 0;
  __shared__ __attribute__((aligned(16))) uint32_t Tb[(DLDS_BYTES + (PARTS >= 2 ? 256 * WAVES : 0)) / 4];
  char* lds = reinterpret_cast<char*>(Tb);
  const int wave = uniform(threadIdx.x >> 6);
  const int64_t gw = (int64_t)blockIdx.x * WAVES + wave;
  const int K = uniform(A.proj.K), N = uniform(A.proj.N);
  constexpr bool wg = PARTS >= 2;
  const uint32_t parts = (uint32_t)uniform(A.parts);
  const DirectItem d = wg ? wg_item<WAVES>(blockIdx.x, gridDim.x, (uint32_t)wave, (uint32_t)uniform64(A.n_tasks), parts,
                                           (uint32_t)uniform(A.n_chunks), DPAIRS, (uint32_t)K)
                          : direct_item<WAVES>((uint32_t)gw, gridDim.x * WAVES, (uint32_t)uniform64(A.n_tasks), parts,
                                               (uint32_t)uniform(A.n_chunks), DPAIRS, (uint32_t)K);
  DualSeg S;
  dual_seg(A.proj, min(d.t0 * RG, N), min(d.t1 * RG, N), A.M, S);
  S.kbeg = uniform(d.kbeg);
  S.kend = uniform(d.kend);
  S.red = nullptr;
  float* red = reinterpret_cast<float*>(lds + DLDS_BYTES);
  if (SPLIT && parts > 1) {
    S.parts = (int)parts;
    if (wg) {
      S.red = red + 64 * wave;
    } else {
      S.acc = uniform_ptr(A.acc);
      S.cnt = uniform_ptr(A.cnt) + d.t0;
    }
  }
  const bool busy = S.nrows > 0 && S.kend > S.kbeg;
  DualRunner<MT, RG, PW, LAYOUT, SM, SPLIT> R(lds, A, S, d.t0);
  if (busy) R.start_ranges();
  DualTableBuild<LAYOUT, NT> tb;
  tb.load(A);
  constexpr int NB = MT == 1 ? 3 : 2;
  DChunk<MT, RG> cb[NB];
  if (busy) R.template start_chunks<NB - 1>(cb);
  tb.store(lds);
  __syncthreads();
  if constexpr (!wg) {
    if (!busy) return;
    if constexpr (MT == 1) R.run_started_one(cb);
    else R.run_started_two(cb);
  } else {
    if (busy) {
      if constexpr (PARTS == 3) R.run_started_single(cb[0]);
      else if constexpr (MT == 1) R.run_started_one(cb);
      else R.run_started_two(cb);
    }
    __syncthreads();   // every wave of the workgroup: the parked sums are in LDS
    const int lane = threadIdx.x & 63;
    if (busy && wave % (int)parts == 0) {
      DReduced o = dred_slot<MT, RG>(A, S, 0, lane);
      float y = 0.f;
      for (int p = 0; p < (int)parts; ++p) y += red[64 * (wave + p) + lane];
      dtask_store<RG>(A, S, 0, o, y);
    }
  }
}

// ------------------------------------------------------------------ tail rows
struct DualTailArgs {
  const pp_dual_proj* projs;
  const pp_quad_item* items;
  int64_t n_items;
  DualStreamArgs S;
  int layout;
  int64_t n_codes;
  const f16* tails[2];
  int64_t tail_len[2];
};

// Up to 8 rows that lie wholly past n_codes: for each model either wholly inside its fp16
// tail (a plain fp16 GEMV, 16-byte loads of 8 weights per lane and row) or wholly past it
// (outputs 0).  Needs n_codes % 8 == 0, K % 8 == 0 and 16-byte aligned tails, so that
// every lane's 8 weights are one aligned load.
template <int MT>
__device__ __forceinline__ void dual_tail_rows(const DualTailArgs& T, const pp_quad_item& it, int lane) {
  constexpr int R = 8, NV = R * 2 * MT, LNV = Log2<NV>::v;
  const pp_dual_proj& P = T.projs[uniform(it.proj)];
  const int K = uniform(P.K), ldc = uniform((int)P.ldc), nr = uniform(it.nrows), row0 = uniform(it.row0);
  const int x_sm = uniform((int)P.x_sm), M = T.S.M;
  const int64_t t0 = uniform64(P.pos0) + (int64_t)row0 * ldc - T.n_codes;   // tail index of (row0, 0)
  const int64_t t_end = t0 + (int64_t)(nr - 1) * ldc + K;
  rsrc_t rt[2];
  bool has[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    has[m] = t0 >= 0 && t_end <= T.tail_len[m];
    rt[m] = make_rsrc(has[m] ? T.tails[m] + t0 : nullptr, has[m] ? 2u * (uint32_t)(t_end - t0) : 0u);
  }
  const rsrc_t rx = make_rsrc(uniform_ptr(P.x), 2u * (uint32_t)((M - 1) * x_sm + K));
  float acc[R][2][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int j = 0; j < MT; ++j) acc[r][m][j] = 0.f;
  // 512 columns per step, the next step's loads in flight while one is summed (columns
  // past K read 0)
  struct Step {
    u32x4 xr[MT];
    u32x4 wr[R][2];
  };
  auto issue = [&](int kc, Step& c) {
    const int k = kc + 8 * lane;
    const bool kin = k < K;
#pragma unroll
    for (int j = 0; j < MT; ++j) vload128c(c.xr[j], (kin && j < M) ? 2u * (uint32_t)(j * x_sm + k) : OOB, rx);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < 2; ++m)
        vload128(c.wr[r][m], (kin && r < nr) ? 2u * (uint32_t)(r * ldc + k) : OOB, rt[m]);
  };
  auto sum = [&](const Step& c) {
    float xv[MT][8];
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const f16x4 h0 = __builtin_bit_cast(f16x4, u32x2{c.xr[j].x, c.xr[j].y});
      const f16x4 h1 = __builtin_bit_cast(f16x4, u32x2{c.xr[j].z, c.xr[j].w});
      xv[j][0] = (float)h0.x; xv[j][1] = (float)h0.y; xv[j][2] = (float)h0.z; xv[j][3] = (float)h0.w;
      xv[j][4] = (float)h1.x; xv[j][5] = (float)h1.y; xv[j][6] = (float)h1.z; xv[j][7] = (float)h1.w;
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const f16x4 h0 = __builtin_bit_cast(f16x4, u32x2{c.wr[r][m].x, c.wr[r][m].y});
        const f16x4 h1 = __builtin_bit_cast(f16x4, u32x2{c.wr[r][m].z, c.wr[r][m].w});
        const float wv[8] = {(float)h0.x, (float)h0.y, (float)h0.z, (float)h0.w,
                             (float)h1.x, (float)h1.y, (float)h1.z, (float)h1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
          for (int j = 0; j < MT; ++j) acc[r][m][j] = fmaf(wv[e], xv[j][e], acc[r][m][j]);
      }
  };
  Step c0, c1;
  issue(0, c0);
  for (int kc = 0; kc < K; kc += 1024) {
    issue(kc + 512, c1);
    sum(c0);
    if (kc + 512 >= K) break;
    issue(kc + 1024, c0);
    sum(c1);
  }
  float v[NV];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int j = 0; j < MT; ++j) v[(r * 2 + m) * MT + j] = acc[r][m][j];
  const float y = wave_transpose_reduce<LNV>(v, lane);
  const int idx = lane >> (6 - LNV);
  const int r = idx / (2 * MT), m = (idx / MT) & 1, j = idx % MT;
  const bool wr_ = (lane & ((1 << (6 - LNV)) - 1)) == 0 && r < nr && j < M;
  const int64_t o_sm = uniform64(P.o_sm);
  const uint32_t off = 2u * (uint32_t)((int64_t)j * o_sm + row0 + r);
  const uint32_t obytes = 2u * (uint32_t)((int64_t)(M - 1) * o_sm + P.N);
  const f16 h = (f16)y;
#pragma unroll
  for (int mm = 0; mm < 2; ++mm)
    vstore16((uint32_t)__builtin_bit_cast(unsigned short, h), (wr_ && m == mm) ? off : OOB,
             make_rsrc(uniform_ptr(P.out[mm]), obytes));
}

// Rows that reach the FP16 tails.  PP_ITEM_FP16 items: see dual_tail_rows.  Other items
// (one row each, straddling n_codes or the end of a model's tail) element by element:
// positions < n_codes decode from the codes (with the plug entries of the row),
// positions >= n_codes read tails[m][pos - n_codes] when model m has them.
template <int MT, int LAYOUT, int SM>
__global__ __launch_bounds__(256) void dual_tail_kernel(const DualTailArgs T) {
  const int64_t ti = (int64_t)blockIdx.x * 4 + uniform(threadIdx.x >> 6);
  if (ti >= T.n_items) return;
  const DualStreamArgs& A = T.S;
  const int lane = threadIdx.x & 63;
  const pp_quad_item it = T.items[ti];
  if (uniform(it.flags) & PP_ITEM_FP16) {
    dual_tail_rows<MT>(T, it, lane);
    return;
  }
  const pp_dual_proj& P = T.projs[it.proj];
  const int K = P.K;
  const int64_t pos_row = P.pos0 + (int64_t)it.row0 * P.ldc;
  const uint16_t* codes = reinterpret_cast<const uint16_t*>(P.codes) + (int64_t)it.row0 * P.ldc;
  const f16* x = reinterpret_cast<const f16*>(P.x);
  float acc[2][MT];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[m][j] = 0.f;
  for (int k = lane; k < K; k += 64) {
    const int64_t pos = pos_row + k;
    float w[2] = {0.f, 0.f};
    if (pos < T.n_codes) {
      const uint32_t code = dual_half<LAYOUT>(codes[k]);
      // the same decode as the row kernel, from global tables
      const uint32_t aq = ((code >> 10) & 63u) ^ (LAYOUT == PP_DUAL_I16_OFFSET ? 32u : 0u);
      const uint32_t ph = code & 1023u;
      float amp = A.amp_lut[aq] * (float)A.scales[dual_group<SM>(A, pos)];
      // plug entry at this position (binary search in the row's plug range)
      int64_t lo = it.plug_lo, hi = it.plug_hi;
      while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((int64_t)A.plug_idx[mid] < pos) lo = mid + 1;
        else hi = mid;
      }
      if (lo < it.plug_hi && (int64_t)A.plug_idx[lo] == pos) amp = (float)A.plug_amp[lo];
      w[0] = amp * A.cos_lut[ph];
      w[1] = amp * A.sin_lut[ph];
    } else {
      const int64_t t = pos - T.n_codes;
#pragma unroll
      for (int m = 0; m < 2; ++m)
        if (t < T.tail_len[m]) w[m] = (float)T.tails[m][t];
    }
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const float xk = j < A.M ? (float)x[(int64_t)j * P.x_sm + k] : 0.f;
#pragma unroll
      for (int m = 0; m < 2; ++m) acc[m][j] = fmaf(w[m], xk, acc[m][j]);
    }
  }
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const bool has = pos_row < T.n_codes || pos_row - T.n_codes < T.tail_len[m];
    f16* o = reinterpret_cast<f16*>(P.out[m]) + it.row0;
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const float v = wave_sum(acc[m][j]);
      if (lane == 0 && j < A.M) o[(int64_t)j * P.o_sm] = (f16)(has ? v : 0.f);
    }
  }
}

// The one-Linear launch's per-task records: task t's entries ent[task_plug[2t] ..
// task_plug[2t+1]) copied to out[t * cap ..], null records (column 0x7FFFF, past any K the
// decode takes, and a zero correction) after them.
__global__ __launch_bounds__(256) void dual_task_entries_kernel(const uint32_t* ent, int64_t plug_n,
                                                                const int64_t* task_plug, int64_t n_tasks,
                                                                int64_t cap, uint32_t* out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_tasks * cap) return;
  const int64_t t = i / cap, src = task_plug[2 * t] + (i - t * cap);
  const bool has = src < task_plug[2 * t + 1] && src < plug_n;
  out[2 * i] = has ? ent[2 * src] : 0x7FFFFu;
  out[2 * i + 1] = has ? ent[2 * src + 1] : 0u;
}

// Records of the plug entries for the stream decode (see DualStreamArgs::plug_ent).
// Projection p covers stream positions [proj_pos0[p], proj_pos0[p] + N_p * proj_k[p]);
// proj_pos0 has n_projs + 1 entries (the last one the end of the stream's projections).
// The correction is the one the decode applies to the pair's amplitude, in float32 with
// one rounding: d = plug_amp - amp_lut[aq] * scale.
__global__ __launch_bounds__(256) void dual_plug_table_kernel(const uint16_t* codes, int64_t n_codes, int layout,
                                                              const f16* scales, int64_t n_groups, int64_t gs,
                                                              int64_t chunk, const float* amp_lut,
                                                              const uint32_t* plug_idx, const f16* plug_amp,
                                                              int64_t plug_n, const int64_t* proj_pos0,
                                                              const int32_t* proj_k, int n_projs, int rows_per_task,
                                                              uint32_t* ent) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= plug_n) return;
  const int64_t p = plug_idx[j];
  uint32_t w0 = 0;
  float d = 0.f;
  if (p < n_codes) {
    const int64_t g = (p / chunk) * ((chunk + gs - 1) / gs) + (p % chunk) / gs;
    const float sc = g < n_groups ? (float)scales[g] : 0.f;
    const uint32_t st = codes[p];
    const uint32_t c = layout == PP_DUAL_U16_BE ? (((st & 0xFFu) << 8) | (st >> 8)) : (st ^ 0x8000u);
    w0 = (c & 0x3FFu) << 22;
    d = fmaf(-amp_lut[c >> 10], sc, (float)plug_amp[j]);
  }
  if (p >= proj_pos0[0] && p < proj_pos0[n_projs]) {
    int lo = 0, hi = n_projs - 1;                   // last projection starting at or before p
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (proj_pos0[mid] <= p) lo = mid;
      else hi = mid - 1;
    }
    const int64_t local = p - proj_pos0[lo], K = proj_k[lo];
    const int64_t row = local / K;
    w0 |= ((uint32_t)(row % rows_per_task) << 19) | (uint32_t)(local - row * K);
  }
  ent[2 * j] = w0;
  ent[2 * j + 1] = __float_as_uint(d);
}

// The group scales regrouped for the stream decode with R rows per task: for every
// projection i (stream positions proj_pos0[i] .. + N_i K_i, rows of K_i columns,
// K_i % gs == 0, proj_pos0[i] % (R gs) == 0, N_i % R == 0) and every run of R rows starting
// at row R b, position P = proj_pos0[i] + R b K_i: tab[P/gs + R j + q] =
// scales[(P + q K_i)/gs + j], the scale of row R b + q, column group j.  A decode step then
// loads the R rows' scales of its group in one load.  Entries outside every projection
// copy scales (0 past n_groups).
__global__ __launch_bounds__(256) void dual_scale_table_kernel(const f16* scales, int64_t n_groups, int log2gs,
                                                               const int64_t* proj_pos0, const int32_t* proj_n,
                                                               const int32_t* proj_k, int n_projs, int R, f16* tab,
                                                               int64_t n_tab) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_tab) return;
  int64_t src = t;
  const int64_t p = t << log2gs;   // stream position of group t
  if (p >= proj_pos0[0]) {
    int lo = 0, hi = n_projs - 1;   // last projection starting at or before p
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (proj_pos0[mid] <= p) lo = mid;
      else hi = mid - 1;
    }
    const int64_t K = proj_k[lo], gk = K >> log2gs;   // column groups per row
    const int64_t local = t - (proj_pos0[lo] >> log2gs);
    if (local < (int64_t)proj_n[lo] * gk) {
      const int64_t blk = local / (R * gk), r = local - blk * R * gk;
      const int64_t j = r / R, q = r - j * R;
      src = (proj_pos0[lo] >> log2gs) + (blk * R + q) * gk + j;
    }
  }
  tab[t] = src < n_groups ? scales[src] : (f16)0.f;
}

// ------------------------------------------------------------------ host side
static int dual_stream_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : 4; }
static int dual_stream_rg(int mt) { return mt == 1 ? DualCfg<1>::RG : mt == 2 ? DualCfg<2>::RG : DualCfg<4>::RG; }
static int dual_stream_nt(int mt) { return mt == 1 ? DualCfg<1>::NT : mt == 2 ? DualCfg<2>::NT : DualCfg<4>::NT; }

template <int MT, int LAYOUT, int SM>
static int launch_dual_stream(const DualStreamArgs& A, int pw, hipStream_t st) {
  const dim3 grid((unsigned)device_cu_count()), block(DualCfg<MT>::NT);
  if (A.ws != nullptr) {
    if (pw == 1) hipLaunchKernelGGL((dual_stream_kernel<MT, 1, LAYOUT, SM, true>), grid, block, 0, st, A);
    else hipLaunchKernelGGL((dual_stream_kernel<MT, 2, LAYOUT, SM, true>), grid, block, 0, st, A);
  } else {
    if (pw == 1) hipLaunchKernelGGL((dual_stream_kernel<MT, 1, LAYOUT, SM, false>), grid, block, 0, st, A);
    else hipLaunchKernelGGL((dual_stream_kernel<MT, 2, LAYOUT, SM, false>), grid, block, 0, st, A);
  }
  PP_LAUNCH_CHECK();
  return PP_OK;
}

template <int MT, int LAYOUT, int SM>
static int launch_dual_direct(const DualStreamArgs& A, int pw, hipStream_t st) {
  const dim3 grid((unsigned)device_cu_count()), block(DualCfg<MT>::NT);
  if (MT == 1 && A.parts > 1 && A.wg_parts && A.parts == A.n_chunks) {
    if (pw == 1) hipLaunchKernelGGL((dual_direct_kernel<MT, 1, LAYOUT, SM, 3>), grid, block, 0, st, A);
    else hipLaunchKernelGGL((dual_direct_kernel<MT, 2, LAYOUT, SM, 3>), grid, block, 0, st, A);
  } else if (A.parts > 1 && A.wg_parts) {
    if (pw == 1) hipLaunchKernelGGL((dual_direct_kernel<MT, 1, LAYOUT, SM, 2>), grid, block, 0, st, A);
    else hipLaunchKernelGGL((dual_direct_kernel<MT, 2, LAYOUT, SM, 2>), grid, block, 0, st, A);
  } else if (A.parts > 1) {
    if (pw == 1) hipLaunchKernelGGL((dual_direct_kernel<MT, 1, LAYOUT, SM, 1>), grid, block, 0, st, A);
    else hipLaunchKernelGGL((dual_direct_kernel<MT, 2, LAYOUT, SM, 1>), grid, block, 0, st, A);
  } else {
    if (pw == 1) hipLaunchKernelGGL((dual_direct_kernel<MT, 1, LAYOUT, SM, 0>), grid, block, 0, st, A);
    else hipLaunchKernelGGL((dual_direct_kernel<MT, 2, LAYOUT, SM, 0>), grid, block, 0, st, A);
  }
  PP_LAUNCH_CHECK();
  return PP_OK;
}

template <int LAYOUT, int SM>
static int dispatch_dual_direct(const DualStreamArgs& A, int mt, int pw, hipStream_t st) {
  switch (mt) {
    case 1: return launch_dual_direct<1, LAYOUT, SM>(A, pw, st);
    case 2: return launch_dual_direct<2, LAYOUT, SM>(A, pw, st);
    default: return launch_dual_direct<4, LAYOUT, SM>(A, pw, st);
  }
}

// One Linear of a dual stream: T tasks and their column slices (direct_parts), the split
// workspace (per-task counters, 256-byte aligned, then accumulators [2][M][N]).
struct DualDirectPlan {
  int mt, rg, parts, n_chunks;
  bool wg;                 // the parts meet in LDS (no workspace)
  int64_t n_tasks, waves, cnt_bytes, split_bytes;
};
static DualDirectPlan dual_direct_plan(int64_t M, int64_t N, int64_t K) {
  DualDirectPlan p;
  p.mt = M <= 1 ? 1 : M <= 2 ? 2 : 4;
  p.rg = p.mt == 1 ? DualCfg<1>::RG : p.mt == 2 ? DualCfg<2>::RG : DualCfg<4>::RG;
  const int nt = p.mt == 1 ? DualCfg<1>::NT : p.mt == 2 ? DualCfg<2>::NT : DualCfg<4>::NT;
  p.waves = (int64_t)device_cu_count() * (nt / 64);
  p.n_tasks = (N + p.rg - 1) / p.rg;
  p.n_chunks = (int)std::max<int64_t>(1, (K + DPAIRS - 1) / DPAIRS);
  p.parts = direct_parts(p.n_tasks, p.waves, p.n_chunks);
  p.wg = wg_parts_ok(p.n_tasks, p.waves, p.parts, nt / 64);
  p.cnt_bytes = p.parts > 1 && !p.wg ? (p.n_tasks * 4 + 255) / 256 * 256 : 0;
  p.split_bytes = p.parts > 1 && !p.wg ? p.cnt_bytes + 4 * 2 * M * N : 0;
  return p;
}

template <int LAYOUT, int SM>
static int dispatch_dual_stream(const DualStreamArgs& A, int mt, int pw, hipStream_t st) {
  switch (mt) {
    case 1: return launch_dual_stream<1, LAYOUT, SM>(A, pw, st);
    case 2: return launch_dual_stream<2, LAYOUT, SM>(A, pw, st);
    default: return launch_dual_stream<4, LAYOUT, SM>(A, pw, st);
  }
}

template <int LAYOUT, int SM>
static int dispatch_dual_tail(const DualTailArgs& T, int mt, hipStream_t st) {
  const unsigned grid = (unsigned)((T.n_items + 3) / 4);
  switch (mt) {
    case 1: hipLaunchKernelGGL((dual_tail_kernel<1, LAYOUT, SM>), dim3(grid), dim3(256), 0, st, T); break;
    case 2: hipLaunchKernelGGL((dual_tail_kernel<2, LAYOUT, SM>), dim3(grid), dim3(256), 0, st, T); break;
    default: hipLaunchKernelGGL((dual_tail_kernel<4, LAYOUT, SM>), dim3(grid), dim3(256), 0, st, T); break;
  }
  PP_LAUNCH_CHECK();
  return PP_OK;
}

}  // namespace pp

using namespace pp;

extern "C" int pp_dual_stream_rows(int64_t M) {
  if (M < 1 || M > 4) {
    set_error("the dual stream decode takes 1..4 tokens, got %lld", (long long)M);
    return 0;
  }
  return dual_stream_rg(dual_stream_mt(M));
}

extern "C" int pp_dual_plug_table(const void* codes, int64_t n_codes, int code_layout, const void* scales,
                                  int64_t n_groups, int64_t group_size, int64_t chunk_size, const float* amp_lut,
                                  const uint32_t* plug_idx, const void* plug_amp, int64_t plug_n,
                                  const int64_t* proj_pos0, const int32_t* proj_k, int64_t n_projs,
                                  int64_t rows_per_task, uint32_t* ent, void* stream) {
  PP_REQUIRE(plug_n >= 0 && plug_n < (1ll << 28), "the stream decode takes fewer than 2^28 plug entries");
  if (plug_n == 0) return PP_OK;
  PP_REQUIRE(codes && scales && amp_lut && plug_idx && plug_amp && proj_pos0 && proj_k && ent, "null pointer");
  PP_REQUIRE(code_layout == PP_DUAL_I16_OFFSET || code_layout == PP_DUAL_U16_BE, "bad code_layout");
  PP_REQUIRE(n_codes >= 0 && n_groups >= 1 && group_size >= 1 && chunk_size >= 1, "bad sizes");
  PP_REQUIRE(n_projs >= 1 && n_projs < (1ll << 30), "bad n_projs");
  PP_REQUIRE(rows_per_task >= 1 && rows_per_task <= 8, "bad rows_per_task");
  hipLaunchKernelGGL(dual_plug_table_kernel, dim3((unsigned)((plug_n + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const uint16_t*>(codes), n_codes,
                     code_layout, reinterpret_cast<const f16*>(scales), n_groups, group_size, chunk_size, amp_lut,
                     plug_idx, reinterpret_cast<const f16*>(plug_amp), plug_n, proj_pos0, proj_k, (int)n_projs,
                     (int)rows_per_task, ent);
  PP_LAUNCH_CHECK();
  return PP_OK;
}

extern "C" int pp_dual_scale_table(const void* scales, int64_t n_groups, int64_t group_size,
                                   const int64_t* proj_pos0, const int32_t* proj_n, const int32_t* proj_k,
                                   int64_t n_projs, int64_t rows_per_task, void* tab, int64_t n_tab, void* stream) {
  PP_REQUIRE(scales && proj_pos0 && proj_n && proj_k && tab, "null pointer");
  PP_REQUIRE(n_groups >= 1 && n_tab >= 1 && n_tab < (1ll << 40), "bad n_groups / n_tab");
  PP_REQUIRE(group_size >= 8 && (group_size & (group_size - 1)) == 0, "group_size must be a power of two >= 8");
  PP_REQUIRE(n_projs >= 1 && n_projs < (1ll << 30), "bad n_projs");
  PP_REQUIRE(rows_per_task == 8 || rows_per_task == 4 || rows_per_task == 2,
             "rows_per_task must be pp_dual_stream_rows(M): 8, 4 or 2");
  int log2gs = 0;
  while ((1ll << log2gs) < group_size) ++log2gs;
  hipLaunchKernelGGL(dual_scale_table_kernel, dim3((unsigned)((n_tab + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), reinterpret_cast<const f16*>(scales), n_groups, log2gs,
                     proj_pos0, proj_n, proj_k, (int)n_projs, (int)rows_per_task, reinterpret_cast<f16*>(tab),
                     n_tab);
  PP_LAUNCH_CHECK();
  return PP_OK;
}

extern "C" int pp_dual_stream_chunk(int64_t M) { return M < 1 || M > 4 ? 0 : DPAIRS; }

extern "C" int64_t pp_dual_stream_waves(int64_t M) {
  if (M < 1 || M > 4) return 0;
  return (int64_t)device_cu_count() * (dual_stream_nt(dual_stream_mt(M)) / 64);
}

extern "C" int pp_dual_rows_parts(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > 4 || N < 1 || K < 1) return 0;
  return dual_direct_plan(M, N, K).parts;
}

extern "C" int64_t pp_dual_rows_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > 4 || N < 1 || K < 1) return 0;
  return dual_direct_plan(M, N, K).split_bytes;
}

extern "C" int pp_dual_task_entries(const uint32_t* plug_ent, int64_t plug_n, const int64_t* task_plug,
                                    int64_t n_tasks, int64_t task_cap, uint32_t* out, void* stream) {
  PP_REQUIRE(plug_n >= 1 && plug_n < (1ll << 28), "pp_dual_task_entries takes 1 .. 2^28 - 1 plug entries");
  PP_REQUIRE(n_tasks >= 1 && task_cap >= 1 && n_tasks * task_cap < (1ll << 28),
             "n_tasks * task_cap must lie in 1 .. 2^28 - 1");
  PP_REQUIRE(plug_ent && task_plug && out, "null pointer");
  hipLaunchKernelGGL(dual_task_entries_kernel, dim3((unsigned)((n_tasks * task_cap + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), plug_ent, plug_n, task_plug, n_tasks, task_cap, out);
  PP_LAUNCH_CHECK();
  return PP_OK;
}

extern "C" int pp_dual_rows(const pp_dual_proj* proj, const int64_t* task_plug, int64_t task_cap,
                            int plug_windows, int code_layout,
                            const void* scales, int64_t n_groups, int64_t group_size, int64_t chunk_size,
                            const void* scale_tab, int64_t n_tab, const float* amp_lut, const float* cos_lut,
                            const float* sin_lut, const uint32_t* plug_idx, const void* plug_amp,
                            const uint32_t* plug_ent, int64_t plug_n, int64_t M, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  PP_REQUIRE(proj != nullptr, "proj is null");
  const pp_dual_proj P = *proj;
  PP_REQUIRE(P.codes && P.x && P.out[0] && P.out[1], "null pointer in proj");
  PP_REQUIRE(P.N >= 1 && P.K >= 8 && P.K % 8 == 0 && P.K < (1 << 19) && P.ldc >= P.K && P.ldc % 8 == 0,
             "the dual row decode needs K % 8 == 0, K < 2^19 and ldc >= K, a multiple of 8");
  PP_REQUIRE(aligned(P.codes, 16) && aligned(P.x, 16) && P.pos0 >= 0 && P.pos0 % 8 == 0,
             "codes and activations must be 16-byte aligned, the position a multiple of 8");
  PP_REQUIRE(M >= 1 && M <= 4 && (M == 1 || (P.x_sm >= P.K && P.x_sm % 8 == 0)) && (M == 1 || P.o_sm >= P.N),
             "the dual row decode takes 1..4 tokens (activation rows a multiple of 8 apart)");
  PP_REQUIRE(2 * ((int64_t)(P.N - 1) * P.ldc + P.K) < (1ll << 31) && (M - 1) * P.x_sm + P.K < (1ll << 30) &&
                 (M - 1) * P.o_sm + P.N < (1ll << 30),
             "a Linear's codes, activations and outputs must each stay below 2 GiB");
  PP_REQUIRE(plug_windows == 1 || plug_windows == 2, "plug_windows must be 1 or 2");
  PP_REQUIRE(code_layout == PP_DUAL_I16_OFFSET || code_layout == PP_DUAL_U16_BE, "bad code_layout");
  PP_REQUIRE(amp_lut && cos_lut && sin_lut && (task_plug || task_cap > 0), "lut pointers or task_plug are null");
  PP_REQUIRE(task_cap >= 0, "task_cap must be 0 (plug ranges in task_plug) or the records per task");
  PP_REQUIRE(scales != nullptr && n_groups >= 1 && 2 * n_groups < (1ll << 31), "bad scales / n_groups");
  PP_REQUIRE(group_size >= 8 && (group_size & (group_size - 1)) == 0,
             "the dual row decode needs a power-of-two group_size >= 8");
  PP_REQUIRE(chunk_size >= 8 && chunk_size % 8 == 0, "the dual row decode needs chunk_size % 8 == 0");
  PP_REQUIRE(scale_tab == nullptr || (n_tab >= 1 && 2 * n_tab < (1ll << 31)), "bad scale_tab / n_tab");
  PP_REQUIRE(plug_n >= 0 && plug_n < (1ll << 28) && (plug_n == 0 || (plug_idx && plug_amp && plug_ent)),
             "plug arrays are null (plug_ent from pp_dual_plug_table)");
  const int sm = chunk_size % group_size == 0 ? (scale_tab != nullptr ? 2 : 0) : 1;
  PP_REQUIRE(sm != 2 || chunk_size % group_size == 0, "the scale table needs chunk_size % group_size == 0");
  const DualDirectPlan p = dual_direct_plan(M, P.N, P.K);
  PP_REQUIRE(p.waves < (1 << 16), "the one-Linear launch deals at most 65,535 wavefronts");
  PP_REQUIRE(p.split_bytes == 0 || (workspace != nullptr && workspace_bytes >= p.split_bytes),
             "workspace too small: need %lld bytes (pp_dual_rows_workspace_size), zero on entry",
             (long long)p.split_bytes);
  DualStreamArgs A = {};
  A.amp_lut = amp_lut;
  A.cos_lut = cos_lut;
  A.sin_lut = sin_lut;
  A.scales = reinterpret_cast<const f16*>(scales);
  A.n_groups = n_groups;
  A.scale_tab = reinterpret_cast<const f16*>(scale_tab);
  A.n_tab = n_tab;
  A.gs = group_size;
  A.chunk = chunk_size;
  A.per_chunk = (chunk_size + group_size - 1) / group_size;
  A.log2gs = 0;
  while ((1ll << A.log2gs) < group_size) ++A.log2gs;
  A.plug_idx = plug_idx;
  A.plug_amp = reinterpret_cast<const f16*>(plug_amp);
  A.plug_ent = plug_ent;
  A.plug_n = plug_n;
  A.task_plug = task_plug;
  A.n_tasks = p.n_tasks;
  if (task_cap > 0) {
    PP_REQUIRE(p.n_tasks * task_cap < (1ll << 28), "n_tasks * task_cap must stay below 2^28");
    A.task_cap = task_cap;
    A.plug_n = plug_n > 0 ? p.n_tasks * task_cap : 0;
  }
  A.M = (int)M;
  A.proj = P;
  A.parts = p.parts;
  A.n_chunks = p.n_chunks;
  A.wg_parts = p.wg ? 1 : 0;
  if (p.parts > 1 && !p.wg) {
    A.cnt = reinterpret_cast<uint32_t*>(workspace);
    A.acc = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + p.cnt_bytes);
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool be = code_layout == PP_DUAL_U16_BE;
  if (sm == 2)
    return be ? dispatch_dual_direct<PP_DUAL_U16_BE, 2>(A, p.mt, plug_windows, st)
              : dispatch_dual_direct<PP_DUAL_I16_OFFSET, 2>(A, p.mt, plug_windows, st);
  if (sm == 0)
    return be ? dispatch_dual_direct<PP_DUAL_U16_BE, 0>(A, p.mt, plug_windows, st)
              : dispatch_dual_direct<PP_DUAL_I16_OFFSET, 0>(A, p.mt, plug_windows, st);
  return be ? dispatch_dual_direct<PP_DUAL_U16_BE, 1>(A, p.mt, plug_windows, st)
            : dispatch_dual_direct<PP_DUAL_I16_OFFSET, 1>(A, p.mt, plug_windows, st);
}

// Joins a side stream back into the caller's stream on every return after the fork, so the
// caller's stream never runs ahead of the side stream's work, and a capture that forked it
// can end (a side stream left unjoined makes ending the capture fail).  finish() joins on
// the success path and reports the status; the destructor joins on the early returns.
struct SideJoin {
  hipEvent_t join = nullptr;
  hipStream_t side = nullptr, main = nullptr;
  void arm(hipEvent_t j, hipStream_t s, hipStream_t m) {
    join = j;
    side = s;
    main = m;
  }
  int finish() {
    if (join == nullptr) return PP_OK;
    const hipEvent_t j = join;
    join = nullptr;
    PP_HIP(hipEventRecord(j, side));
    PP_HIP(hipStreamWaitEvent(main, j, 0));
    return PP_OK;
  }
  ~SideJoin() {
    if (join != nullptr) {
      (void)hipEventRecord(join, side);
      (void)hipStreamWaitEvent(main, join, 0);
    }
  }
};

extern "C" int pp_dual_stream(const pp_dual_proj* projs, int64_t n_projs, const pp_quad_seg* segs, int64_t n_segs,
                              const int64_t* seg_bounds, int64_t n_waves, void* workspace, const int64_t* task_plug,
                              int64_t n_tasks,
                              int plug_windows, const pp_quad_item* tail_items,
                              int64_t n_tail, int code_layout, const void* scales, int64_t n_groups,
                              int64_t group_size, int64_t chunk_size, const void* scale_tab, int64_t n_tab,
                              const float* amp_lut, const float* cos_lut,
                              const float* sin_lut, const uint32_t* plug_idx, const void* plug_amp,
                              const uint32_t* plug_ent, int64_t plug_n,
                              int64_t n_codes, const void* const* tails, const int64_t* tail_len, int64_t M,
                              void* stream) {
  PP_REQUIRE(projs != nullptr && n_projs >= 1, "no projections");
  PP_REQUIRE(n_segs >= 0 && (n_segs == 0 || (segs != nullptr && seg_bounds != nullptr)), "segs / seg_bounds is null");
  PP_REQUIRE(n_segs == 0 || (task_plug != nullptr && n_tasks >= 1 && n_tasks < (1ll << 27)),
             "task_plug is null or n_tasks out of range");
  PP_REQUIRE(plug_windows == 1 || plug_windows == 2, "plug_windows must be 1 or 2");
  PP_REQUIRE(plug_n < (1ll << 28), "the stream decode takes fewer than 2^28 plug entries");
  PP_REQUIRE(n_tail == 0 || tail_items != nullptr, "tail_items is null");
  PP_REQUIRE(code_layout == PP_DUAL_I16_OFFSET || code_layout == PP_DUAL_U16_BE, "bad code_layout");
  PP_REQUIRE(amp_lut && cos_lut && sin_lut, "lut pointers are null");
  PP_REQUIRE(scales != nullptr && n_groups >= 1 && 2 * n_groups < (1ll << 31), "bad scales / n_groups");
  PP_REQUIRE(group_size >= 8 && (group_size & (group_size - 1)) == 0,
             "the stream decode needs a power-of-two group_size >= 8");
  PP_REQUIRE(chunk_size >= 8 && chunk_size % 8 == 0, "the stream decode needs chunk_size % 8 == 0");
  PP_REQUIRE(scale_tab == nullptr || (n_tab >= 1 && 2 * n_tab < (1ll << 31)), "bad scale_tab / n_tab");
  PP_REQUIRE(plug_n >= 0 && (plug_n == 0 || (plug_idx != nullptr && plug_amp != nullptr)), "plug arrays are null");
  PP_REQUIRE(plug_n == 0 || n_segs == 0 || plug_ent != nullptr, "plug_ent is null (build it with pp_dual_plug_table)");
  PP_REQUIRE(M >= 1 && M <= 4, "the dual stream decode takes 1..4 tokens, got %lld", (long long)M);
  PP_REQUIRE(n_segs == 0 || n_waves == pp_dual_stream_waves(M),
             "seg_bounds were built for %lld waves, this device launches %lld", (long long)n_waves,
             (long long)pp_dual_stream_waves(M));
  const int sm = chunk_size % group_size == 0 ? 0 : 1;
  PP_REQUIRE(sm == 0 || n_codes < (1ll << 32), "chunked group restarts need fewer than 2^32 positions");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int mt = dual_stream_mt(M);
  DualStreamArgs A = {};
  A.projs = projs;
  A.segs = segs;
  A.seg_bounds = seg_bounds;
  A.amp_lut = amp_lut;
  A.cos_lut = cos_lut;
  A.sin_lut = sin_lut;
  A.scales = reinterpret_cast<const f16*>(scales);
  A.n_groups = n_groups;
  A.scale_tab = reinterpret_cast<const f16*>(scale_tab);
  A.n_tab = n_tab;
  A.gs = group_size;
  A.chunk = chunk_size;
  A.per_chunk = (chunk_size + group_size - 1) / group_size;
  A.log2gs = 0;
  while ((1ll << A.log2gs) < group_size) ++A.log2gs;
  A.plug_idx = plug_idx;
  A.plug_amp = reinterpret_cast<const f16*>(plug_amp);
  A.plug_ent = plug_ent;
  A.plug_n = plug_n;
  A.task_plug = task_plug;
  A.n_tasks = n_tasks;
  A.M = (int)M;
  A.ws = workspace;
  const bool be = code_layout == PP_DUAL_U16_BE;
  // With both launches, the tail rows (fp16 streaming, little arithmetic) run on a side
  // stream beside the row kernel (bound by its decode arithmetic, not by HBM): the two write
  // disjoint rows and share no workspace.  The side stream forks from and joins back into
  // the caller's stream, so the call orders like one launch on it.
  std::unique_lock<std::mutex> side_held;
  hipStream_t tail_st = st;
  SideJoin joiner;
  if (n_segs > 0 && n_tail > 0) {
    hipEvent_t fork = nullptr, join = nullptr;
    if (int rc = side_stream(&tail_st, &fork, &join)) return rc;
    side_held = std::unique_lock<std::mutex>(side_lock());
    PP_HIP(hipEventRecord(fork, st));
    // from here on every return joins the side stream back (joiner's destructor)
    joiner.arm(join, tail_st, st);
    PP_HIP(hipStreamWaitEvent(tail_st, fork, 0));
  }
  if (n_segs > 0) {
    int rc;
    const int pw = plug_windows;
    if (sm == 0 && scale_tab != nullptr) {
      rc = be ? dispatch_dual_stream<PP_DUAL_U16_BE, 2>(A, mt, pw, st)
              : dispatch_dual_stream<PP_DUAL_I16_OFFSET, 2>(A, mt, pw, st);
    } else if (be) {
      rc = sm == 0 ? dispatch_dual_stream<PP_DUAL_U16_BE, 0>(A, mt, pw, st)
                   : dispatch_dual_stream<PP_DUAL_U16_BE, 1>(A, mt, pw, st);
    } else {
      rc = sm == 0 ? dispatch_dual_stream<PP_DUAL_I16_OFFSET, 0>(A, mt, pw, st)
                   : dispatch_dual_stream<PP_DUAL_I16_OFFSET, 1>(A, mt, pw, st);
    }
    if (rc) return rc;
  }
  if (n_tail > 0) {
    DualTailArgs T = {};
    T.projs = projs;
    T.items = tail_items;
    T.n_items = n_tail;
    T.S = A;
    T.layout = code_layout;
    T.n_codes = n_codes;
    for (int m = 0; m < 2; ++m) {
      T.tails[m] = tails ? reinterpret_cast<const f16*>(tails[m]) : nullptr;
      T.tail_len[m] = tail_len ? tail_len[m] : 0;
    }
    int rc;
    if (be) rc = sm == 0 ? dispatch_dual_tail<PP_DUAL_U16_BE, 0>(T, mt, tail_st)
                         : dispatch_dual_tail<PP_DUAL_U16_BE, 1>(T, mt, tail_st);
    else rc = sm == 0 ? dispatch_dual_tail<PP_DUAL_I16_OFFSET, 0>(T, mt, tail_st)
                      : dispatch_dual_tail<PP_DUAL_I16_OFFSET, 1>(T, mt, tail_st);
    if (rc) return rc;
  }
  return joiner.finish();
}
