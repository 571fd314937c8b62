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
// in flight while one is decoded, plug corrections / reduction / stores of a task done in
// the first step of the next.  Per lane and row a chunk is one 16-byte load (8 pairs that
// share one group scale, so the scale multiplies a per-lane partial sum once per 8 pairs)
// and one 2-byte scale load.
//
// LDS tables (136 KiB): (cos, sin) of the 1024 phases in 128-byte rows of 16 replicas,
// the 64 amplitudes in 128-byte rows of 32 replicas.  For the int16 layout the amplitude
// rows are stored at index amp_q ^ 32, so the stored bits index them directly.
#include "pp_common.h"
#include "rows_common.h"

namespace pp {

constexpr int DPAIRS = 512;                    // pairs per wave per row per chunk (64 lanes x 8)
constexpr uint32_t DLDS_CS = 0;                // (cos, sin) rows: phase p at p*128 + 8*(lane % 16)
constexpr uint32_t DLDS_AMP = 0x20000;         // amplitude rows: a at DLDS_AMP + a*128 + 4*(lane % 32)
constexpr uint32_t DLDS_BYTES = 0x20000 + 64 * 128;

template <int MT> struct DualCfg;
template <> struct DualCfg<1> { static constexpr int RG = 8, NT = 512; };
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
  int64_t gs, chunk, per_chunk;
  int log2gs;
  const uint32_t* plug_idx;
  const f16* plug_amp;
  int64_t plug_n;
  int M;
};

// Stored 32-bit word (two pairs) -> two codes in the table-index form: the file layout is
// byte-swapped per half, the int16 layout is used as stored.
template <int LAYOUT>
__device__ __forceinline__ uint32_t dual_word(uint32_t w) {
  if constexpr (LAYOUT == PP_DUAL_U16_BE) return __builtin_amdgcn_perm(w, w, 0x02030001u);
  else return w;
}
template <int LAYOUT>
__device__ __forceinline__ uint32_t dual_half(uint32_t h16) {
  if constexpr (LAYOUT == PP_DUAL_U16_BE) return ((h16 & 0xFFu) << 8) | ((h16 >> 8) & 0xFFu);
  else return h16 & 0xFFFFu;
}

struct DualLane {
  uint32_t cs, amp;   // lane offsets inside a row
};

__device__ __forceinline__ DualLane dual_lane(int l) {
  DualLane o;
  o.cs = DLDS_CS | (8u * (l & 15));
  o.amp = DLDS_AMP | (4u * (l & 31));
  return o;
}

// Table values of the code in the low 16 bits (H = 0) or the high 16 bits (H = 1) of w.
template <int H>
__device__ __forceinline__ void dual_lookup(const char* lds, uint32_t w, const DualLane& o, float& an, float2& cs) {
  const uint32_t a_cs = (H ? ((w >> 9) & 0x1FF80u) : ((w << 7) & 0x1FF80u)) | o.cs;
  const uint32_t a_amp = (H ? ((w >> 19) & 0x1F80u) : ((w >> 3) & 0x1F80u)) | o.amp;
  an = *reinterpret_cast<const float*>(lds + a_amp);
  cs = *reinterpret_cast<const float2*>(lds + a_cs);
}

template <int LAYOUT>
__device__ __forceinline__ void dual_build_lds(char* lds, const DualStreamArgs& A) {
  for (int i = threadIdx.x; i < 1024 * 16; i += blockDim.x) {
    const int p = i >> 4, j = i & 15;
    *reinterpret_cast<float2*>(lds + DLDS_CS + p * 128 + 8 * j) = make_float2(A.cos_lut[p], A.sin_lut[p]);
  }
  for (int i = threadIdx.x; i < 64 * 32; i += blockDim.x) {
    const int a = i >> 5, j = i & 31;
    const int src = LAYOUT == PP_DUAL_I16_OFFSET ? (a ^ 32) : a;
    *reinterpret_cast<float*>(lds + DLDS_AMP + a * 128 + 4 * j) = A.amp_lut[src];
  }
}

// Uniform state of a segment.
struct DualSeg {
  rsrc_t rx;
  const uint16_t* codes;
  const f16* x;
  int64_t pos0;        // stream position of the segment's first row
  int ldc, K, nrows, x_sm;
  f16* out[2];
  int64_t o_sm;
};

// Group (scale index) of stream position p.  SM = 0: chunk is a multiple of gs, so
// groups never restart mid-group and group = p / gs; SM = 1: the general rule.
template <int SM>
__device__ __forceinline__ uint32_t dual_group(const DualStreamArgs& A, int64_t p) {
  if constexpr (SM == 0) {
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
  uint32_t sc[RG];      // their group scale (fp16 bits)
  u32x4 xr[MT];         // 8 fp16 activations per lane
};

template <int MT, int RG, int SM>
__device__ __forceinline__ void dchunk_issue(const DualStreamArgs& A, const DualSeg& S, int row, int kc,
                                             const uint32_t (&voff)[RG], int lane, DChunk<MT, RG>& c) {
  const int64_t first = (int64_t)row * S.ldc + kc;
  const int64_t end = (int64_t)(S.nrows - 1) * S.ldc + S.K;
  const rsrc_t rc = make_rsrc(S.codes + first, 2u * (uint32_t)(end - first));
  const rsrc_t rs = make_rsrc(A.scales, 2u * (uint32_t)A.n_groups);
#pragma unroll
  for (int r = 0; r < RG; ++r) vload128(c.q[r], voff[r], rc);
  const int k = kc + 8 * lane;
  const int64_t base = S.pos0 + first;   // stream position of (row, kc): uniform
#pragma unroll
  for (int r = 0; r < RG; ++r) {
    const bool in = (row + r) < S.nrows && k < S.K;
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
  if constexpr (MT == 1) {
    const rsrc_t rx = make_rsrc(S.x + kc, 2u * (uint32_t)(S.K - kc));
    vload128(c.xr[0], 16u * lane, rx);
  } else {
#pragma unroll
    for (int j = 0; j < MT; ++j) vload128(c.xr[j], k < S.K ? 2u * (uint32_t)(j * S.x_sm + k) : OOB, S.rx);
  }
}

template <int MT, int RG, int LAYOUT>
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
    const uint32_t w4[4] = {dual_word<LAYOUT>(c.q[r].x), dual_word<LAYOUT>(c.q[r].y), dual_word<LAYOUT>(c.q[r].z),
                            dual_word<LAYOUT>(c.q[r].w)};
    float an[8];
    float2 cs[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dual_lookup<0>(lds, w4[e], lo, an[2 * e], cs[2 * e]);
      dual_lookup<1>(lds, w4[e], lo, an[2 * e + 1], cs[2 * e + 1]);
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
    const float sc = h2f(c.sc[r]);
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      acc[r][0][j] = fmaf(sc, l1[j], acc[r][0][j]);
      acc[r][1][j] = fmaf(sc, l2[j], acc[r][1][j]);
    }
  }
}

// Plug entries of a task (the same in-order consumption as the quad kernel).
template <int MT>
struct DPlug {
  uint32_t idx;      // position of entry pc + lane
  int row;           // row in the task, -1 when none
  uint32_t code;     // stored 16-bit code at the entry
  uint32_t sc;       // its group scale (fp16 bits)
  uint32_t pa;       // plug amplitude (fp16 bits)
  uint32_t xk[MT];   // x at its column (fp16 bits)
  bool dense;
};

__device__ __forceinline__ rsrc_t dplug_rsrc(const void* base, int64_t plug_n, int64_t pc, int esize) {
  const int64_t left = plug_n - pc;
  const uint32_t bytes = left <= 0 ? 0u : (uint32_t)std::min<int64_t>(left * esize, 0x7FFFFFF0);
  return make_rsrc(reinterpret_cast<const char*>(base) + (left > 0 ? pc : 0) * esize, bytes);
}

template <int RG>
__device__ __forceinline__ int dplug_locate(int64_t pos, int64_t tpos0, int ldc, int K, int nr, int& k) {
  const int64_t off = pos - tpos0;
  int row = 0;
#pragma unroll
  for (int r = 1; r < RG; ++r)
    if (off >= (int64_t)r * ldc) row = r;
  k = (int)(off - (int64_t)row * ldc);
  return (off >= 0 && row < nr && k < K) ? row : -1;
}

template <int MT, int RG, int SM>
__device__ __forceinline__ void dplug_begin(const DualStreamArgs& A, const DualSeg& S, int ti, int lane, int64_t& pc,
                                            DPlug<MT>& P) {
  const int64_t tpos0 = S.pos0 + (int64_t)ti * RG * S.ldc;
  const int nr = min(RG, S.nrows - ti * RG);
  const int64_t tend = tpos0 + (int64_t)nr * S.ldc;
  const bool in = (pc + lane < A.plug_n) && ((int64_t)P.idx < tend);
  const int cnt = __popcll(__ballot(in));
  int k = 0;
  const int row = in ? dplug_locate<RG>((int64_t)P.idx, tpos0, S.ldc, S.K, nr, k) : -1;
  P.row = row;
  const bool v = row >= 0;
  const int64_t first = (int64_t)ti * RG * S.ldc;
  const int64_t end = (int64_t)(S.nrows - 1) * S.ldc + S.K;
  const rsrc_t rc = make_rsrc(S.codes + first, 2u * (uint32_t)(end - first));
  vload16(P.code, v ? 2u * (uint32_t)(row * S.ldc + k) : OOB, rc);
  const uint32_t g = dual_group<SM>(A, tpos0 + (int64_t)row * S.ldc + k);
  vload16(P.sc, v ? 2u * g : OOB, make_rsrc(A.scales, 2u * (uint32_t)A.n_groups));
  vload16(P.pa, in ? 2u * lane : OOB, dplug_rsrc(A.plug_amp, A.plug_n, pc, 2));
#pragma unroll
  for (int j = 0; j < MT; ++j) vload16(P.xk[j], (v && j < A.M) ? 2u * (uint32_t)(j * S.x_sm + k) : OOB, S.rx);
  P.dense = cnt == 64;
  pc += cnt;
  vload32(P.idx, 4u * lane, dplug_rsrc(A.plug_idx, A.plug_n, pc, 4));
}

// Correction of one entry: the amplitude amp_lut[aq]*scale is replaced by the plug value.
template <int MT, int RG, int LAYOUT>
__device__ __forceinline__ void dplug_correct(const char* lds, const DualLane& lo, int row, uint32_t code16,
                                              float sc, float pa, const float (&xk)[MT], float (&acc)[RG][2][MT]) {
  float an;
  float2 cs;
  dual_lookup<0>(lds, dual_half<LAYOUT>(code16), lo, an, cs);
  const float d = pa - an * sc;
#pragma unroll
  for (int q = 0; q < RG; ++q) {
    const float on = q == row ? d : 0.f;
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const float t = on * xk[j];
      acc[q][0][j] = fmaf(t, cs.x, acc[q][0][j]);
      acc[q][1][j] = fmaf(t, cs.y, acc[q][1][j]);
    }
  }
}

template <int MT, int RG, int LAYOUT, int SM>
__device__ __forceinline__ void dplug_end(const char* lds, const DualLane& lo, const DualStreamArgs& A,
                                          const DualSeg& S, int ti, int lane, int64_t& pc, DPlug<MT>& P,
                                          float (&acc)[RG][2][MT]) {
  if (P.row >= 0) {
    float xk[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) xk[j] = h2f(P.xk[j]);
    dplug_correct<MT, RG, LAYOUT>(lds, lo, P.row, P.code, h2f(P.sc), h2f(P.pa), xk, acc);
  }
  if (!P.dense) return;
  const int64_t tpos0 = S.pos0 + (int64_t)ti * RG * S.ldc;
  const int nr = min(RG, S.nrows - ti * RG);
  const int64_t tend = tpos0 + (int64_t)nr * S.ldc;
  for (;;) {
    const int64_t q = pc + lane;
    const bool has = q < A.plug_n;
    const int64_t pos = has ? (int64_t)A.plug_idx[q] : tend;
    const bool in = pos < tend;
    const int cnt = __popcll(__ballot(in));
    int k = 0;
    const int row = in ? dplug_locate<RG>(pos, tpos0, S.ldc, S.K, nr, k) : -1;
    if (row >= 0) {
      float xk[MT];
#pragma unroll
      for (int j = 0; j < MT; ++j) xk[j] = j < A.M ? (float)S.x[(int64_t)j * S.x_sm + k] : 0.f;
      const uint32_t code = S.codes[(int64_t)(ti * RG + row) * S.ldc + k];
      const float sc = (float)A.scales[dual_group<SM>(A, pos)];
      dplug_correct<MT, RG, LAYOUT>(lds, lo, row, code, sc, (float)A.plug_amp[q], xk, acc);
    }
    pc += cnt;
    if (cnt < 64) break;
  }
  vload32(P.idx, 4u * lane, dplug_rsrc(A.plug_idx, A.plug_n, pc, 4));
  asm volatile("" : : "v"(P.idx));   // wait here, not at the next (common) use
}

template <int MT, int RG>
__device__ __forceinline__ void dtask_write(const DualStreamArgs& A, const DualSeg& S, int ti, int lane,
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
  const float y = wave_transpose_reduce<LNV>(v, lane);
  const int idx = lane >> (6 - LNV);
  const int r = idx / (2 * MT), m = (idx / MT) & 1, j = idx % MT;
  const int nr = min(RG, S.nrows - ti * RG);
  const bool wr = (lane & ((1 << (6 - LNV)) - 1)) == 0 && r < nr && j < A.M;
  const uint32_t off = 2u * (uint32_t)((int64_t)j * S.o_sm + (int64_t)(ti * RG + r));
  const uint32_t obytes = 2u * (uint32_t)((int64_t)(A.M - 1) * S.o_sm + (int64_t)S.nrows);
  const f16 h = (f16)y;
#pragma unroll
  for (int mm = 0; mm < 2; ++mm)
    vstore16((uint32_t)__builtin_bit_cast(unsigned short, h), (wr && m == mm) ? off : OOB, make_rsrc(S.out[mm], obytes));
}

template <int MT, int RG>
__device__ __forceinline__ void dzero(float (&acc)[RG][2][MT]) {
#pragma unroll
  for (int r = 0; r < RG; ++r)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[r][0][j] = acc[r][1][j] = 0.f;
}

template <int MT, int RG, int LAYOUT, int SM>
struct DualRunner {
  const char* lds;
  DualLane lo;
  const DualStreamArgs& A;
  const DualSeg& S;
  int lane, nck, ntask;
  uint32_t voff[RG];
  float acc[RG][2][MT];
  float pend[RG][2][MT];
  int pend_ti;
  DPlug<MT> P;
  int64_t pc;
  Cursor lc;

  __device__ __forceinline__ DualRunner(const char* l, const DualStreamArgs& a, const DualSeg& s, int64_t plug_lo)
      : lds(l), A(a), S(s), pend_ti(-1), pc(plug_lo) {
    lane = threadIdx.x & 63;
    lo = dual_lane(lane);
    nck = (S.K + DPAIRS - 1) / DPAIRS;
    ntask = (S.nrows + RG - 1) / RG;
    lc = {0, 0};
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

  __device__ __forceinline__ void prefetch(DChunk<MT, RG>& c) {
    dchunk_issue<MT, RG, SM>(A, S, lc.ti * RG, lc.ck * DPAIRS, voff, lane, c);
    Cursor nx = lc;
    advance(nx);
    if (nx.ti < ntask) lc = nx;
  }

  __device__ __forceinline__ void finish_pending() {
    dplug_end<MT, RG, LAYOUT, SM>(lds, lo, A, S, pend_ti, lane, pc, P, pend);
    dtask_write<MT, RG>(A, S, pend_ti, lane, pend);
    pend_ti = -1;
  }

  // prefetch | [first chunk] finish the previous task, this task's plug loads | decode |
  // [last chunk] park the sums (see SegRunner in quad_rows.hip)
  __device__ __forceinline__ bool step(Cursor& cur, DChunk<MT, RG>& comp, DChunk<MT, RG>& pref) {
    prefetch(pref);
    if (cur.ck == 0) {
      if (pend_ti >= 0) finish_pending();
      dplug_begin<MT, RG, SM>(A, S, cur.ti, lane, pc, P);
    }
    dchunk_compute<MT, RG, LAYOUT>(lds, lo, comp, acc);
    if (cur.ck == nck - 1) {
#pragma unroll
      for (int r = 0; r < RG; ++r)
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
          for (int j = 0; j < MT; ++j) pend[r][m][j] = acc[r][m][j];
      dzero<MT, RG>(acc);
      pend_ti = cur.ti;
    }
    advance(cur);
    return cur.ti < ntask;
  }

  __device__ __forceinline__ void run() {
    if (ntask <= 0 || S.K <= 0) return;
    DChunk<MT, RG> c0, c1;
    Cursor cur = {0, 0};
    vload32(P.idx, 4u * lane, dplug_rsrc(A.plug_idx, A.plug_n, pc, 4));
    prefetch(c0);
    for (;;) {
      if (!step(cur, c0, c1)) break;
      if (!step(cur, c1, c0)) break;
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
#pragma unroll
  for (int m = 0; m < 2; ++m) S.out[m] = reinterpret_cast<f16*>(uniform_ptr(P.out[m])) + row0;
  S.o_sm = uniform64(P.o_sm);
}

template <int MT, int LAYOUT, int SM>
__global__ __launch_bounds__(DualCfg<MT>::NT) void dual_stream_kernel(const DualStreamArgs A) {
  constexpr int RG = DualCfg<MT>::RG, WAVES = DualCfg<MT>::NT / 64;
  __shared__ __attribute__((aligned(16))) uint32_t T[DLDS_BYTES / 4];
  char* lds = reinterpret_cast<char*>(T);
  dual_build_lds<LAYOUT>(lds, A);
  __syncthreads();
  const int64_t gw = (int64_t)blockIdx.x * WAVES + uniform(threadIdx.x >> 6);
  const int64_t s0 = uniform64(A.seg_bounds[gw]), s1 = uniform64(A.seg_bounds[gw + 1]);
  for (int64_t si = s0; si < s1; ++si) {
    const pp_quad_seg g = A.segs[si];
    DualSeg S;
    dual_seg(A.projs[uniform(g.proj)], g.row0, g.row1, A.M, S);
    DualRunner<MT, RG, LAYOUT, SM> R(lds, A, S, uniform64(g.plug_lo));
    R.run();
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

// A row that reaches the FP16 tails, element by element: positions < n_codes decode
// from the codes (with the plug entries of the row), positions >= n_codes read
// tails[m][pos - n_codes] when model m has them.
template <int MT, int LAYOUT, int SM>
__global__ __launch_bounds__(256) void dual_tail_kernel(const DualTailArgs T) {
  const int64_t ti = (int64_t)blockIdx.x * 4 + uniform(threadIdx.x >> 6);
  if (ti >= T.n_items) return;
  const DualStreamArgs& A = T.S;
  const int lane = threadIdx.x & 63;
  const pp_quad_item it = T.items[ti];
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

// ------------------------------------------------------------------ host side
static int dual_stream_mt(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : 4; }
static int dual_stream_rg(int mt) { return mt == 1 ? DualCfg<1>::RG : mt == 2 ? DualCfg<2>::RG : DualCfg<4>::RG; }
static int dual_stream_nt(int mt) { return mt == 1 ? DualCfg<1>::NT : mt == 2 ? DualCfg<2>::NT : DualCfg<4>::NT; }

template <int MT, int LAYOUT, int SM>
static int launch_dual_stream(const DualStreamArgs& A, hipStream_t st) {
  hipLaunchKernelGGL((dual_stream_kernel<MT, LAYOUT, SM>), dim3((unsigned)device_cu_count()), dim3(DualCfg<MT>::NT),
                     0, st, A);
  PP_LAUNCH_CHECK();
  return PP_OK;
}

template <int LAYOUT, int SM>
static int dispatch_dual_stream(const DualStreamArgs& A, int mt, hipStream_t st) {
  switch (mt) {
    case 1: return launch_dual_stream<1, LAYOUT, SM>(A, st);
    case 2: return launch_dual_stream<2, LAYOUT, SM>(A, st);
    default: return launch_dual_stream<4, LAYOUT, SM>(A, st);
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

extern "C" int64_t pp_dual_stream_waves(int64_t M) {
  if (M < 1 || M > 4) return 0;
  return (int64_t)device_cu_count() * (dual_stream_nt(dual_stream_mt(M)) / 64);
}

extern "C" int pp_dual_stream(const pp_dual_proj* projs, int64_t n_projs, const pp_quad_seg* segs, int64_t n_segs,
                              const int64_t* seg_bounds, int64_t n_waves, const pp_quad_item* tail_items,
                              int64_t n_tail, int code_layout, const void* scales, int64_t n_groups,
                              int64_t group_size, int64_t chunk_size, const float* amp_lut, const float* cos_lut,
                              const float* sin_lut, const uint32_t* plug_idx, const void* plug_amp, int64_t plug_n,
                              int64_t n_codes, const void* const* tails, const int64_t* tail_len, int64_t M,
                              void* stream) {
  PP_REQUIRE(projs != nullptr && n_projs >= 1, "no projections");
  PP_REQUIRE(n_segs >= 0 && (n_segs == 0 || (segs != nullptr && seg_bounds != nullptr)), "segs / seg_bounds is null");
  PP_REQUIRE(n_tail == 0 || tail_items != nullptr, "tail_items is null");
  PP_REQUIRE(code_layout == PP_DUAL_I16_OFFSET || code_layout == PP_DUAL_U16_BE, "bad code_layout");
  PP_REQUIRE(amp_lut && cos_lut && sin_lut, "lut pointers are null");
  PP_REQUIRE(scales != nullptr && n_groups >= 1 && 2 * n_groups < (1ll << 31), "bad scales / n_groups");
  PP_REQUIRE(group_size >= 8 && (group_size & (group_size - 1)) == 0,
             "the stream decode needs a power-of-two group_size >= 8");
  PP_REQUIRE(chunk_size >= 8 && chunk_size % 8 == 0, "the stream decode needs chunk_size % 8 == 0");
  PP_REQUIRE(plug_n >= 0 && (plug_n == 0 || (plug_idx != nullptr && plug_amp != nullptr)), "plug arrays are null");
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
  A.gs = group_size;
  A.chunk = chunk_size;
  A.per_chunk = (chunk_size + group_size - 1) / group_size;
  A.log2gs = 0;
  while ((1ll << A.log2gs) < group_size) ++A.log2gs;
  A.plug_idx = plug_idx;
  A.plug_amp = reinterpret_cast<const f16*>(plug_amp);
  A.plug_n = plug_n;
  A.M = (int)M;
  const bool be = code_layout == PP_DUAL_U16_BE;
  if (n_segs > 0) {
    int rc;
    if (be) rc = sm == 0 ? dispatch_dual_stream<PP_DUAL_U16_BE, 0>(A, mt, st) : dispatch_dual_stream<PP_DUAL_U16_BE, 1>(A, mt, st);
    else rc = sm == 0 ? dispatch_dual_stream<PP_DUAL_I16_OFFSET, 0>(A, mt, st)
                      : dispatch_dual_stream<PP_DUAL_I16_OFFSET, 1>(A, mt, st);
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
    if (be) rc = sm == 0 ? dispatch_dual_tail<PP_DUAL_U16_BE, 0>(T, mt, st) : dispatch_dual_tail<PP_DUAL_U16_BE, 1>(T, mt, st);
    else rc = sm == 0 ? dispatch_dual_tail<PP_DUAL_I16_OFFSET, 0>(T, mt, st)
                      : dispatch_dual_tail<PP_DUAL_I16_OFFSET, 1>(T, mt, st);
    if (rc) return rc;
  }
  return PP_OK;
}
