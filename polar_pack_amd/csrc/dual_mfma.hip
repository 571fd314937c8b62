// Dual-pack decode GEMM for batches of 9 tokens and more on the matrix cores: one fused
// pass over the int16 (K,N) codes quantize_polar_bitpacked returns produces both models'
// outputs
//   out_m[j, n] = fp16( sum_k x[j, k] * W_m[k, n] ),   W_1 = amp cos, W_2 = amp sin,
//   amp = amp_lut[amp_q] * bmax[(k*N + n) / group_size]
// with each weight rounded to fp16 before the product, as the reference's tl.dot takes its
// operands (polar_kernels.py:60-86), plug amplitudes substituted (polar_bitpack.py:240-243),
// and no weight written to memory.
//
// Work item = 16 output columns n x 16*TT tokens x one K slice, one wavefront,
// v_mfma_f32_16x16x32_f16 (the A operand holds the weights of 16 columns n at 32
// consecutive k, the B operand x as stored):
//  * per 32-row step lane l reads the codes of column n0 + l%16 at rows k0 + 8(l/16) .. +7
//    (8 two-byte loads, 32-byte runs over 16 lanes) and their 8 group scales, looks up
//    amplitude and (cos, sin) in the dual LDS tables and rounds the two weights to fp16
//    (up to 32 tokens without a plug table, rows of 8 codes are loaded instead and the
//    weights transposed through LDS: see "Transposing loads" below);
//  * 2 models x TT token tiles of 16 x 16 fp32 sums stay in registers: two waves per SIMD
//    (8 per workgroup, one workgroup per CU: the tables take 129 KiB of LDS), so one
//    wave's decode runs beside the other's products;
//  * codes, scales and x of the next step load while a step is decoded; the walk runs in
//    whole pairs of steps with no exit between them (a step past the slice end reads x
//    through an empty buffer record, i.e. zeros).
// Plug entries replace the amplitude of their element (the table amplitude times the
// group scale); positions are read in an (N,K) frame (position ppos0 + n*pld + k: the host
// moves the (K,N) storage positions there), a window of 4 per lane.  With one K slice a
// wave writes its fp16 outputs; otherwise it adds its sums into float32 accumulators
// [m][n][j] with device-scope atomics and dual_mfma_finish_kernel writes the outputs and
// leaves zeros for the next launch.
#include "dual_lds.h"
#include "finish_tile.h"
#include "rows_common.h"

namespace pp {

typedef _Float16 dh8 __attribute__((ext_vector_type(8)));
typedef float df4 __attribute__((ext_vector_type(4)));

constexpr int DM_NT = 512;       // 8 waves, two per SIMD
constexpr int DM_WAVES = DM_NT / 64;

struct DualMfmaArgs {
  const uint16_t* codes;   // row k at codes + k*ldk (int16 (K,N) layout, stored = code ^ 0x8000)
  int64_t ldk;
  const f16* x;            // (M, K), row stride x_sm
  int64_t x_sm;
  f16* out[2];             // (M, N), row stride o_sm
  int64_t o_sm;
  int N, K, M;
  int tiles, tblocks;      // ceil(N / 16), ceil(M / (16 TT))
  int slices, ks;          // K slices of ks rows (a multiple of 64)
  const f16* scales;       // bmax, one per group_size consecutive (k*N + n)
  int64_t n_groups;
  int log2gs;
  DualLuts luts;
  const uint32_t* plug_idx;   // sorted positions in the (N,K) frame
  const f16* plug_amp;
  int64_t plug_n;
  const int64_t* row_plug;    // [n*slices + s]: first entry of (column n, slice s); N*slices + 1 entries
  int64_t ppos0, pld;
  float* acc;              // slices > 1: [2][N][M] float32, zero on entry
  int xcd_remap;
  int vec_out;             // outputs 8-byte aligned with o_sm % 4 == 0
  int gcols;               // transposing loads: N / group_size (group of (k, n) = k gcols + n / gs)
};

// Transposing loads (2 token tiles, no plug table, N % 16 == 0, N % group_size == 0,
// 16-byte aligned rows): per 32-row step lane l loads the 8 codes of row k0 + l/2 at columns
// n0 + 8(l%2) .. +7 (one 16-byte load) and their one group scale, decodes them and writes
// the 16 fp16 weights of each model into the wave's LDS area transposed ([n][k], rows of
// DM_TROW bytes); the A operands are then one 16-byte LDS read per model.  This replaces
// 8 two-byte code loads and 8 scale loads per lane and step.
constexpr int DM_TROW = 80;                 // bytes per n row (32 k of fp16 + 16 padding: spreads the banks)
constexpr int DM_TMODEL = 16 * DM_TROW;     // one model's 16 x 32 block
constexpr int DM_TWAVE = 2 * DM_TMODEL;     // per wave
constexpr uint32_t DM_LDS_BYTES = DLDS_BYTES + DM_WAVES * DM_TWAVE;

template <int TT>
struct DmStage {
  uint32_t c[8];           // 8 stored codes of the lane's column (low 16 bits)
  uint32_t sc[8];          // their group scales (fp16 bits)
  u32x4 cq;                // transposing loads: 8 stored codes of the lane's row
  uint32_t sq;             // and their group scale
  u32x4 xb[TT];            // 8 fp16 x of token 16t + l%16
};

// The lane's window of 4 plug entries of its column: rows (INT_MAX past the end, INT_MIN
// once applied) and amplitudes.
struct DmPlug {
  int k[4];
  float a[4];
  int64_t next, end;
};

template <class Args>
__device__ __forceinline__ void dplug_load(const Args& A, DmPlug& P, int64_t rowpos) {
  const rsrc_t ri = make_rsrc(A.plug_idx, 4u * (uint32_t)A.plug_n);
  const rsrc_t ra = make_rsrc(A.plug_amp, 2u * (uint32_t)A.plug_n);
  uint32_t idx[4], am[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t e = P.next + i;
    const bool has = e < P.end;
    vload32(idx[i], has ? 4u * (uint32_t)e : OOB, ri);
    vload16(am[i], has ? 2u * (uint32_t)e : OOB, ra);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    P.k[i] = P.next + i < P.end ? (int)((int64_t)idx[i] - rowpos) : 0x7FFFFFFF;
    P.a[i] = h2f(am[i]);
  }
  P.next += 4;
}

// Substitute the window's entries in the lane's rows kk .. kk+7 (step rows ks .. ks+31)
// into the amplitudes; refill a window used up within the step.  Wave-uniform control.
template <class Args>
__device__ __forceinline__ void dplug_patch(const Args& A, DmPlug& P, int64_t rowpos, int kk, int ks,
                                            float (&amp)[8]) {
  for (;;) {
    int hit = -1;
#pragma unroll
    for (int i = 3; i >= 0; --i) hit = (unsigned)(P.k[i] - kk) < 8u ? i : hit;
    if (__ballot(hit >= 0)) {
      const int e = hit >= 0 ? (hit == 0 ? P.k[0] : hit == 1 ? P.k[1] : hit == 2 ? P.k[2] : P.k[3]) - kk : -1;
      const float v = hit == 0 ? P.a[0] : hit == 1 ? P.a[1] : hit == 2 ? P.a[2] : P.a[3];
#pragma unroll
      for (int ee = 0; ee < 8; ++ee) amp[ee] = e == ee ? v : amp[ee];
#pragma unroll
      for (int i = 0; i < 4; ++i) P.k[i] = hit == i ? (int)0x80000000 : P.k[i];
      continue;
    }
    const bool refill = P.k[3] < ks + 32 && P.next < P.end;
    if (!__ballot(refill)) break;
    DmPlug R = P;
    dplug_load(A, R, rowpos);
    if (refill) P = R;
  }
}

// Issue the loads of the step at row k0 (codes clamped to the last step; x of a step at or
// past the slice end ke through an empty record).  voc: the lane's code offset (OOB past
// N), the 8 rows 2*ldk bytes apart in the scalar operand; gbase: group index of (k0 = 0,
// the lane's column); vox: x offsets per token tile.
template <int TT, bool TL>
__device__ __forceinline__ void dm_issue(const DualMfmaArgs& A, int n0, int n, bool ok, int q, int k0, int ke,
                                         uint32_t voc, uint32_t vos, const uint32_t (&vox)[TT], const f16* xblk,
                                         int j0, DmStage<TT>& S) {
  const uint32_t xrec = k0 < ke ? 2u * (uint32_t)((int64_t)(A.M - 1 - j0) * A.x_sm + (ke - k0)) : 0u;
  k0 = min(k0, A.K - 32);
  const rsrc_t rc = make_rsrc(A.codes + (int64_t)k0 * A.ldk + n0,
                              2u * (uint32_t)((int64_t)(A.K - 1 - k0) * A.ldk + (A.N - n0)));
  if constexpr (TL) {
    // voc: the lane's row and 8 columns; vos: its group in the step's first row
    S.cq = __builtin_amdgcn_raw_buffer_load_b128(rc, (int)voc, 0, NT_AUX);
    const int64_t g0 = (int64_t)k0 * A.gcols;
    vload16(S.sq, vos, make_rsrc(A.scales + g0, 2u * (uint32_t)(A.n_groups - g0)));
  } else {
    const int st = (int)(2 * A.ldk);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      S.c[e] = __builtin_amdgcn_raw_buffer_load_b16(rc, (int)voc, e * st, NT_AUX);
    const rsrc_t rs = make_rsrc(A.scales, 2u * (uint32_t)A.n_groups);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t g = ((int64_t)(k0 + 8 * q + e) * A.N + n) >> A.log2gs;
      vload16(S.sc[e], ok ? 2u * (uint32_t)g : OOB, rs);
    }
  }
  const rsrc_t rx = make_rsrc(xblk + min(k0, A.K - 32), xrec);
#pragma unroll
  for (int t = 0; t < TT; ++t) vload128c(S.xb[t], vox[t], rx);
}

template <int TT, bool PLUG, bool TL>
struct DmRun {
  const char* lds;
  DualLane lo;
  const DualMfmaArgs& A;
  const f16* xblk;
  int n0, n, j0, q, ke;
  bool ok;
  uint32_t voc, vos;
  uint32_t vox[TT];
  char* tw;                // TL: the wave's transpose area
  uint32_t twr, twa;       // TL: the lane's write offset (row k, first of its 8 columns), read offset
  int64_t rowpos;
  DmPlug P;
  df4 C[2][TT];

  // Consume the step at k0 from cur while the step at k0 + 32 loads into nxt.
  __device__ __forceinline__ void step(const DmStage<TT>& cur, DmStage<TT>& nxt, int k0) {
    dm_issue<TT, TL>(A, n0, n, ok, q, k0 + 32, ke, voc, vos, vox, xblk, j0, nxt);
    dh8 a0, a1;
    if constexpr (TL) {
      const float sc = h2f(cur.sq);
      const uint32_t w4[4] = {cur.cq.x, cur.cq.y, cur.cq.z, cur.cq.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float an[2];
        float2 cs[2];
        dual_lookup2<PP_DUAL_I16_OFFSET>(lds, w4[e], lo, an, cs);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float amp = an[h] * sc;
          // the weights are rounded as the reference rounds them, the float32 product then
          // fp16: the products are hidden from the compiler, which would otherwise fold
          // product and conversion into one mixed-precision multiply that rounds once
          float w1 = amp * cs[h].x, w2 = amp * cs[h].y;
          asm volatile("" : "+v"(w1), "+v"(w2));
          const uint32_t o = twr + (2 * e + h) * DM_TROW;
          *reinterpret_cast<_Float16*>(tw + o) = (_Float16)w1;
          *reinterpret_cast<_Float16*>(tw + DM_TMODEL + o) = (_Float16)w2;
        }
      }
      // the reads below take values other lanes wrote: wait until the writes are done
      // (lgkmcnt(0); vmcnt and expcnt left at their maxima, so the loads in flight are not
      // waited for)
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_wave_barrier();
      a0 = *reinterpret_cast<const dh8*>(tw + twa);
      a1 = *reinterpret_cast<const dh8*>(tw + DM_TMODEL + twa);
      __builtin_amdgcn_wave_barrier();
    } else {
      float amp[8];
      float2 cs[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float an;
        dual_lookup1(lds, cur.c[e] & 0xFFFFu, lo, an, cs[e]);
        amp[e] = an * h2f(cur.sc[e]);
      }
      if constexpr (PLUG) dplug_patch(A, P, rowpos, k0 + 8 * q, k0, amp);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        a0[e] = (_Float16)(amp[e] * cs[e].x);
        a1[e] = (_Float16)(amp[e] * cs[e].y);
      }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const dh8 b = __builtin_bit_cast(dh8, cur.xb[t]);
      C[0][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b, C[0][t], 0, 0, 0);
      C[1][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b, C[1][t], 0, 0, 0);
    }
  }
};

template <int TT, bool PLUG, bool TL>
__device__ __forceinline__ void dm_body(char* lds, const DualMfmaArgs& A) {
  const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
  const DualLane lo = dual_lane(lane);
  int b = blockIdx.x;
  if (A.xcd_remap) b = (b & 7) * (int)(gridDim.x >> 3) + (b >> 3);
  const int64_t gw = (int64_t)b * DM_WAVES + uniform(threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * DM_WAVES;
  // groups of DM_WAVES column tiles sharing a token block and K slice, one per workgroup
  const int64_t tgroups = (A.tiles + DM_WAVES - 1) / DM_WAVES;
  const int64_t items = tgroups * DM_WAVES * A.tblocks * A.slices;
  for (int64_t it = gw; it < items; it += nw) {
    const int64_t w = uniform64(it / DM_WAVES);
    const int tile = (int)(uniform64(w / ((int64_t)A.slices * A.tblocks)) * DM_WAVES + it % DM_WAVES);
    const int sl = (int)(w % A.slices), tb = (int)((w / A.slices) % A.tblocks);
    if (tile >= A.tiles) continue;
    const int n0 = tile * 16, j0 = tb * 16 * TT;
    const int kb = sl * A.ks, ke = min(A.K, kb + A.ks);
    const int n = n0 + i;
    const bool ok = n < A.N;
    DmRun<TT, PLUG, TL> R{lds, lo, A, A.x + (int64_t)j0 * A.x_sm, n0, n, j0, q, ke, ok};
    if constexpr (TL) {
      // lane l: row k0 + l/2 of the step, columns n0 + 8(l%2) .. +7 (N % 16 == 0: all in range)
      const int kr = lane >> 1, nh = 8 * (lane & 1);
      R.voc = 2u * (uint32_t)(kr * A.ldk + nh);
      R.vos = 2u * (uint32_t)(kr * A.gcols + ((n0 + nh) >> A.log2gs));
      R.tw = lds + DLDS_BYTES + uniform(threadIdx.x >> 6) * DM_TWAVE;
      R.twr = (uint32_t)(nh * DM_TROW + 2 * kr);
      R.twa = (uint32_t)(i * DM_TROW + 16 * q);
    } else {
      R.voc = ok ? 2u * (uint32_t)(8 * q * A.ldk + i) : OOB;
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const int jl = 16 * t + i;
      R.vox[t] = j0 + jl < A.M ? 2u * (uint32_t)(jl * A.x_sm + 8 * q) : OOB;
    }
    if constexpr (PLUG) {
      R.rowpos = A.ppos0 + (int64_t)n * A.pld;
      R.P.next = ok ? A.row_plug[(int64_t)n * A.slices + sl] : 0;
      R.P.end = ok ? A.row_plug[(int64_t)n * A.slices + sl + 1] : 0;
      dplug_load(A, R.P, R.rowpos);
    }
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int t = 0; t < TT; ++t) R.C[m][t] = df4{0.f, 0.f, 0.f, 0.f};
    DmStage<TT> S0, S1;
    dm_issue<TT, TL>(A, n0, n, ok, q, kb, ke, R.voc, R.vos, R.vox, R.xblk, j0, S0);
    for (int k0 = kb; k0 < ke; k0 += 64) {
      R.step(S0, S1, k0);
      R.step(S1, S0, k0 + 32);
    }
    // epilogue: lane holds columns n0 + 4q + r, r = 0..3, of token j0 + 16t + i
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const int j = j0 + 16 * t + i;
        const int nn = n0 + 4 * q;
        const df4 c = R.C[m][t];
        if (j >= A.M || nn >= A.N) continue;
        if (A.slices == 1) {
          f16* o = A.out[m] + (int64_t)j * A.o_sm + nn;
          if (A.vec_out && nn + 3 < A.N) {
            const f16x4 h = {(f16)c[0], (f16)c[1], (f16)c[2], (f16)c[3]};
            *reinterpret_cast<f16x4*>(o) = h;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (nn + r < A.N) o[r] = (f16)c[r];
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (nn + r < A.N)
              __hip_atomic_fetch_add(A.acc + ((int64_t)m * A.N + nn + r) * A.M + j, c[r], __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        }
      }
  }
}

template <int TT>
__global__ __launch_bounds__(DM_NT) __attribute__((amdgpu_waves_per_eu(2, 2))) void dual_mfma_kernel(
    const DualMfmaArgs A) {
  __shared__ __attribute__((aligned(16))) char T[DM_LDS_BYTES];
  if (A.luts.dtype == PP_F16) dual_tables_of<DM_NT, PP_DUAL_I16_OFFSET, f16>(T, A.luts);
  else dual_tables_of<DM_NT, PP_DUAL_I16_OFFSET, float>(T, A.luts);
  // transposing loads for 2 token tiles (up to 32 tokens): 33.0-33.4 against 35.2-36.7 us
  // on the 4096 x 4096 layer at 8 tokens; with 4 tiles they measured slower (47 -> 51 us
  // at 64 tokens), the LDS round trip no longer hidden behind the products
  if constexpr (TT == 2) {
    if (A.gcols > 0) {
      dm_body<TT, false, true>(T, A);
      return;
    }
  }
  if (A.plug_n > 0) dm_body<TT, true, false>(T, A);
  else dm_body<TT, false, false>(T, A);
}

// ------------------------------------------------------------ producer/consumer form
// From 65 tokens on the rows the transposing loads take (no plug table, N % 16 == 0, N a
// multiple of the group size, 16-byte aligned rows): a workgroup of 8 waves takes 64 output
// columns x a block of 64 TT tokens (TT = 2 or 4, dpc_tt) x one K slice.  Waves 0-3 decode
// (producers): per 32-row super-step wave p loads column tile p's 16 columns x 32 rows (lane
// l: row l/2, columns 8(l%2) .. +7, one 16-byte load and one group scale, codes loaded
// DPC_G super-steps ahead), decodes them as the transposing loads do and stores the two
// models' fp16 weights transposed into LDS as the MFMA A operands.  Waves 4-7 multiply
// (consumers): wave c takes the TT token tiles 16 TT c .. of the block with the previous
// super-step's 4 x 2 operands.  One of each per SIMD, so a SIMD's decode and its products
// come from two waves; two 8 KiB operand buffers alternate with one barrier per
// super-step.  Each code is decoded once per 64 TT tokens (the one-wave form: once per 16
// TT, with its x reloaded by every 16-column tile).
#ifndef PP_DPC_G
#define PP_DPC_G 4
#endif
constexpr int DPC_COLS = 64, DPC_G = PP_DPC_G, DPC_NT = 512;
// An operand block (one column tile, one model) holds lane l's 16 bytes at slot l + l / 8
// (16 bytes of padding after every 8 lanes), so the producers' 2-byte stores of one
// instruction, which go to lanes 8 and 16 apart, fall in different banks.
#ifndef PP_DPC_PAD
#define PP_DPC_PAD 1
#endif
constexpr uint32_t DPC_MBLK = PP_DPC_PAD ? 72 * 16 : 64 * 16;
constexpr uint32_t DPC_ABUF = DLDS_BYTES, DPC_ABYTES = 8 * DPC_MBLK;   // [tile 4][model 2] blocks
constexpr uint32_t DPC_LDS = DPC_ABUF + 2 * DPC_ABYTES;
static_assert(DPC_LDS <= 160 * 1024, "the tables and both operand buffers must fit in LDS");

__device__ __forceinline__ uint32_t dpc_slot(int lane) { return 16u * (uint32_t)(lane + (PP_DPC_PAD ? lane >> 3 : 0)); }
__device__ __forceinline__ uint32_t dpc_aoff(int buf, int ct, int m, int lane) {
  return DPC_ABUF + (uint32_t)buf * DPC_ABYTES + (uint32_t)(ct * 2 + m) * DPC_MBLK + dpc_slot(lane);
}

// Super-steps of a slice, rounded up to whole rounds of DPC_G (the producers' code
// buffers rotate with the super-step; super-steps past the slice read zero codes and x).
__device__ __forceinline__ int dpc_steps(int kb, int ke) { return ((ke - kb + 31) / 32 + DPC_G - 1) / DPC_G * DPC_G; }

struct DpcCodes {
  u32x4 c;                 // 8 stored codes of the lane's row
  uint32_t sc;             // their group scale (fp16 bits)
};

__device__ __forceinline__ void dpc_load(const DualMfmaArgs& A, int n0, bool ok, int k0, int ke, uint32_t voc,
                                         uint32_t vos, DpcCodes& C) {
  const bool live = ok && k0 < ke;
  const int kc = min(k0, A.K - 32);
  const rsrc_t rc = make_rsrc(A.codes + (int64_t)kc * A.ldk + n0,
                              live ? 2u * (uint32_t)((int64_t)(A.K - 1 - kc) * A.ldk + (A.N - n0)) : 0u);
  C.c = __builtin_amdgcn_raw_buffer_load_b128(rc, (int)voc, 0, NT_AUX);
  const int64_t g0 = (int64_t)kc * A.gcols;
  vload16(C.sc, vos, make_rsrc(A.scales + g0, live ? 2u * (uint32_t)(A.n_groups - g0) : 0u));
}

__device__ __forceinline__ void dpc_producer(char* lds, const DualMfmaArgs& A, int p, int n0b, int kb, int ke) {
  const int lane = threadIdx.x & 63;
  const DualLane lo = dual_lane(lane);
  const int kr = lane >> 1, nh = 8 * (lane & 1);
  const int n0 = n0b + 16 * p;
  const bool ok = n0 < A.N;              // N % 16 == 0: a column tile is whole or past N
  const uint32_t voc = 2u * (uint32_t)(kr * A.ldk + nh);
  const uint32_t vos = 2u * (uint32_t)(kr * A.gcols + ((min(n0, A.N - 16) + nh) >> A.log2gs));
  // the lane's 8 weights of row kr go to operand lanes nh + j + 16 (kr / 8), element kr % 8
  // (j < 8: their slots are consecutive)
  const uint32_t wofs = dpc_slot(nh + 16 * (kr >> 3)) + 2u * (uint32_t)(kr & 7);
  const int ns = dpc_steps(kb, ke);
  DpcCodes C[DPC_G];
#pragma unroll
  for (int g = 0; g + 1 < DPC_G; ++g) dpc_load(A, n0, ok, kb + 32 * g, ke, voc, vos, C[g]);
  auto decode = [&](const DpcCodes& c, int s) {
    const float sc = h2f(c.sc);
    const uint32_t w4[4] = {c.c.x, c.c.y, c.c.z, c.c.w};
    char* dst = lds + dpc_aoff(s & 1, p, 0, 0) + wofs;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float an[2];
      float2 cs[2];
      dual_lookup2<PP_DUAL_I16_OFFSET>(lds, w4[e], lo, an, cs);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float amp = an[h] * sc;
        // the float32 product, then fp16, as the reference rounds its operands (hidden from
        // the compiler, which would fold the two into one mixed-precision multiply)
        float w1 = amp * cs[h].x, w2 = amp * cs[h].y;
        asm volatile("" : "+v"(w1), "+v"(w2));
        *reinterpret_cast<_Float16*>(dst + 16 * (2 * e + h)) = (_Float16)w1;
        *reinterpret_cast<_Float16*>(dst + DPC_MBLK + 16 * (2 * e + h)) = (_Float16)w2;
      }
    }
  };
  // C[k % G] holds super-step k.  Prologue: super-step 0 into operand buffer 0, its code
  // buffer refilled with super-step G.
  dpc_load(A, n0, ok, kb + 32 * (DPC_G - 1), ke, voc, vos, C[DPC_G - 1]);
  decode(C[0], 0);
  dpc_load(A, n0, ok, kb + 32 * DPC_G, ke, voc, vos, C[0]);
  __syncthreads();
  for (int s = 0; s < ns; s += DPC_G) {
#pragma unroll
    for (int g = 0; g < DPC_G; ++g) {
      // while the consumers multiply super-step s + g, decode d = s + g + 1 into the other
      // operand buffer and refill its code buffer with d + G
      const int d = s + g + 1;
      decode(C[(g + 1) % DPC_G], d);
      dpc_load(A, n0, ok, kb + 32 * (d + DPC_G), ke, voc, vos, C[(g + 1) % DPC_G]);
      __syncthreads();
    }
  }
}

template <int TT>
__device__ __forceinline__ void dpc_consumer(const char* lds, const DualMfmaArgs& A, int c, int n0b, int j0b, int kb,
                                             int ke) {
  const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
  const int j0 = j0b + 16 * TT * c;
  const int jx = min(j0, A.M - 1);
  const f16* xblk = A.x + (int64_t)jx * A.x_sm;
  uint32_t vox[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int jl = 16 * t + i;
    vox[t] = j0 + jl < A.M ? 2u * (uint32_t)(jl * A.x_sm + 8 * q) : OOB;
  }
  const int ns = dpc_steps(kb, ke);
  df4 Cacc[4][2][TT];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int t = 0; t < TT; ++t) Cacc[ct][m][t] = df4{0.f, 0.f, 0.f, 0.f};
  u32x4 X[2][TT];
  auto loadx = [&](u32x4(&xb)[TT], int s) {
    const int k0 = kb + 32 * s;
    const uint32_t rec = k0 < ke ? 2u * (uint32_t)((int64_t)(A.M - 1 - jx) * A.x_sm + (ke - k0)) : 0u;
    const rsrc_t rx = make_rsrc(xblk + min(k0, A.K - 32), rec);
#pragma unroll
    for (int t = 0; t < TT; ++t) vload128c(xb[t], vox[t], rx);
  };
  // the 8 operands of a super-step are read in 4 pairs (column tile) of the 2 models; pair
  // ct + 1 is requested before pair ct's products
  auto multiply = [&](const u32x4(&xb)[TT], int s) {
    dh8 a[2][2];
#pragma unroll
    for (int m = 0; m < 2; ++m) a[0][m] = *reinterpret_cast<const dh8*>(lds + dpc_aoff(s & 1, 0, m, lane));
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      if (ct < 3) {
#pragma unroll
        for (int m = 0; m < 2; ++m)
          a[(ct + 1) & 1][m] = *reinterpret_cast<const dh8*>(lds + dpc_aoff(s & 1, ct + 1, m, lane));
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int t = 0; t < TT; ++t)
          Cacc[ct][m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[ct & 1][m], __builtin_bit_cast(dh8, xb[t]),
                                                                  Cacc[ct][m][t], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  loadx(X[0], 0);
  __syncthreads();
  // the fences keep the next super-step's x loads issued ahead of this one's products
  for (int s = 0; s < ns; s += 2) {
    loadx(X[1], s + 1);
    __builtin_amdgcn_sched_barrier(0);
    multiply(X[0], s);
    __syncthreads();
    loadx(X[0], s + 2);
    __builtin_amdgcn_sched_barrier(0);
    multiply(X[1], s + 1);
    __syncthreads();
  }
  // lane holds columns n0b + 16 ct + 4q + r, r = 0..3, of token j0 + 16t + i
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const int j = j0 + 16 * t + i;
        const int nn = n0b + 16 * ct + 4 * q;
        const df4 v = Cacc[ct][m][t];
        if (j >= A.M || nn >= A.N) continue;
        if (A.slices == 1) {
          f16* o = A.out[m] + (int64_t)j * A.o_sm + nn;
          if (A.vec_out) {    // N % 16 == 0: the 4 columns are in range
            const f16x4 h = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
            *reinterpret_cast<f16x4*>(o) = h;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) o[r] = (f16)v[r];
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            __hip_atomic_fetch_add(A.acc + ((int64_t)m * A.N + nn + r) * A.M + j, v[r], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
      }
}

template <int TT>
__global__ __launch_bounds__(DPC_NT) void dual_pc_kernel(const DualMfmaArgs A) {
  __shared__ __attribute__((aligned(16))) char T[DPC_LDS];
  if (A.luts.dtype == PP_F16) dual_tables_of<DPC_NT, PP_DUAL_I16_OFFSET, f16>(T, A.luts);
  else dual_tables_of<DPC_NT, PP_DUAL_I16_OFFSET, float>(T, A.luts);
  const int wave = uniform(threadIdx.x >> 6);
  int b = blockIdx.x;
  if (A.xcd_remap) b = (b & 7) * (int)(gridDim.x >> 3) + (b >> 3);
  // items ordered slice, token block, column block: consecutive workgroups (one XCD after
  // the remap) share token blocks (x) and slices
  const int cblocks = (A.N + DPC_COLS - 1) / DPC_COLS;
  const int64_t items = (int64_t)cblocks * A.tblocks * A.slices;
  for (int64_t it = b; it < items; it += gridDim.x) {
    const int cb = (int)uniform64(it % cblocks);
    const int64_t w = it / cblocks;
    const int tb = (int)uniform64(w % A.tblocks), sl = (int)uniform64(w / A.tblocks);
    const int n0b = cb * DPC_COLS, j0b = tb * 64 * TT;
    const int kb = sl * A.ks, ke = min(A.K, kb + A.ks);
    if (wave < 4) dpc_producer(T, A, wave, n0b, kb, ke);
    else dpc_consumer<TT>(T, A, wave - 4, n0b, j0b, kb, ke);
  }
}

// Sliced launches: out_m[j, n] = fp16(acc[m][n][j]), acc left zero (finish_tile).
__global__ __launch_bounds__(256) void dual_mfma_finish_kernel(float* acc, f16* o0, f16* o1, int64_t o_sm, int N,
                                                               int M, bool vec) {
  int m, n0, j0;
  finish_coords(N, M, m, n0, j0);
  finish_tile(acc + (int64_t)m * N * M, m == 0 ? o0 : o1, o_sm, N, M, n0, j0, vec);
}

// ------------------------------------------------------------ (N,K) container rows
// The same product over the rows of a .dualpack stream: codes (N,K) row-major (row n at
// codes + n*ldc, K contiguous), 16-bit pairs in the file's byte order (or the int16
// layout), group scales by the container rule on the stream position p = elem_base +
// n*ldc + k: g = (p / chunk) * ceil(chunk / gs) + (p % chunk) / gs (polar_bitpack.py:201-203,
// 224-238).  Per 32-column step lane l reads row n0 + l%16 at columns k0 + 8(l/16) .. +7:
// one 16-byte load of 8 codes, which is the A operand's own layout (no transpose), and one
// group scale (elem_base, ldc, the chunk size and gs are multiples of 8, so the 8 codes
// share a group).  The lane keeps the chunk index and offset of its next load position and
// advances them by 32 per step: no division in the loop.  Plug entries are stream
// positions; the window logic, slices, epilogue and finish pass are dual_mfma_kernel's.
struct DualNkArgs {
  const uint16_t* codes;   // row n at codes + n*ldc
  int64_t ldc;
  int64_t elem_base;       // stream position of (row 0, column 0)
  const f16* x;            // (M, K), row stride x_sm
  int64_t x_sm;
  f16* out[2];             // (M, N), row stride o_sm
  int64_t o_sm;
  int N, K, M;
  int tiles, tblocks;      // ceil(N / 16), ceil(M / (16 TT))
  int slices, ks;          // K slices of ks columns (a multiple of 64)
  const f16* scales;       // the stream's group scales
  int64_t n_groups;
  int chunk;               // chunk size (>= 32, a multiple of 8)
  int64_t gpc;             // groups per chunk, ceil(chunk / gs)
  int log2gs;
  DualLuts luts;
  const uint32_t* plug_idx;   // sorted stream positions
  const f16* plug_amp;
  int64_t plug_n;
  const int64_t* row_plug;    // [n*slices + s]: first entry of (row n, slice s); N*slices + 1 entries
  float* acc;              // slices > 1: [2][N][M] float32, zero on entry
  int xcd_remap;
  int vec_out;
};

template <int TT>
struct DnStage {
  u32x4 c;                 // 8 stored codes of the lane's row
  uint32_t sc;             // their group scale (fp16 bits)
  u32x4 xb[TT];            // 8 fp16 x of token 16t + l%16
};

// The chunk index and offset of a lane's position.
struct DnPos {
  int64_t c;
  int r;
  __device__ __forceinline__ void set(int64_t p, int chunk) {
    c = p / chunk;
    r = (int)(p - c * chunk);
  }
  __device__ __forceinline__ void advance32(int chunk) {   // chunk >= 32
    r += 32;
    const bool w = r >= chunk;
    r = w ? r - chunk : r;
    c += w ? 1 : 0;
  }
};

// Issue the loads of the step at column k0 (codes clamped to the last step; x of a step at
// or past the slice end ke through an empty record) and advance the scale position.
template <int TT>
__device__ __forceinline__ void dn_issue(const DualNkArgs& A, const uint16_t* ctile, int nrows, uint32_t voc, bool ok,
                                         DnPos& pos, int k0, int ke, const uint32_t (&vox)[TT], const f16* xblk,
                                         int j0, DnStage<TT>& S) {
  const uint32_t xrec = k0 < ke ? 2u * (uint32_t)((int64_t)(A.M - 1 - j0) * A.x_sm + (ke - k0)) : 0u;
  k0 = min(k0, A.K - 32);
  const rsrc_t rc = make_rsrc(ctile + k0, 2u * (uint32_t)((int64_t)(nrows - 1) * A.ldc + (A.K - k0)));
  S.c = __builtin_amdgcn_raw_buffer_load_b128(rc, (int)voc, 0, NT_AUX);
  const int64_t g = pos.c * A.gpc + (pos.r >> A.log2gs);
  vload16(S.sc, ok ? 2u * (uint32_t)g : OOB, make_rsrc(A.scales, 2u * (uint32_t)A.n_groups));
  pos.advance32(A.chunk);
  const rsrc_t rx = make_rsrc(xblk + k0, xrec);
#pragma unroll
  for (int t = 0; t < TT; ++t) vload128c(S.xb[t], vox[t], rx);
}

template <int TT, int LAYOUT, bool PLUG>
struct DnRun {
  const char* lds;
  DualLane lo;
  const DualNkArgs& A;
  const uint16_t* ctile;
  const f16* xblk;
  int nrows, j0, q, ke;
  bool ok;
  uint32_t voc;
  uint32_t vox[TT];
  DnPos pos;
  int64_t rowpos;
  DmPlug P;
  df4 C[2][TT];

  // Consume the step at k0 from cur while the step at k0 + 32 loads into nxt.
  __device__ __forceinline__ void step(const DnStage<TT>& cur, DnStage<TT>& nxt, int k0) {
    dn_issue<TT>(A, ctile, nrows, voc, ok, pos, k0 + 32, ke, vox, xblk, j0, nxt);
    const float sc = h2f(cur.sc);
    const uint32_t w4[4] = {cur.c.x, cur.c.y, cur.c.z, cur.c.w};
    float amp[8];
    float2 cs[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float an[2];
      float2 c2[2];
      dual_lookup2<LAYOUT>(lds, w4[e], lo, an, c2);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        amp[2 * e + h] = an[h] * sc;
        cs[2 * e + h] = c2[h];
      }
    }
    if constexpr (PLUG) dplug_patch(A, P, rowpos, k0 + 8 * q, k0, amp);
    dh8 a0, a1;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // the float32 product, then fp16, as the reference rounds the weights: hidden from the
      // compiler, which would otherwise fold product and conversion into one multiply
      float w1 = amp[e] * cs[e].x, w2 = amp[e] * cs[e].y;
      asm volatile("" : "+v"(w1), "+v"(w2));
      a0[e] = (_Float16)w1;
      a1[e] = (_Float16)w2;
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const dh8 b = __builtin_bit_cast(dh8, cur.xb[t]);
      C[0][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b, C[0][t], 0, 0, 0);
      C[1][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b, C[1][t], 0, 0, 0);
    }
  }
};

template <int TT, int LAYOUT, bool PLUG>
__device__ __forceinline__ void dn_body(const char* lds, const DualNkArgs& A) {
  const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
  const DualLane lo = dual_lane(lane);
  int b = blockIdx.x;
  if (A.xcd_remap) b = (b & 7) * (int)(gridDim.x >> 3) + (b >> 3);
  const int64_t gw = (int64_t)b * DM_WAVES + uniform(threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * DM_WAVES;
  // groups of DM_WAVES row tiles sharing a token block and K slice, one per workgroup
  const int64_t tgroups = (A.tiles + DM_WAVES - 1) / DM_WAVES;
  const int64_t items = tgroups * DM_WAVES * A.tblocks * A.slices;
  for (int64_t it = gw; it < items; it += nw) {
    const int64_t w = uniform64(it / DM_WAVES);
    const int tile = (int)(uniform64(w / ((int64_t)A.slices * A.tblocks)) * DM_WAVES + it % DM_WAVES);
    const int sl = (int)(w % A.slices), tb = (int)((w / A.slices) % A.tblocks);
    if (tile >= A.tiles) continue;
    const int n0 = tile * 16, j0 = tb * 16 * TT;
    const int kb = sl * A.ks, ke = min(A.K, kb + A.ks);
    const int n = n0 + i;
    const bool ok = n < A.N;
    const int nrows = min(16, A.N - n0);
    DnRun<TT, LAYOUT, PLUG> R{lds, lo, A, A.codes + (int64_t)n0 * A.ldc, A.x + (int64_t)j0 * A.x_sm, nrows, j0, q,
                              ke, ok};
    R.voc = ok ? 2u * (uint32_t)(i * A.ldc + 8 * q) : OOB;
    R.rowpos = A.elem_base + (int64_t)min(n, A.N - 1) * A.ldc;
    R.pos.set(R.rowpos + kb + 8 * q, A.chunk);
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const int jl = 16 * t + i;
      R.vox[t] = j0 + jl < A.M ? 2u * (uint32_t)(jl * A.x_sm + 8 * q) : OOB;
    }
    if constexpr (PLUG) {
      R.P.next = ok ? A.row_plug[(int64_t)n * A.slices + sl] : 0;
      R.P.end = ok ? A.row_plug[(int64_t)n * A.slices + sl + 1] : 0;
      dplug_load(A, R.P, R.rowpos);
    }
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int t = 0; t < TT; ++t) R.C[m][t] = df4{0.f, 0.f, 0.f, 0.f};
    DnStage<TT> S0, S1;
    dn_issue<TT>(A, R.ctile, nrows, R.voc, ok, R.pos, kb, ke, R.vox, R.xblk, j0, S0);
    for (int k0 = kb; k0 < ke; k0 += 64) {
      R.step(S0, S1, k0);
      R.step(S1, S0, k0 + 32);
    }
    // epilogue: lane holds rows n0 + 4q + r, r = 0..3, of token j0 + 16t + i
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const int j = j0 + 16 * t + i;
        const int nn = n0 + 4 * q;
        const df4 c = R.C[m][t];
        if (j >= A.M || nn >= A.N) continue;
        if (A.slices == 1) {
          f16* o = A.out[m] + (int64_t)j * A.o_sm + nn;
          if (A.vec_out && nn + 3 < A.N) {
            const f16x4 h = {(f16)c[0], (f16)c[1], (f16)c[2], (f16)c[3]};
            *reinterpret_cast<f16x4*>(o) = h;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (nn + r < A.N) o[r] = (f16)c[r];
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (nn + r < A.N)
              __hip_atomic_fetch_add(A.acc + ((int64_t)m * A.N + nn + r) * A.M + j, c[r], __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        }
      }
  }
}

template <int TT, int LAYOUT>
__global__ __launch_bounds__(DM_NT) __attribute__((amdgpu_waves_per_eu(2, 2))) void dual_nk_mfma_kernel(
    const DualNkArgs A) {
  __shared__ __attribute__((aligned(16))) char T[DLDS_BYTES];
  if (A.luts.dtype == PP_F16) dual_tables_of<DM_NT, LAYOUT, f16>(T, A.luts);
  else dual_tables_of<DM_NT, LAYOUT, float>(T, A.luts);
  if (A.plug_n > 0) dn_body<TT, LAYOUT, true>(T, A);
  else dn_body<TT, LAYOUT, false>(T, A);
}

static int dm_tt(int64_t M) { return M <= 32 ? 2 : M <= 64 ? 4 : 8; }

// Token tiles per consumer of the producer/consumer form: 128-token blocks (TT = 2) to 255
// tokens, and above where 256-token blocks would fill at most half the CUs while 128-token
// ones fill them all; 256 otherwise.
static int dpc_tt(int64_t M, int64_t N) {
  if (M < 256) return 2;
  const int64_t cus = device_cu_count(), cb = (N + DPC_COLS - 1) / DPC_COLS;
  const int64_t g4 = cb * ((M + 255) / 256), g2 = cb * ((M + 127) / 128);
  return 2 * g4 <= cus && g2 >= cus ? 2 : 4;
}

// Its K slices: only when the items would leave more than half the CUs idle, into as few as
// fill them (whole pairs of 32-row steps).
static void dpc_plan(int64_t M, int64_t N, int64_t K, int64_t* slices, int64_t* cols) {
  const int64_t cus = device_cu_count(), tok = 64 * dpc_tt(M, N);
  const int64_t groups = (N + DPC_COLS - 1) / DPC_COLS * ((M + tok - 1) / tok);
  int64_t s = 1;
  if (2 * groups <= cus) s = std::max<int64_t>(1, std::min<int64_t>(K / 64, (cus + groups - 1) / groups));
  const int64_t c = ((K + s - 1) / s + 63) / 64 * 64;
  *cols = c;
  *slices = (K + c - 1) / c;
}

// From 65 tokens the plan is the producer/consumer form's (the one-wave form, which takes
// plug tables and the other layouts at these sizes, runs any plan).
static void dm_plan(int64_t M, int64_t N, int64_t K, int64_t* slices, int64_t* cols) {
  if (M >= 65) return dpc_plan(M, N, K, slices, cols);
  const int64_t waves = (int64_t)device_cu_count() * DM_WAVES;
  const int64_t units = ((N + 15) / 16) * ((M + 16 * dm_tt(M) - 1) / (16 * dm_tt(M)));
  int64_t s = std::max<int64_t>(1, std::min<int64_t>(K / 64, waves / std::max<int64_t>(1, units)));
  const int64_t c = ((K + s - 1) / s + 63) / 64 * 64;   // whole pairs of 32-row steps
  *cols = c;
  *slices = (K + c - 1) / c;
}

}  // namespace pp

using namespace pp;

extern "C" int pp_dual_mfma_plan(int64_t M, int64_t N, int64_t K, int64_t* slices, int64_t* slice_cols) {
  PP_REQUIRE(slices != nullptr && slice_cols != nullptr, "null pointer argument");
  PP_REQUIRE(M >= 1 && N >= 1 && K >= 32, "needs M, N >= 1 and K >= 32");
  dm_plan(M, N, K, slices, slice_cols);
  return PP_OK;
}

extern "C" int64_t pp_dual_mfma_workspace_size(int64_t M, int64_t N, int64_t slices) {
  if (slices <= 1) return 0;
  return (2 * N * M * 4 + 255) / 256 * 256;
}

extern "C" int pp_dual_mfma(const void* codes, int64_t ldk, const void* a, int64_t a_sm, const void* bmax,
                            int64_t group_size, const void* amp_lut, int amp_n, const void* cos_lut,
                            const void* sin_lut, int phase_n, int lut_dtype, const uint32_t* plug_idx,
                            const void* plug_amp, int64_t plug_n, const int64_t* row_plug, int64_t plug_pos0,
                            int64_t plug_ld, int64_t slices, int64_t slice_cols, void* out1, void* out2,
                            int64_t o_sm, int64_t M, int64_t N, int64_t K, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  PP_REQUIRE(codes && a && bmax && amp_lut && cos_lut && sin_lut && out1 && out2, "null pointer argument");
  PP_REQUIRE(lut_dtype == PP_F16 || lut_dtype == PP_F32, "bad lut_dtype");
  PP_REQUIRE(amp_n >= 1 && amp_n <= 64 && phase_n >= 1 && phase_n <= 1024, "amp_n must be 1..64, phase_n 1..1024");
  PP_REQUIRE(M >= 1 && N >= 1 && K >= 32 && K % 32 == 0, "needs M, N >= 1 and K a multiple of 32 (N=%lld, K=%lld)",
             (long long)N, (long long)K);
  PP_REQUIRE(ldk >= N && aligned(codes, 2), "codes: (K,N) rows of ldk >= N int16 codes");
  PP_REQUIRE(group_size >= 1 && (group_size & (group_size - 1)) == 0, "group_size must be a power of two");
  PP_REQUIRE(aligned(a, 16) && (M == 1 || (a_sm >= K && a_sm % 8 == 0)),
             "activations must be 16-byte aligned with a row stride that is a multiple of 8");
  PP_REQUIRE(o_sm >= N, "o_sm must be >= N");
  PP_REQUIRE(slices >= 1 && slice_cols >= 64 && slice_cols % 64 == 0 && slices * slice_cols >= K &&
                 (slices - 1) * slice_cols < K,
             "slices x slice_cols must cover K in multiples of 64 rows");
  PP_REQUIRE(plug_n >= 0 && plug_n < (1ll << 29) && (plug_n == 0 || (plug_idx && plug_amp && row_plug)),
             "plug arrays are null (or more than 2^29 entries)");
  const int64_t n_groups = (K * N + group_size - 1) / group_size;
  PP_REQUIRE(K * ldk * 2 < (1ll << 31) && n_groups * 2 < (1ll << 31) && (M - 1) * a_sm + K < (1ll << 30),
             "the codes, the scales and the activations must each stay below 2 GiB");
  const int64_t need = pp_dual_mfma_workspace_size(M, N, slices);
  PP_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need), "workspace too small: need %lld bytes",
             (long long)need);
  PP_REQUIRE(need == 0 || aligned(workspace, 16), "the workspace must be 16-byte aligned");
  DualMfmaArgs A = {};
  A.codes = reinterpret_cast<const uint16_t*>(codes);
  A.ldk = ldk;
  A.x = reinterpret_cast<const f16*>(a);
  A.x_sm = M > 1 ? a_sm : K;
  A.out[0] = reinterpret_cast<f16*>(out1);
  A.out[1] = reinterpret_cast<f16*>(out2);
  A.o_sm = o_sm;
  A.vec_out = o_sm % 4 == 0 && aligned(out1, 8) && aligned(out2, 8);
  A.N = (int)N;
  A.K = (int)K;
  A.M = (int)M;
  const int tt = dm_tt(M);
  A.tiles = (int)((N + 15) / 16);
  A.tblocks = (int)((M + 16 * tt - 1) / (16 * tt));
  A.slices = (int)slices;
  A.ks = (int)slice_cols;
  A.scales = reinterpret_cast<const f16*>(bmax);
  A.n_groups = n_groups;
  int lg = 0;
  while ((1ll << lg) < group_size) ++lg;
  A.log2gs = lg;
  A.gcols = plug_n == 0 && N % 16 == 0 && group_size >= 8 && N % group_size == 0 && ldk % 8 == 0 &&
                    aligned(codes, 16)
                ? (int)(N / group_size)
                : 0;
  A.luts.amp = amp_lut;
  A.luts.cs[0] = cos_lut;
  A.luts.cs[1] = sin_lut;
  A.luts.amp_n = amp_n;
  A.luts.phase_n = phase_n;
  A.luts.dtype = lut_dtype;
  A.plug_idx = plug_idx;
  A.plug_amp = reinterpret_cast<const f16*>(plug_amp);
  A.plug_n = plug_n;
  A.row_plug = row_plug;
  A.ppos0 = plug_pos0;
  A.pld = plug_ld;
  A.acc = reinterpret_cast<float*>(workspace);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (M >= 65 && A.gcols > 0) {
    const int ptt = dpc_tt(M, N);
    A.tblocks = (int)((M + 64 * ptt - 1) / (64 * ptt));
    const int64_t items = (N + DPC_COLS - 1) / DPC_COLS * A.tblocks * slices;
    const int64_t grid = std::min<int64_t>(device_cu_count(), items);
    A.xcd_remap = grid % 8 == 0;
    if (ptt == 2) hipLaunchKernelGGL(dual_pc_kernel<2>, dim3((unsigned)grid), dim3(DPC_NT), 0, st, A);
    else hipLaunchKernelGGL(dual_pc_kernel<4>, dim3((unsigned)grid), dim3(DPC_NT), 0, st, A);
  } else {
    const int64_t groups = (int64_t)(A.tiles + DM_WAVES - 1) / DM_WAVES * A.tblocks * slices;
    const int64_t grid = std::min<int64_t>(device_cu_count(), groups);
    A.xcd_remap = grid % 8 == 0;
    switch (tt) {
      case 2: hipLaunchKernelGGL(dual_mfma_kernel<2>, dim3((unsigned)grid), dim3(DM_NT), 0, st, A); break;
      case 4: hipLaunchKernelGGL(dual_mfma_kernel<4>, dim3((unsigned)grid), dim3(DM_NT), 0, st, A); break;
      default: hipLaunchKernelGGL(dual_mfma_kernel<8>, dim3((unsigned)grid), dim3(DM_NT), 0, st, A); break;
    }
  }
  PP_LAUNCH_CHECK();
  if (slices > 1) {
    hipLaunchKernelGGL(dual_mfma_finish_kernel, dim3((unsigned)finish_tiles(2, N, M)), dim3(256), 0, st, A.acc,
                       A.out[0], A.out[1], o_sm, A.N, A.M, o_sm % 4 == 0 && aligned(out1, 8) && aligned(out2, 8));
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
}

extern "C" int pp_dual_nk_mfma(const void* codes, int code_layout, int64_t ldc, int64_t elem_base, const void* a,
                               int64_t a_sm, const void* scales, int64_t n_groups, int64_t group_size,
                               int64_t chunk_size, const void* amp_lut, int amp_n, const void* cos_lut,
                               const void* sin_lut, int phase_n, int lut_dtype, const uint32_t* plug_idx,
                               const void* plug_amp, int64_t plug_n, const int64_t* row_plug, int64_t slices,
                               int64_t slice_cols, void* out1, void* out2, int64_t o_sm, int64_t M, int64_t N,
                               int64_t K, void* workspace, int64_t workspace_bytes, void* stream) {
  PP_REQUIRE(codes && a && scales && amp_lut && cos_lut && sin_lut && out1 && out2, "null pointer argument");
  PP_REQUIRE(code_layout == PP_DUAL_U16_BE || code_layout == PP_DUAL_I16_OFFSET, "bad code_layout");
  PP_REQUIRE(lut_dtype == PP_F16 || lut_dtype == PP_F32, "bad lut_dtype");
  PP_REQUIRE(amp_n >= 1 && amp_n <= 64 && phase_n >= 1 && phase_n <= 1024, "amp_n must be 1..64, phase_n 1..1024");
  PP_REQUIRE(M >= 1 && N >= 1 && N < (1ll << 30) && K >= 32 && K % 32 == 0,
             "needs M, N >= 1 and K a multiple of 32 (N=%lld, K=%lld)", (long long)N, (long long)K);
  PP_REQUIRE(ldc >= K && ldc % 8 == 0 && aligned(codes, 16) && elem_base >= 0 && elem_base % 8 == 0,
             "codes: 16-byte aligned (N,K) rows of ldc >= K pairs, ldc and elem_base multiples of 8");
  PP_REQUIRE(group_size >= 8 && (group_size & (group_size - 1)) == 0, "group_size must be a power of two >= 8");
  PP_REQUIRE(chunk_size >= 32 && chunk_size % 8 == 0 && chunk_size < (1ll << 30),
             "chunk_size must be a multiple of 8 in [32, 2^30)");
  PP_REQUIRE(n_groups >= 1 && n_groups < (1ll << 30), "n_groups must be in [1, 2^30)");
  PP_REQUIRE(aligned(a, 16) && (M == 1 || (a_sm >= K && a_sm % 8 == 0)),
             "activations must be 16-byte aligned with a row stride that is a multiple of 8");
  PP_REQUIRE(o_sm >= N, "o_sm must be >= N");
  PP_REQUIRE(slices >= 1 && slice_cols >= 64 && slice_cols % 64 == 0 && slices * slice_cols >= K &&
                 (slices - 1) * slice_cols < K,
             "slices x slice_cols must cover K in multiples of 64 columns");
  PP_REQUIRE(plug_n >= 0 && plug_n < (1ll << 29) && (plug_n == 0 || (plug_idx && plug_amp && row_plug)),
             "plug arrays are null (or more than 2^29 entries)");
  PP_REQUIRE(16 * ldc * 2 < (1ll << 31) && (M - 1) * a_sm + K < (1ll << 30),
             "a row tile's codes and the activations must each stay below 2 GiB");
  const int64_t need = pp_dual_mfma_workspace_size(M, N, slices);
  PP_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need), "workspace too small: need %lld bytes",
             (long long)need);
  PP_REQUIRE(need == 0 || aligned(workspace, 16), "the workspace must be 16-byte aligned");
  DualNkArgs A = {};
  A.codes = reinterpret_cast<const uint16_t*>(codes);
  A.ldc = ldc;
  A.elem_base = elem_base;
  A.x = reinterpret_cast<const f16*>(a);
  A.x_sm = M > 1 ? a_sm : K;
  A.out[0] = reinterpret_cast<f16*>(out1);
  A.out[1] = reinterpret_cast<f16*>(out2);
  A.o_sm = o_sm;
  A.vec_out = o_sm % 4 == 0 && aligned(out1, 8) && aligned(out2, 8);
  A.N = (int)N;
  A.K = (int)K;
  A.M = (int)M;
  const int tt = dm_tt(M);
  A.tiles = (int)((N + 15) / 16);
  A.tblocks = (int)((M + 16 * tt - 1) / (16 * tt));
  A.slices = (int)slices;
  A.ks = (int)slice_cols;
  A.scales = reinterpret_cast<const f16*>(scales);
  A.n_groups = n_groups;
  A.chunk = (int)chunk_size;
  A.gpc = (chunk_size + group_size - 1) / group_size;
  int lg = 0;
  while ((1ll << lg) < group_size) ++lg;
  A.log2gs = lg;
  A.luts.amp = amp_lut;
  A.luts.cs[0] = cos_lut;
  A.luts.cs[1] = sin_lut;
  A.luts.amp_n = amp_n;
  A.luts.phase_n = phase_n;
  A.luts.dtype = lut_dtype;
  A.plug_idx = plug_idx;
  A.plug_amp = reinterpret_cast<const f16*>(plug_amp);
  A.plug_n = plug_n;
  A.row_plug = row_plug;
  A.acc = reinterpret_cast<float*>(workspace);
  const int64_t groups = (int64_t)(A.tiles + DM_WAVES - 1) / DM_WAVES * A.tblocks * slices;
  const int64_t grid = std::min<int64_t>(device_cu_count(), groups);
  A.xcd_remap = grid % 8 == 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool be = code_layout == PP_DUAL_U16_BE;
  using KernelFn = void (*)(DualNkArgs);
  static const KernelFn kernels[3][2] = {
      {dual_nk_mfma_kernel<2, PP_DUAL_I16_OFFSET>, dual_nk_mfma_kernel<2, PP_DUAL_U16_BE>},
      {dual_nk_mfma_kernel<4, PP_DUAL_I16_OFFSET>, dual_nk_mfma_kernel<4, PP_DUAL_U16_BE>},
      {dual_nk_mfma_kernel<8, PP_DUAL_I16_OFFSET>, dual_nk_mfma_kernel<8, PP_DUAL_U16_BE>}};
  hipLaunchKernelGGL(kernels[tt == 2 ? 0 : tt == 4 ? 1 : 2][be ? 1 : 0], dim3((unsigned)grid), dim3(DM_NT), 0, st, A);
  PP_LAUNCH_CHECK();
  if (slices > 1) {
    hipLaunchKernelGGL(dual_mfma_finish_kernel, dim3((unsigned)finish_tiles(2, N, M)), dim3(256), 0, st, A.acc,
                       A.out[0], A.out[1], o_sm, A.N, A.M, o_sm % 4 == 0 && aligned(out1, 8) && aligned(out2, 8));
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
}
