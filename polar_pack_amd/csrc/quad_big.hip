// Quad-pack decode GEMM on the matrix cores for large batches (more than 64 tokens, and 33-64
// on (K,N) storage: the producer/consumer form below), and for fewer tokens on (K,N)
// storage: one fused pass produces the 4 models' outputs
//   out_m[j, n] = fp16( s_m * sum_k x[j, k] * W_m[n, k] )
// (quad_kernels.py:123-134) with W_m decoded from the codes in registers
// (quad_kernels.py:103-121, quaternion_packer.py:173-185), the plug table patched into
// the decoded operands (quaternion_packer.py:187-193), and no weight ever written to
// memory.
//
// The one-wave form (to 64 tokens on (N,K) rows, to 32 on (K,N) codes): work item = 16
// weight rows x TT token tiles of 16 (TT = 1, 2 or 4, the fewest that hold the batch) x one
// K slice, one wavefront, v_mfma_f32_16x16x32_f16 (operand layouts as in quad_mfma.hip):
//  * per 32-column step a lane decodes 8 code words of its row (n0 + i, i = lane % 16,
//    columns k0 + 8(lane/16) .. +7), so each code word is decoded once per 16 TT tokens and
//    feeds 4 models x TT token tiles of products;
//  * x is the B operand as stored: lane l reads tokens 16t + l%16 at the same 8 columns;
//  * 4 models x TT token tiles of 16 x 16 fp32 sums stay in registers, with G buffers of
//    codes (loaded G - 1 steps ahead), two of x (loaded a step before the products that
//    use it) and two of decoded operands (QbCfg);
//  * the products of step s - 1 are issued between the arithmetic of step s, after step
//    s's LDS lookups (with one tile, step s + 1's).
// Codes in either storage: (N,K) rows (the stream container, K contiguous: two 16-byte
// loads per step) or (K,N) (pack_quad_layer, N contiguous: 8 four-byte loads per step,
// each a 64-byte run over 16 lanes).  Plug positions are read in an (N,K) frame (position
// ppos0 + n*pld + k): for (K,N) storage the host moves them there first.
// Slices: with one slice a wave writes its fp16 outputs; otherwise it adds its scaled sums
// into float32 accumulators [m][n][j] with device-scope atomics and quad_big_finish_kernel
// writes the outputs and leaves zeros for the next launch.
#include "quad_mfma.h"

namespace pp {

constexpr int QB_ROWS = 16;     // weight rows per item

// TT 16-token tiles per item (1, 2 or 4: up to 16, 32 or 64 tokens).  A wavefront fits in
// half of a SIMD's register file: on (N,K) rows two waves share a SIMD (8 per workgroup); on
// (K,N) storage one wave per SIMD with twice the items measured faster (4096 x 4096 at 16 /
// 32 / 64 tokens: 27 / 32 / 44 against 31 / 39 / 51 us; the second wave of a SIMD ran its
// items 1.29x slower than the first, and the (K,N) step's 8 four-byte code loads per lane
// leave less to overlap).  One workgroup per CU: the decode tables fill the LDS.
// G: steps per loop pass = code buffers, the codes of a step loaded G - 1 steps before it
// (2 KiB per wave and step: with few token tiles the decode is short and a wave needs
// several steps of codes in flight to cover the HBM latency).
template <int TT, bool KN> struct QbCfg {
  static constexpr int WPE = KN ? 1 : 2;               // waves per SIMD
  static constexpr int NT = 256 * WPE;
  static constexpr int WAVES = NT / 64;
  static constexpr int G = TT <= 2 ? 4 : 2;
};

// Token tiles per item for a batch of M tokens.
static inline int qb_tt(int64_t M) { return M <= 16 ? 1 : M <= 32 ? 2 : 4; }

struct QuadBigArgs {
  const uint32_t* codes;
  int64_t ldc;             // (N,K) storage: words between rows n; (K,N): words between rows k
  const f16* x;            // (M, K), row stride x_sm
  int64_t x_sm;
  f16* out[4];             // (M, N), row stride o_sm
  int64_t o_sm;
  int N, K, M;
  int tiles, tblocks;      // ceil(N / 16), ceil(M / 128)
  int slices, ks;          // K slices of ks columns (a multiple of 32)
  QuadLuts luts;
  float s[4];
  PlugSrc plug;
  const int64_t* row_plug; // [n*slices + s]: first plug entry of (row n, slice s); N*slices + 1 entries
  int64_t ppos0, pld;      // plug position of (row n, column k): ppos0 + n*pld + k
  float* acc;              // slices > 1: [4][N][M] float32, zero on entry
  int xcd_remap;           // grid a multiple of 8: consecutive items on the workgroups of one XCD
  int vec_out;             // outputs 8-byte aligned with o_sm % 4 == 0: 4 rows per store
};

struct QbCodes {
  u32x4 c[2];              // 8 code words of the lane's row
};
template <int TT>
struct QbX {
  u32x4 xb[TT];            // 8 fp16 x of token 16t + l%16
};

// Issue the code loads of the step at column k0, clamped to the slice's last step (ke - 32:
// a step past the slice end reloads codes just read, whose products are zero).  voc: the
// lane's code offset (OOB for a row past N).  (K,N) storage: the 8 columns' rows are 4*ldc
// bytes apart, an offset carried in the scalar operand.
template <bool KN>
__device__ __forceinline__ void qb_codes(const QuadBigArgs& A, const uint32_t* ctile, int n0, int k0, int ke,
                                         uint32_t voc, QbCodes& S) {
  k0 = min(k0, ke - 32);
  if constexpr (!KN) {
    const int nr = min(QB_ROWS, A.N - n0);
    const rsrc_t rc = make_rsrc(ctile + k0, 4u * (uint32_t)((int64_t)(nr - 1) * A.ldc + (A.K - k0)));
    vload128(S.c[0], voc, rc);
    vload128(S.c[1], voc + 16u, rc);
  } else {
    const rsrc_t rc = make_rsrc(ctile + (int64_t)k0 * A.ldc,
                                4u * (uint32_t)((int64_t)(A.K - 1 - k0) * A.ldc + (A.N - n0)));
    const int st = (int)(4 * A.ldc);
#pragma unroll
    for (int e = 0; e < 8; ++e) S.c[e >> 2][e & 3] = __builtin_amdgcn_raw_buffer_load_b32(rc, (int)voc, e * st, NT_AUX);
  }
}

// Issue the x loads of the step at column k0: vox, the lane's offsets per token tile (OOB
// past M).  A step at or past the slice end ke (the walk runs whole groups of steps) reads
// through an empty buffer record, i.e. zeros, so its products add nothing.
template <int TT>
__device__ __forceinline__ void qb_x(const QuadBigArgs& A, int k0, int ke, const uint32_t (&vox)[TT],
                                     const f16* xblk, int j0, QbX<TT>& S) {
  const uint32_t xrec = k0 < ke ? 2u * (uint32_t)((int64_t)(A.M - 1 - j0) * A.x_sm + (ke - k0)) : 0u;
  const rsrc_t rx = make_rsrc(xblk + min(k0, A.K - 32), xrec);
#pragma unroll
  for (int t = 0; t < TT; ++t) vload128c(S.xb[t], vox[t], rx);
}

// The LDS lookups of 8 code words, issued together, and the arithmetic on them.
struct Look8 {
  float r[8];
  float2 a[8], b[8], c[8];
};

template <class L>
__device__ __forceinline__ void look8(const char* lds, const LaneOff& lo, const u32x4& c0, const u32x4& c1,
                                      Look8& o) {
  const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) lookup<L>(lds, cw[e], lo, o.r[e], o.a[e], o.b[e], o.c[e]);
}

__device__ __forceinline__ void math8(const Look8& o, h8 (&a)[4]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float rs = o.r[e] * o.a[e].y, rss = rs * o.b[e].y;
    a[0][e] = (_Float16)(o.r[e] * o.a[e].x);
    a[1][e] = (_Float16)(rs * o.b[e].x);
    a[2][e] = (_Float16)(rss * o.c[e].x);
    a[3][e] = (_Float16)(rss * o.c[e].y);
  }
}

template <int TT, bool KN, bool PLUG, class L>
struct QbRun {
  const char* lds;
  LaneOff lo;
  const QuadBigArgs& A;
  const uint32_t* ctile;
  const f16* xblk;
  int n0, j0, q, ke;
  uint32_t voc;
  uint32_t vox[TT];
  int64_t rowpos;
  MPlug P;
  f4 C[4][TT];

  __device__ __forceinline__ void mfma(const h8 (&a)[4], const QbX<TT>& S) {
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const h8 b = __builtin_bit_cast(h8, S.xb[t]);
#pragma unroll
      for (int m = 0; m < 4; ++m) C[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m], b, C[m][t], 0, 0, 0);
    }
  }

  // Step at k0: issue the x loads of k0 into xnow (used by the next step) and the code
  // loads of k0 + 32 (G - 1) into nxt, look up cur's codes, then the products of the
  // previous step (operands aprev, x in xprev) interleaved with the arithmetic of this one
  // into anew.  x goes first: the wait for it in the next step (the memory counter drains
  // in issue order) then leaves the code loads issued after it in flight.
  __device__ __forceinline__ void step(const QbCodes& cur, QbCodes& nxt, QbX<TT>& xnow, const QbX<TT>& xprev,
                                       const h8 (&aprev)[4], h8 (&anew)[4], int k0) {
    qb_x(A, k0, ke, vox, xblk, j0, xnow);
    qb_codes<KN>(A, ctile, n0, k0 + 32 * (QbCfg<TT, KN>::G - 1), ke, voc, nxt);
    Look8 lk;
    look8<L>(lds, lo, cur.c[0], cur.c[1], lk);
    __builtin_amdgcn_sched_barrier(0);
    mfma(aprev, xprev);
    math8(lk, anew);
    // 4 TT products against about 64 arithmetic instructions: one product, then 16 / TT
#pragma unroll
    for (int i = 0; i < 4 * TT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 16 / TT, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PLUG) mplug_patch(A.plug, P, rowpos, k0 + 8 * q, k0, anew);
  }
};

template <int TT, bool KN, bool PLUG, class L>
__device__ __forceinline__ void qb_body(const char* lds, const QuadBigArgs& A) {
  constexpr int WAVES = QbCfg<TT, KN>::WAVES;
  const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
  const LaneOff lo = L::lane(lane);
  int b = blockIdx.x;
  if (A.xcd_remap) b = (b & 7) * (int)(gridDim.x >> 3) + (b >> 3);
  const int64_t gw = (int64_t)b * WAVES + uniform(threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * WAVES;
  // Items in groups of WAVES row tiles that share a token block and K slice, one group
  // per workgroup (its waves read the same x, through the CU's L1); groups ordered slice,
  // token block, row tiles, so the workgroups of one XCD (consecutive after the remap)
  // share row tiles (codes) and token blocks (x) through its L2.
  const int64_t tgroups = (A.tiles + WAVES - 1) / WAVES;
  const int64_t items = tgroups * WAVES * A.tblocks * A.slices;
  for (int64_t it = gw; it < items; it += nw) {
    const int64_t w = uniform64(it / WAVES);
    const int tile = (int)(uniform64(w / ((int64_t)A.slices * A.tblocks)) * WAVES + it % WAVES);
    const int sl = (int)(w % A.slices), tb = (int)((w / A.slices) % A.tblocks);
    if (tile >= A.tiles) continue;
    const int n0 = tile * QB_ROWS, j0 = tb * 16 * TT;
    const int kb = sl * A.ks, ke = min(A.K, kb + A.ks);
    QbRun<TT, KN, PLUG, L> R{lds, lo, A, KN ? A.codes + n0 : A.codes + (int64_t)n0 * A.ldc,
                             A.x + (int64_t)j0 * A.x_sm, n0, j0, q, ke};
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const int jl = 16 * t + i;
      R.vox[t] = j0 + jl < A.M ? 2u * (uint32_t)(jl * A.x_sm + 8 * q) : OOB;
    }
    const int n = n0 + i;
    const bool ok = n < A.N;
    R.voc = !ok ? OOB : KN ? 4u * (uint32_t)(8 * q * A.ldc + i) : 4u * (uint32_t)(i * A.ldc + 8 * q);
    uint32_t pidx[MPW];
    if constexpr (PLUG) {
      R.rowpos = A.ppos0 + (int64_t)n * A.pld;
      R.P.next = ok ? A.row_plug[(int64_t)n * A.slices + sl] : 0;
      R.P.end = ok ? A.row_plug[(int64_t)n * A.slices + sl + 1] : 0;
      mplug_issue(A.plug, R.P, pidx);
    }
    constexpr int G = QbCfg<TT, KN>::G;
    QbCodes C[G];
    QbX<TT> X0, X1;
#pragma unroll
    for (int g = 0; g + 1 < G; ++g) qb_codes<KN>(A, R.ctile, n0, kb + 32 * g, ke, R.voc, C[g]);
    if constexpr (PLUG) mplug_take(R.P, pidx, R.rowpos);
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int t = 0; t < TT; ++t) R.C[m][t] = f4{0.f, 0.f, 0.f, 0.f};
    // step s reads code buffer s % 2, loads x buffer s % 2 and writes operand set s % 2;
    // the "previous step" of the first one multiplies zeros
    h8 Aa[4], Ab[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) Ab[m] = h8{};
#pragma unroll
    for (int t = 0; t < TT; ++t) X1.xb[t] = u32x4{0u, 0u, 0u, 0u};
    // whole groups of steps with no exit between them, so that each load is issued in the
    // step that starts it (not moved by the compiler towards the block that reads it)
    for (int k0 = kb; k0 < ke; k0 += 32 * G) {
#pragma unroll
      for (int g = 0; g < G; g += 2) {
        R.step(C[g], C[(g + G - 1) % G], X0, X1, Ab, Aa, k0 + 32 * g);
        R.step(C[g + 1], C[g], X1, X0, Aa, Ab, k0 + 32 * (g + 1));
      }
    }
    R.mfma(Ab, X1);   // the last step's products
    // epilogue: lane holds rows n0 + 4q + r, r = 0..3, of token j0 + 16t + i
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const int j = j0 + 16 * t + i;
        const int nn = n0 + 4 * q;
        const f4 c = R.C[m][t] * A.s[m];
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

template <int TT, bool KN>
__global__ __launch_bounds__((QbCfg<TT, KN>::NT))
__attribute__((amdgpu_waves_per_eu(QbCfg<TT, KN>::WPE, QbCfg<TT, KN>::WPE))) void quad_big_kernel(
    const QuadBigArgs A) {
  __shared__ __attribute__((aligned(16))) uint32_t Tb[QLDS_BYTES / 4];
  const char* lds = reinterpret_cast<const char*>(Tb);
  const bool shared = quad_tables<QbCfg<TT, KN>::NT>(Tb, A.luts);
  if (A.plug.n > 0) {
    if (shared) qb_body<TT, KN, true, LayShared>(lds, A);
    else qb_body<TT, KN, true, LaySplit>(lds, A);
  } else {
    if (shared) qb_body<TT, KN, false, LayShared>(lds, A);
    else qb_body<TT, KN, false, LaySplit>(lds, A);
  }
}

// ---------------------------------------------------------------- producer/consumer form
// From 65 tokens (33 on (K,N) codes, pc_use): a workgroup of 8 waves takes an item of 32
// weight rows x a block of 64 TT tokens (TT = 1, 2 or 4, pc_tt) x one K slice.  Waves 0-3
// decode (producers) and waves 4-7 multiply (consumers), one of each per SIMD, so a SIMD's
// VALU decode and its matrix products come from two
// waves and run side by side (the one-wave form issues them in turn).  Per super-step of
// 64 columns, producer p decodes row tile p % 2 at column half p / 2 (8 code words per
// lane, as above) into LDS as the MFMA A operands of the 4 models; consumer c multiplies
// the previous super-step's 2 x 2 x 4 operands with its TT token tiles of x (tokens
// 16 TT c .. 16 TT (c + 1) - 1 of the block).  Each code word is decoded once per 64 TT
// tokens.  The tables take the split layout (128 KiB, any LUTs), the two operand buffers
// the rest.
// (K,N) codes at 33-64 tokens: 64-token blocks measured faster than the one-wave form
// (4096x4096 / K x N = 2048x11008 / 11008x2048 at 48 tokens 37.5 / 55 / 44 against 42 / 73 /
// 50 us, at 64 38 / 56 / 45 against 45 / 80 / 56; from 16 to 32 tokens they tie or lose:
// 4096x4096 at 16 tokens 35 against 31 us).  On (N,K) rows the one-wave form is kept to
// 64 tokens (the drop-in operator takes pp_quad_mfma there).
static bool pc_use(int64_t M, bool kn) { return M >= 65 || (kn && M >= 33); }
constexpr int PC_ROWS = 32, PC_NT = 512;
#ifndef PP_PC_G
#define PP_PC_G 4
#endif
constexpr int PC_G = PP_PC_G;                             // code buffers of a producer
// The operand buffers come first in LDS, so that every operand access is one lane base plus
// an immediate offset (below 64 KiB); the tables follow.
constexpr uint32_t PC_ABUF = 0, PC_ABYTES = 0x4000;       // [rt 2][kh 2][m 4][lane 64] x 16 B
constexpr uint32_t PC_TABLES = 2 * PC_ABYTES;
static_assert(PC_TABLES + 0x20000 <= QLDS_BYTES, "the split tables must fit after the operand buffers");

__device__ __forceinline__ uint32_t pc_aoff(int buf, int rt, int kh, int m, int lane) {
  return PC_ABUF + (uint32_t)buf * PC_ABYTES + (uint32_t)((((rt * 2 + kh) * 4 + m) * 64 + lane) * 16);
}

// An item's super-steps, rounded up to whole rounds of PC_G (the producers' code buffers and
// the consumers' x buffers rotate with the super-step; super-steps past the slice read
// zero x, so their products add nothing).
__device__ __forceinline__ int pc_steps(int kb, int ke) { return ((ke - kb + 63) / 64 + PC_G - 1) / PC_G * PC_G; }

template <bool KN, bool PLUG>
__device__ __forceinline__ void pc_producer(char* lds, const QuadBigArgs& A, int p, int n0b, int kb, int ke, int sl) {
  const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
  const int rt = p & 1, kh = p >> 1;
  const int n0 = n0b + 16 * rt;
  const LaneOff lo = LaySplit::lane(lane);
  const int n = n0 + i;
  const bool ok = n < A.N;
  const uint32_t voc = !ok ? OOB : KN ? 4u * (uint32_t)(8 * q * A.ldc + i) : 4u * (uint32_t)(i * A.ldc + 8 * q);
  // a row tile past N (the second of a 32-row block at the end): resources based on the
  // last row, every lane out of range (nothing read)
  const int n0c = min(n0, A.N - 1);
  const uint32_t* ctile = KN ? A.codes + n0c : A.codes + (int64_t)n0c * A.ldc;
  MPlug P;
  int64_t rowpos = 0;
  uint32_t pidx[MPW];
  if constexpr (PLUG) {
    rowpos = A.ppos0 + (int64_t)n * A.pld;
    P.next = ok ? A.row_plug[(int64_t)n * A.slices + sl] : 0;
    P.end = ok ? A.row_plug[(int64_t)n * A.slices + sl + 1] : 0;
    mplug_issue(A.plug, P, pidx);
  }
  const int ns = pc_steps(kb, ke);
  QbCodes C[PC_G];
#pragma unroll
  for (int g = 0; g + 1 < PC_G; ++g) qb_codes<KN>(A, ctile, n0c, kb + 64 * g + 32 * kh, ke, voc, C[g]);
  if constexpr (PLUG) mplug_take(P, pidx, rowpos);
  // super-step s: decode C[s % G] into operand buffer s % 2
  auto decode = [&](const QbCodes& c, int s) {
    Look8 lk;
    look8<LaySplit>(lds + PC_TABLES, lo, c.c[0], c.c[1], lk);
    h8 a[4];
    math8(lk, a);
    const int k0 = kb + 64 * s + 32 * kh;
#pragma unroll
    for (int m = 0; m < 4; ++m) *reinterpret_cast<h8*>(lds + pc_aoff(s & 1, rt, kh, m, lane)) = a[m];
    if constexpr (PLUG) mplug_patch_lds(A.plug, P, rowpos, k0 + 8 * q, k0, lds + pc_aoff(s & 1, rt, kh, 0, lane), 1024u);
  };
  // C[k % G] holds super-step k.  Prologue: super-step 0 into operand buffer 0, its code
  // buffer refilled with super-step G.
  qb_codes<KN>(A, ctile, n0c, kb + 64 * (PC_G - 1) + 32 * kh, ke, voc, C[PC_G - 1]);
  decode(C[0], 0);
  qb_codes<KN>(A, ctile, n0c, kb + 64 * PC_G + 32 * kh, ke, voc, C[0]);
  __syncthreads();
  for (int s = 0; s < ns; s += PC_G) {
#pragma unroll
    for (int g = 0; g < PC_G; ++g) {
      // while the consumers multiply super-step s + g (operand buffer (s + g) % 2), decode
      // d = s + g + 1 into the other buffer and refill its code buffer with d + G
      const int d = s + g + 1;
      decode(C[(g + 1) % PC_G], d);
      qb_codes<KN>(A, ctile, n0c, kb + 64 * (d + PC_G) + 32 * kh, ke, voc, C[(g + 1) % PC_G]);
      __syncthreads();
    }
  }
}

template <bool KN, int TT>
__device__ __forceinline__ void pc_consumer(const char* lds, const QuadBigArgs& A, int c, int n0b, int j0b, int kb,
                                            int ke) {
  const int lane = threadIdx.x & 63, i = lane & 15, q = lane >> 4;
  const int j0 = j0b + 16 * TT * c;
  const f16* xblk = A.x + (int64_t)min(j0, A.M - 1) * A.x_sm;
  uint32_t vox[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int jl = 16 * t + i;
    vox[t] = j0 + jl < A.M ? 2u * (uint32_t)(jl * A.x_sm + 8 * q) : OOB;
  }
  const int jx = min(j0, A.M - 1);
  const int ns = pc_steps(kb, ke);
  f4 Cacc[2][4][TT];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int t = 0; t < TT; ++t) Cacc[rt][m][t] = f4{0.f, 0.f, 0.f, 0.f};
  QbX<TT> X[2][2];   // [buffer][column half]
  auto loadx = [&](QbX<TT>(&xb)[2], int s) {
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) qb_x<TT>(A, kb + 64 * s + 32 * kh, ke, vox, xblk, jx, xb[kh]);
  };
  // The 16 operands of a super-step are read in 4 groups (row tile, column half) of the 4
  // models; group g + 1 is requested before group g's products, so the products do not
  // wait on LDS.
  auto multiply = [&](const QbX<TT>(&xb)[2], int s) {
    h8 a[2][4];
#pragma unroll
    for (int m = 0; m < 4; ++m) a[0][m] = *reinterpret_cast<const h8*>(lds + pc_aoff(s & 1, 0, 0, m, lane));
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int rt = g >> 1, kh = g & 1;
      if (g < 3) {
#pragma unroll
        for (int m = 0; m < 4; ++m)
          a[(g + 1) & 1][m] = *reinterpret_cast<const h8*>(lds + pc_aoff(s & 1, (g + 1) >> 1, (g + 1) & 1, m, lane));
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int t = 0; t < TT; ++t)
          Cacc[rt][m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[g & 1][m], __builtin_bit_cast(h8, xb[kh].xb[t]),
                                                                  Cacc[rt][m][t], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  loadx(X[0], 0);
  __syncthreads();
  // The fences keep the next super-step's x loads issued ahead of this one's products, so
  // the products wait only for their own x.
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
  // lane holds rows n0b + 16 rt + 4q + r, r = 0..3, of token j0 + 16t + i
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const int j = j0 + 16 * t + i;
        const int nn = n0b + 16 * rt + 4 * q;
        const f4 v = Cacc[rt][m][t] * A.s[m];
        if (j >= A.M || nn >= A.N) continue;
        if (A.slices == 1) {
          f16* o = A.out[m] + (int64_t)j * A.o_sm + nn;
          if (A.vec_out && nn + 3 < A.N) {
            const f16x4 h = {(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
            *reinterpret_cast<f16x4*>(o) = h;
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (nn + r < A.N) o[r] = (f16)v[r];
          }
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (nn + r < A.N)
              __hip_atomic_fetch_add(A.acc + ((int64_t)m * A.N + nn + r) * A.M + j, v[r], __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        }
      }
}

template <bool KN, int TT>
__global__ __launch_bounds__(PC_NT) void quad_big_pc_kernel(const QuadBigArgs A) {
  __shared__ __attribute__((aligned(16))) uint32_t Tb[QLDS_BYTES / 4];
  char* lds = reinterpret_cast<char*>(Tb);
  if (A.luts.dtype == PP_F16) LaySplit::build<PC_NT, f16>(lds + PC_TABLES, A.luts);
  else LaySplit::build<PC_NT, float>(lds + PC_TABLES, A.luts);
  __syncthreads();
  const int wave = uniform(threadIdx.x >> 6);
  int b = blockIdx.x;
  if (A.xcd_remap) b = (b & 7) * (int)(gridDim.x >> 3) + (b >> 3);
  // items ordered slice, token block, row block: consecutive workgroups (one XCD after
  // the remap) share token blocks (x) and slices
  const int64_t items = (int64_t)A.tiles * A.tblocks * A.slices;
  for (int64_t it = b; it < items; it += gridDim.x) {
    const int rb = (int)uniform64(it % A.tiles);
    const int64_t w = it / A.tiles;
    const int tb = (int)uniform64(w % A.tblocks), sl = (int)uniform64(w / A.tblocks);
    const int n0b = rb * PC_ROWS, j0b = tb * 64 * TT;
    const int kb = sl * A.ks, ke = min(A.K, kb + A.ks);
    if (wave < 4) {
      if (A.plug.n > 0) pc_producer<KN, true>(lds, A, wave, n0b, kb, ke, sl);
      else pc_producer<KN, false>(lds, A, wave, n0b, kb, ke, sl);
    } else {
      pc_consumer<KN, TT>(lds, A, wave - 4, n0b, j0b, kb, ke);
    }
  }
}

template <int TT>
static void qb_launch(bool kn, int64_t grid, hipStream_t st, const QuadBigArgs& A) {
  if (kn) hipLaunchKernelGGL((quad_big_kernel<TT, true>), dim3((unsigned)grid), dim3(QbCfg<TT, true>::NT), 0, st, A);
  else hipLaunchKernelGGL((quad_big_kernel<TT, false>), dim3((unsigned)grid), dim3(QbCfg<TT, false>::NT), 0, st, A);
}

// Sliced launches: out_m[j, n] = fp16(acc[m][n][j]), acc left zero (finish_tile).
__global__ __launch_bounds__(256) void quad_big_finish_kernel(float* acc, f16* o0, f16* o1, f16* o2, f16* o3,
                                                              int64_t o_sm, int N, int M, bool vec) {
  int m, n0, j0;
  finish_coords(N, M, m, n0, j0);
  f16* o = m == 0 ? o0 : m == 1 ? o1 : m == 2 ? o2 : o3;
  finish_tile(acc + (int64_t)m * N * M, o, o_sm, N, M, n0, j0, vec);
}


// K slices for an (N, K) product at M tokens: as many whole 32-column slices as keep the
// items within one per wavefront.
template <int TT>
static int64_t qb_waves_of(bool kn) { return kn ? QbCfg<TT, true>::WAVES : QbCfg<TT, false>::WAVES; }
static int64_t qb_waves(int tt, bool kn) {
  return tt == 1 ? qb_waves_of<1>(kn) : tt == 2 ? qb_waves_of<2>(kn) : qb_waves_of<4>(kn);
}

// Token tiles per consumer of the producer/consumer form: blocks of 64 tokens (TT = 1) to
// 64 tokens, of 128 (TT = 2) to 255 tokens, and above where 256-token blocks would leave half the CUs idle while 128-token
// ones fill them; 256 otherwise.  A super-step of 128 tokens takes ~2/3 of one of 256
// (4096x4096 at 256 tokens: 65 against 98 us with 256-token blocks in 2 K slices; at 128 /
// 192: 57 / 64 against 83 / 117 us on the one-wave form; 11008x2048 rows at 128 / 192: 110
// / 153 against 163 / 223; but 11008x2048 at 256 tokens 156 against 128, 2048x11008 165
// against 122, 4096x4096 at 384 121 against 98).
static int pc_tt(int64_t M, int64_t N) {
  if (M <= 64) return 1;
  if (M < 256) return 2;
  const int64_t cus = device_cu_count(), rb = (N + PC_ROWS - 1) / PC_ROWS;
  const int64_t g4 = rb * ((M + 255) / 256), g2 = rb * ((M + 127) / 128);
  return 2 * g4 <= cus && g2 >= cus ? 2 : 4;
}

// The producer/consumer form's K slices: only when the items would leave more than half
// the CUs idle, into as few as fill them: the slices' sums go through float32 atomics and a
// second launch (gate 11008x2048 at 256 tokens: 214 us with 2 slices, 344 items, against
// one slice).
static void pc_plan(int64_t M, int64_t N, int64_t K, int64_t* slices, int64_t* cols) {
  const int64_t cus = device_cu_count(), steps = K / 32, tok = 64 * pc_tt(M, N);
  const int64_t groups = (N + PC_ROWS - 1) / PC_ROWS * ((M + tok - 1) / tok);
  int64_t s = 1;
  if (2 * groups <= cus) s = std::min<int64_t>(steps, (cus + groups - 1) / groups);
  const int64_t per = (steps + s - 1) / s;
  *cols = 32 * per;
  *slices = (K + *cols - 1) / *cols;
}

static void qb_plan(int64_t M, int64_t N, int64_t K, bool kn, int64_t* slices, int64_t* cols) {
  if (pc_use(M, kn)) return pc_plan(M, N, K, slices, cols);
  const int tt = qb_tt(M);
  const int64_t cus = device_cu_count(), wv = qb_waves(tt, kn);
  const int64_t g = tt == 1 ? QbCfg<1, false>::G : tt == 2 ? QbCfg<2, false>::G : QbCfg<4, false>::G;
  const int64_t steps = K / 32;
  // groups of wv row tiles (one per workgroup and round) for s slices; a launch takes
  // ceil(groups / CUs) rounds of items of ceil(steps / s) steps (whole loop passes of g),
  // each with about 4 steps of fixed cost (its first loads, its epilogue); the slice
  // count with the fewest step-times wins, fewer slices on ties
  const int64_t tgroups = ((N + QB_ROWS - 1) / QB_ROWS + wv - 1) / wv * ((M + 16 * tt - 1) / (16 * tt));
  int64_t best = 1, best_cost = -1;
  for (int64_t s = 1; s <= std::min<int64_t>(steps, 64); ++s) {
    const int64_t per = (steps + s - 1) / s;
    if ((steps + per - 1) / per != s) continue;        // s slices of `per` steps do not exist
    const int64_t rounds = (tgroups * s + cus - 1) / cus;
    const int64_t cost = rounds * ((per + g - 1) / g * g + 4);
    if (best_cost < 0 || cost < best_cost) {
      best = s;
      best_cost = cost;
    }
  }
  const int64_t per = (steps + best - 1) / best;
  *cols = 32 * per;
  *slices = (K + *cols - 1) / *cols;
}

}  // namespace pp

using namespace pp;

extern "C" int pp_quad_big_plan(int64_t M, int64_t N, int64_t K, int layout, int64_t* slices, int64_t* slice_cols) {
  PP_REQUIRE(slices != nullptr && slice_cols != nullptr, "null pointer argument");
  PP_REQUIRE(M >= 1 && N >= 1 && K >= 32, "needs M, N >= 1 and K >= 32");
  PP_REQUIRE(layout == PP_QUAD_NK || layout == PP_QUAD_KN, "layout must be PP_QUAD_NK or PP_QUAD_KN");
  qb_plan(M, N, K, layout == PP_QUAD_KN, slices, slice_cols);
  return PP_OK;
}

extern "C" int64_t pp_quad_big_workspace_size(int64_t M, int64_t N, int64_t slices) {
  if (slices <= 1) return 0;
  return (4 * N * M * 4 + 255) / 256 * 256;
}

extern "C" int pp_quad_big(const uint32_t* codes, int layout, int64_t ldc, const void* a, int64_t a_sm,
                           const void* const* luts, int lut_dtype, const float* scales, const uint32_t* plug_idx,
                           const void* plug_vals, int64_t plug_n, const int64_t* row_plug, int64_t plug_pos0,
                           int64_t plug_ld, int64_t slices, int64_t slice_cols, void* const* out, int64_t o_sm,
                           int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* stream) {
  PP_REQUIRE(codes != nullptr && a != nullptr && out != nullptr && luts != nullptr && scales != nullptr,
             "null pointer argument");
  for (int m = 0; m < 4; ++m) PP_REQUIRE(out[m] != nullptr, "out[%d] is null", m);
  for (int i = 0; i < 7; ++i) PP_REQUIRE(luts[i] != nullptr, "lut %d is null", i);
  PP_REQUIRE(lut_dtype == PP_F16 || lut_dtype == PP_F32, "bad lut_dtype");
  PP_REQUIRE(layout == PP_QUAD_NK || layout == PP_QUAD_KN, "layout must be PP_QUAD_NK or PP_QUAD_KN");
  PP_REQUIRE(M >= 1 && N >= 1 && K >= 32 && K % 32 == 0, "needs M, N >= 1 and K a multiple of 32 (N=%lld, K=%lld)",
             (long long)N, (long long)K);
  const bool kn = layout == PP_QUAD_KN;
  PP_REQUIRE(kn ? ldc >= N : (ldc >= K && ldc % 4 == 0 && aligned(codes, 16)),
             "codes: (N,K) rows must be 16-byte aligned with ldc >= K words (a multiple of 4); (K,N) rows need "
             "ldc >= N");
  PP_REQUIRE(aligned(codes, 4), "codes must be 4-byte aligned");
  PP_REQUIRE(aligned(a, 16) && (M == 1 || (a_sm >= K && a_sm % 8 == 0)),
             "activations must be 16-byte aligned with a row stride that is a multiple of 8");
  PP_REQUIRE(o_sm >= N, "o_sm must be >= N");
  PP_REQUIRE(slices >= 1 && slice_cols >= 32 && slice_cols % 32 == 0 && slices * slice_cols >= K &&
                 (slices - 1) * slice_cols < K,
             "slices x slice_cols must cover K in multiples of 32 columns");
  PP_REQUIRE(plug_n >= 0 && (plug_n == 0 || (plug_idx && plug_vals && row_plug)), "plug arrays are null");
  PP_REQUIRE(plug_n < (1ll << 28), "at most 2^28 plug entries");
  PP_REQUIRE((kn ? K * ldc * 4 : QB_ROWS * ldc * 4) < (1ll << 31) && (M - 1) * a_sm + K < (1ll << 30),
             "the codes a launch walks and the activations must each stay below 2 GiB");
  const int64_t need = pp_quad_big_workspace_size(M, N, slices);
  PP_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need), "workspace too small: need %lld bytes",
             (long long)need);
  PP_REQUIRE(need == 0 || aligned(workspace, 16), "the workspace must be 16-byte aligned");
  QuadBigArgs A = {};
  A.codes = codes;
  A.ldc = ldc;
  A.x = reinterpret_cast<const f16*>(a);
  A.x_sm = M > 1 ? a_sm : K;
  bool vec = o_sm % 4 == 0;
  for (int m = 0; m < 4; ++m) {
    A.out[m] = reinterpret_cast<f16*>(out[m]);
    vec = vec && aligned(out[m], 8);
  }
  A.vec_out = vec;
  A.o_sm = o_sm;
  A.N = (int)N;
  A.K = (int)K;
  A.M = (int)M;
  const int tt = qb_tt(M);
  A.tiles = (int)((N + QB_ROWS - 1) / QB_ROWS);
  A.tblocks = (int)((M + 16 * tt - 1) / (16 * tt));
  A.slices = (int)slices;
  A.ks = (int)slice_cols;
  for (int i = 0; i < 7; ++i) A.luts.p[i] = luts[i];
  A.luts.dtype = lut_dtype;
  for (int m = 0; m < 4; ++m) A.s[m] = scales[m];
  A.plug = PlugSrc{plug_idx, reinterpret_cast<const f16*>(plug_vals), plug_n};
  A.row_plug = row_plug;
  A.ppos0 = plug_pos0;
  A.pld = plug_ld;
  A.acc = reinterpret_cast<float*>(workspace);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (pc_use(M, kn)) {
    const int ptt = pc_tt(M, N);
    A.tiles = (int)((N + PC_ROWS - 1) / PC_ROWS);
    A.tblocks = (int)((M + 64 * ptt - 1) / (64 * ptt));
    const int64_t items = (int64_t)A.tiles * A.tblocks * slices;
    const int64_t grid = std::min<int64_t>(device_cu_count(), items);
    A.xcd_remap = grid % 8 == 0;
    const dim3 g((unsigned)grid), b(PC_NT);
    if (ptt == 1) {
      if (kn) hipLaunchKernelGGL((quad_big_pc_kernel<true, 1>), g, b, 0, st, A);
      else hipLaunchKernelGGL((quad_big_pc_kernel<false, 1>), g, b, 0, st, A);
    } else if (ptt == 2) {
      if (kn) hipLaunchKernelGGL((quad_big_pc_kernel<true, 2>), g, b, 0, st, A);
      else hipLaunchKernelGGL((quad_big_pc_kernel<false, 2>), g, b, 0, st, A);
    } else {
      if (kn) hipLaunchKernelGGL((quad_big_pc_kernel<true, 4>), g, b, 0, st, A);
      else hipLaunchKernelGGL((quad_big_pc_kernel<false, 4>), g, b, 0, st, A);
    }
  } else {
  const int64_t wv = qb_waves(tt, kn);
  const int64_t groups = (int64_t)(A.tiles + wv - 1) / wv * A.tblocks * slices;
  const int64_t cus = device_cu_count();
  int64_t grid = std::min<int64_t>(cus, groups);
  A.xcd_remap = grid % 8 == 0;
  switch (tt) {
    case 1: qb_launch<1>(kn, grid, st, A); break;
    case 2: qb_launch<2>(kn, grid, st, A); break;
    default: qb_launch<4>(kn, grid, st, A); break;
  }
  }
  PP_LAUNCH_CHECK();
  if (slices > 1) {
    hipLaunchKernelGGL(quad_big_finish_kernel, dim3((unsigned)finish_tiles(4, N, M)), dim3(256), 0, st, A.acc,
                       A.out[0], A.out[1], A.out[2], A.out[3], o_sm, A.N, A.M, (bool)A.vec_out);
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
}
