// Fused dual-pack decode GEMV for codes laid out (K,N) with unit column stride: the
// layout quantize_polar_bitpacked returns (polar_kernels.py:118-140) and
// polar_dual_bitpacked_kernel reads (polar_kernels.py:27-95), for 1..8 tokens per launch.
//
//   out_m[j, n] = fp16( sum_k a[j, k] * W_m[k, n] ),   m = 1, 2,
//   W_1 = amp cos_lut[phase],  W_2 = amp sin_lut[phase],
//   amp = amp_lut[amp_q] * bmax[(k*N + n) / gs]            (polar_kernels.py:64-79)
//
// with the LDS tables of dual_lds.h.  Work item = 512 columns x one slice of rows, one
// wavefront: lane l owns columns n0 + 8l .. +7 (one 16-byte load per row; 8 tokens: 256
// columns, 4 per lane, so the accumulators fit in registers), 8 rows per step,
// the next step's loads in flight while one is decoded.  The 8 codes of a lane and row
// share one group scale (gs is a power of two >= 8 and N % 8 == 0, so (k*N + n) / gs is
// the same for the 8 columns), one 2-byte load per row; the activations of a row are the
// same for every lane (one 16-byte load of 8 rows per token).  Each lane keeps its own 8
// columns' sums, so no cross-lane reduction.  With one slice and no plug table the wave
// writes its fp16 outputs; otherwise every slice stores its float32 partial sums
// [slice][m][j][n], plug corrections are added to slice 0 by dual_kn_plug_kernel (one
// thread per entry) and dual_kn_finish_kernel sums the slices into the fp16 outputs.
#include "dual_kn.h"
#include "dual_lds.h"
#include "rows_common.h"

namespace pp {

constexpr int DKN_R = 8;       // rows per step
constexpr int DKN_NT = 512;    // threads per workgroup (one per CU: the tables take most of LDS)

struct DualKnArgs {
  const uint16_t* codes;   // code of (row 0, col 0); row k at codes + k*ldk
  int64_t ldk;
  const f16* a;            // (M, K), row stride a_sm, unit column stride
  int64_t a_sm;
  f16* out[2];             // (M, N): element (j, n) at out + j*o_sm + n*o_sn
  int64_t o_sm, o_sn;
  int M, N, K;
  int slices, ks;          // K slices of ks rows (a multiple of DKN_R)
  int64_t nblk;            // ceil(N / (64 * codes per lane))
  const f16* scales;       // bmax, one per group of gs consecutive (k*N + n)
  int64_t n_groups;
  int log2gs;
  DualLuts luts;
  float* part;             // partial sums [slice][2][M][N] (slices > 1 or plug), else null
};

// Tables from the caller's LUTs (fp16 or float32): every LUT load of a thread is issued
// before its stores, the (cos, sin) rows written as 16-byte units in address order.
template <int LAYOUT, typename E>
__device__ __forceinline__ void dkn_tables_of(char* lds, const DualLuts& L) {
  constexpr int KU = (8192 + DKN_NT - 1) / DKN_NT;
  const E* cp = reinterpret_cast<const E*>(L.cs[0]);
  const E* sp = reinterpret_cast<const E*>(L.cs[1]);
  float c[KU], s[KU];
#pragma unroll
  for (int k = 0; k < KU; ++k) {
    const int p = (threadIdx.x + k * DKN_NT) >> 3;
    c[k] = p < L.phase_n ? (float)cp[p] : 0.f;
    s[k] = p < L.phase_n ? (float)sp[p] : 0.f;
  }
  float amp = 0.f;
  if (threadIdx.x < 64) {
    // the int16 layout stores code ^ 0x8000: entry a holds amplitude a ^ 32
    const int e = LAYOUT == PP_DUAL_I16_OFFSET ? (threadIdx.x ^ 32) : threadIdx.x;
    amp = e < L.amp_n ? (float)reinterpret_cast<const E*>(L.amp)[e] : 0.f;
    *reinterpret_cast<float*>(lds + DLDS_AMP + 4 * threadIdx.x) = amp;
  }
#pragma unroll
  for (int k = 0; k < KU; ++k)
    *reinterpret_cast<float4*>(lds + DLDS_CS + 16 * (threadIdx.x + k * DKN_NT)) = make_float4(c[k], s[k], c[k], s[k]);
}

// CL codes (columns) per lane and row: 8 (16-byte loads) for 1-4 tokens, 4 (8-byte
// loads) for 8 tokens, where the accumulators of 8 columns would not fit in registers.
template <int CL> struct DknVec;
template <> struct DknVec<8> { typedef u32x4 T; };
template <> struct DknVec<4> { typedef u32x2 T; };

template <int MT, int CL>
struct DknStep {
  typename DknVec<CL>::T q[DKN_R];   // CL codes (columns) per row
  uint32_t sc[DKN_R];                 // their group scale (fp16 bits)
  u32x4 x[MT];                        // 8 fp16 activations (the step's rows) per token
};

template <int MT, int CL>
__device__ __forceinline__ void dkn_issue(const DualKnArgs& A, int k, int kend, int n, uint32_t voff,
                                          DknStep<MT, CL>& S) {
  // rows [k, kend) of the slice: the resource ends at row kend, so rows past it read 0
  const int rows = max(0, kend - k);
  const rsrc_t rc = make_rsrc(A.codes + (int64_t)min(k, kend) * A.ldk, 2u * (uint32_t)((int64_t)rows * A.ldk));
#pragma unroll
  for (int r = 0; r < DKN_R; ++r) {
    if constexpr (CL == 8) vload128(S.q[r], voff + 2u * (uint32_t)(r * A.ldk), rc);
    else S.q[r] = __builtin_amdgcn_raw_buffer_load_b64(rc, (int)(voff + 2u * (uint32_t)(r * A.ldk)), 0, NT_AUX);
  }
  const rsrc_t rs = make_rsrc(A.scales, 2u * (uint32_t)A.n_groups);
#pragma unroll
  for (int r = 0; r < DKN_R; ++r) {
    // group of (k + r, n .. n+CL-1); K*N < 2^32 on this path
    const uint32_t p = (uint32_t)(k + r) * (uint32_t)A.N + (uint32_t)n;
    vload16(S.sc[r], r < rows && n < A.N ? 2u * (p >> A.log2gs) : OOB, rs);
  }
#pragma unroll
  for (int j = 0; j < MT; ++j) {
    // 8 activations of the step's rows: past kend they read 0 (with the codes, they add 0)
    const rsrc_t rx = make_rsrc(A.a + (int64_t)j * A.a_sm + min(k, kend), 2u * (uint32_t)rows);
    vload128c(S.x[j], j < A.M ? 0u : OOB, rx);
  }
}

// Table entries of one row's CL codes.
template <int CL>
struct DknRowLk {
  float an[CL];
  float2 cs[CL];
};

template <int LAYOUT, int CL>
__device__ __forceinline__ void dkn_lookup_row(const char* lds, const DualLane& lo,
                                               const typename DknVec<CL>::T& q, DknRowLk<CL>& L) {
#pragma unroll
  for (int e = 0; e < CL / 2; ++e) {
    float an[2];
    float2 cs[2];
    dual_lookup2<LAYOUT>(lds, q[e], lo, an, cs);
    L.an[2 * e] = an[0];
    L.an[2 * e + 1] = an[1];
    L.cs[2 * e] = cs[0];
    L.cs[2 * e + 1] = cs[1];
  }
}

// Activation of token j, row r of the step, converted on use.
template <int MT>
__device__ __forceinline__ float dkn_x(const u32x4 (&x)[MT], int j, int r) {
  const uint32_t w = r < 2 ? x[j].x : r < 4 ? x[j].y : r < 6 ? x[j].z : x[j].w;
  return h2f((r & 1) ? (w >> 16) : (w & 0xFFFFu));
}

// The lookups of row r + 1 are issued before the arithmetic of row r (the barrier keeps
// the compiler from moving them back behind it), so a wave has a row of LDS reads in
// flight while it multiplies.
template <int MT, int CL, int LAYOUT>
__device__ __forceinline__ void dkn_compute(const char* lds, const DualLane& lo, const DknStep<MT, CL>& S,
                                            float (&acc)[CL][2][MT]) {
  DknRowLk<CL> buf[2];
  dkn_lookup_row<LAYOUT, CL>(lds, lo, S.q[0], buf[0]);
#pragma unroll
  for (int r = 0; r < DKN_R; ++r) {
    if (r + 1 < DKN_R) dkn_lookup_row<LAYOUT, CL>(lds, lo, S.q[r + 1], buf[(r + 1) & 1]);
    __builtin_amdgcn_sched_barrier(0);
    const DknRowLk<CL>& L = buf[r & 1];
    const float sc = h2f(S.sc[r]);
    float xs[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) xs[j] = dkn_x<MT>(S.x, j, r) * sc;
#pragma unroll
    for (int c = 0; c < CL; ++c)
#pragma unroll
      for (int j = 0; j < MT; ++j) {
        const float t = L.an[c] * xs[j];
        acc[c][0][j] = fmaf(t, L.cs[c].x, acc[c][0][j]);
        acc[c][1][j] = fmaf(t, L.cs[c].y, acc[c][1][j]);
      }
  }
}

// A wave's item: its 64 * CL columns and row slice.
struct DknItem {
  int n, k0, k1, sl;
  uint32_t voff;
};

template <int CL>
__device__ __forceinline__ DknItem dkn_item(const DualKnArgs& A, int64_t it, int lane) {
  DknItem I;
  const int blk = (int)uniform64(it / A.slices);
  I.sl = (int)uniform64(it % A.slices);
  I.n = blk * 64 * CL + CL * lane;          // the lane's first column
  I.k0 = I.sl * A.ks;
  I.k1 = min(A.K, I.k0 + A.ks);
  I.voff = I.n < A.N ? 2u * (uint32_t)I.n : OOB;
  return I;
}

// One item, its first step already issued into s0.
template <int MT, int CL, int LAYOUT>
__device__ __forceinline__ void dkn_run(const char* lds, const DualLane& lo, const DualKnArgs& A, const DknItem& I,
                                        DknStep<MT, CL>& s0, DknStep<MT, CL>& s1) {
  float acc[CL][2][MT];
#pragma unroll
  for (int c = 0; c < CL; ++c)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[c][0][j] = acc[c][1][j] = 0.f;
  for (int k = I.k0; k < I.k1; k += 2 * DKN_R) {
    dkn_issue<MT, CL>(A, k + DKN_R, I.k1, I.n, I.voff, s1);
    dkn_compute<MT, CL, LAYOUT>(lds, lo, s0, acc);
    if (k + DKN_R >= I.k1) break;
    dkn_issue<MT, CL>(A, k + 2 * DKN_R, I.k1, I.n, I.voff, s0);
    dkn_compute<MT, CL, LAYOUT>(lds, lo, s1, acc);
  }
  const int n = I.n;
  if (A.part == nullptr) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const rsrc_t ro = make_rsrc(A.out[m], 2u * (uint32_t)((int64_t)(A.M - 1) * A.o_sm + (int64_t)(A.N - 1) * A.o_sn + 1));
#pragma unroll
      for (int j = 0; j < MT; ++j)
#pragma unroll
        for (int c = 0; c < CL; ++c) {
          const f16 h = (f16)acc[c][m][j];
          const bool ok = n + c < A.N && j < A.M;
          vstore16((uint32_t)__builtin_bit_cast(unsigned short, h),
                   ok ? 2u * (uint32_t)((int64_t)j * A.o_sm + (int64_t)(n + c) * A.o_sn) : OOB, ro);
        }
    }
  } else {
    // partials [sl][m][j][n .. n+CL-1] as 16-byte stores (N % 8 == 0 on this path)
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int j = 0; j < MT; ++j)
        if (n < A.N && j < A.M) {
          float4* p = reinterpret_cast<float4*>(A.part + (((int64_t)I.sl * 2 + m) * A.M + j) * A.N + n);
#pragma unroll
          for (int h = 0; h < CL / 4; ++h)
            p[h] = make_float4(acc[4 * h][m][j], acc[4 * h + 1][m][j], acc[4 * h + 2][m][j], acc[4 * h + 3][m][j]);
        }
  }
}

template <int MT, int CL, int LAYOUT>
__global__ __launch_bounds__(DKN_NT) void dual_kn_kernel(const DualKnArgs A) {
  __shared__ __attribute__((aligned(16))) char T[DLDS_BYTES];
  constexpr int WAVES = DKN_NT / 64;
  const int lane = threadIdx.x & 63;
  const DualLane lo = dual_lane(lane);
  // items dealt round-robin over the workgroups, so a launch with fewer items than
  // wavefronts still spreads them over every CU
  const int64_t gw = (int64_t)uniform(threadIdx.x >> 6) * gridDim.x + blockIdx.x;
  const int64_t nw = (int64_t)gridDim.x * WAVES;
  const int64_t items = A.nblk * A.slices;
  // the first item's first loads travel while the tables are built (1-2 tokens: with
  // more they would stay live through the build and spill)
  constexpr bool early = MT <= 2;
  DknStep<MT, CL> s0, s1;
  DknItem I = dkn_item<CL>(A, gw < items ? gw : 0, lane);
  if (early && gw < items) dkn_issue<MT, CL>(A, I.k0, I.k1, I.n, I.voff, s0);
  if (A.luts.dtype == PP_F16) dkn_tables_of<LAYOUT, f16>(T, A.luts);
  else dkn_tables_of<LAYOUT, float>(T, A.luts);
  __syncthreads();
  for (int64_t it = gw; it < items; it += nw) {
    if (it != gw || !early) {
      I = dkn_item<CL>(A, it, lane);
      dkn_issue<MT, CL>(A, I.k0, I.k1, I.n, I.voff, s0);
    }
    dkn_run<MT, CL, LAYOUT>(T, lo, A, I, s0, s1);
  }
}

// Plug corrections, one entry per thread, added to slice 0's partial sums after the
// tile kernel: x * (plug amp - amp_lut[amp_q] * bmax) * (cos, sin)(phase) for every token
// (the plug amplitude replaces the decoded one, polar_bitpack.py:240-243).  Positions are
// relative to elem_base in the (K,N) storage, row stride ldk.
struct DualKnPlugArgs {
  DualKnArgs T;
  int layout;
  const uint32_t* plug_idx;
  const f16* plug_amp;
  int64_t plug_n, elem_base;
};

__global__ __launch_bounds__(256) void dual_kn_plug_kernel(const DualKnPlugArgs P) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= P.plug_n) return;
  const DualKnArgs& A = P.T;
  const int64_t pos = (int64_t)P.plug_idx[e] - P.elem_base;
  if (pos < 0) return;
  const int64_t k = pos / A.ldk, n = pos % A.ldk;
  if (k >= A.K || n >= A.N) return;
  const uint32_t raw = A.codes[pos];
  const uint32_t code = P.layout == PP_DUAL_U16_BE ? (((raw & 0xFFu) << 8) | (raw >> 8)) : (raw ^ 0x8000u);
  const int aq = (int)((code >> 10) & 63u), ph = (int)(code & 1023u);
  const DualLuts& L = A.luts;
  const float an = aq < L.amp_n ? lut_at(L.amp, L.dtype, aq) : 0.f;
  const float c = ph < L.phase_n ? lut_at(L.cs[0], L.dtype, ph) : 0.f;
  const float s = ph < L.phase_n ? lut_at(L.cs[1], L.dtype, ph) : 0.f;
  const float sc = (float)A.scales[(k * A.N + n) >> A.log2gs];
  const float d = (float)P.plug_amp[e] - an * sc;
  for (int j = 0; j < A.M; ++j) {
    const float xd = (float)A.a[(int64_t)j * A.a_sm + k] * d;
    atomicAdd(A.part + (int64_t)j * A.N + n, xd * c);
    atomicAdd(A.part + ((int64_t)A.M + j) * A.N + n, xd * s);
  }
}

// out_m[j, n] = fp16(sum over slices of part[sl][m][j][n]): a workgroup takes 64 runs of
// 4 consecutive columns (N % 8 == 0 on this path), its 8 wavefronts every 8th slice each,
// summed through LDS, so the slices' loads are in flight together.
constexpr int KN_FIN_NT = 512;

__global__ __launch_bounds__(KN_FIN_NT) void dual_kn_finish_kernel(const DualKnArgs A) {
  __shared__ float4 red[KN_FIN_NT / 64][64];
  const int lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int64_t total = 2ll * A.M * A.N;
  const int64_t i0 = 4 * ((int64_t)blockIdx.x * 64 + lane);
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (i0 < total) {
#pragma unroll 4
    for (int sl = grp; sl < A.slices; sl += KN_FIN_NT / 64) {
      const float4 t = *reinterpret_cast<const float4*>(A.part + (int64_t)sl * total + i0);
      v.x += t.x;
      v.y += t.y;
      v.z += t.z;
      v.w += t.w;
    }
  }
  red[grp][lane] = v;
  __syncthreads();
  if (grp != 0 || i0 >= total) return;
#pragma unroll
  for (int g = 1; g < KN_FIN_NT / 64; ++g) {
    const float4 t = red[g][lane];
    v.x += t.x;
    v.y += t.y;
    v.z += t.z;
    v.w += t.w;
  }
  const int64_t mj = i0 / A.N;
  const int n = (int)(i0 % A.N), j = (int)(mj % A.M), m = (int)(mj / A.M);
  f16* o = m == 0 ? A.out[0] : A.out[1];
  const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int c = 0; c < 4; ++c) o[(int64_t)j * A.o_sm + (int64_t)(n + c) * A.o_sn] = (f16)vv[c];
}

// ------------------------------------------------------------------ host side
#ifndef PP_DKN_MIN_ROWS
#define PP_DKN_MIN_ROWS 16   // slices of at least this many rows (4096x4096: 1..4 tokens measured best)
#endif

struct DknPlan {
  int slices, ks;
  int64_t nblk;
};

// Codes (columns) per lane for a block of M tokens.
static int dkn_cl(int64_t M) { return M <= 4 ? 8 : 4; }

static DknPlan dkn_plan(int64_t M, int64_t N, int64_t K) {
  DknPlan p;
  const int64_t cols = 64 * dkn_cl(M);
  p.nblk = (N + cols - 1) / cols;
  const int64_t waves = (int64_t)device_cu_count() * (DKN_NT / 64);
  // about one item per wavefront, slices of at least PP_DKN_MIN_ROWS rows
  int64_t s = std::max<int64_t>(
      1, std::min<int64_t>(waves / std::max<int64_t>(p.nblk, 1), (K + PP_DKN_MIN_ROWS - 1) / PP_DKN_MIN_ROWS));
  int64_t ks = (K + s - 1) / s;
  ks = (ks + DKN_R - 1) / DKN_R * DKN_R;
  p.ks = (int)std::max<int64_t>(ks, DKN_R);
  p.slices = (int)((K + p.ks - 1) / p.ks);
  return p;
}

bool dual_kn_ok(const void* a, int64_t a_sm, int64_t a_sk, const void* codes, int64_t c_sk, int64_t c_sn,
                int64_t group_size, int64_t chunk_size, int64_t M, int64_t N, int64_t K) {
  return c_sn == 1 && c_sk >= N && c_sk % 8 == 0 && N % 8 == 0 && N > 0 && K > 0 && K % 8 == 0 && M >= 1 &&
         M <= 8 && aligned(codes, 16) && chunk_size == 0 && group_size >= 8 && (group_size & (group_size - 1)) == 0 &&
         a_sk == 1 && (M == 1 || a_sm % 8 == 0) && aligned(a, 16) && K * N < (1ll << 32) &&
         2 * c_sk * K < (1ll << 31);
}

int64_t dual_kn_workspace(int64_t M, int64_t N, int64_t K, int64_t plug_n) {
  const DknPlan p = dkn_plan(M, N, K);
  if (p.slices == 1 && plug_n == 0) return 0;
  return (int64_t)p.slices * 2 * M * N * (int64_t)sizeof(float);
}

int dual_kn_gemm(const void* a, int64_t a_sm, const void* codes, int code_layout, int64_t ldk, const void* bmax,
                 int64_t group_size, const DualLuts& luts, const uint32_t* plug_idx, const void* plug_amp,
                 int64_t plug_n, int64_t elem_base, void* const* out, int64_t o_sm, int64_t o_sn, int64_t M,
                 int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, hipStream_t st) {
  const DknPlan p = dkn_plan(M, N, K);
  const int64_t need = dual_kn_workspace(M, N, K, plug_n);
  PP_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need), "workspace too small: need %lld bytes",
             (long long)need);
  DualKnArgs A = {};
  A.codes = reinterpret_cast<const uint16_t*>(codes);
  A.ldk = ldk;
  A.a = reinterpret_cast<const f16*>(a);
  A.a_sm = a_sm;
  A.out[0] = reinterpret_cast<f16*>(out[0]);
  A.out[1] = reinterpret_cast<f16*>(out[1]);
  A.o_sm = o_sm;
  A.o_sn = o_sn;
  A.M = (int)M;
  A.N = (int)N;
  A.K = (int)K;
  A.slices = p.slices;
  A.ks = p.ks;
  A.nblk = p.nblk;
  A.scales = reinterpret_cast<const f16*>(bmax);
  A.n_groups = (K * N + group_size - 1) / group_size;
  A.log2gs = 0;
  while ((1ll << A.log2gs) < group_size) ++A.log2gs;
  A.luts = luts;
  A.part = need > 0 ? reinterpret_cast<float*>(workspace) : nullptr;
  const int64_t items = p.nblk * p.slices;
  const unsigned grid = (unsigned)std::min<int64_t>(device_cu_count(), (items + DKN_NT / 64 - 1) / (DKN_NT / 64));
  const bool be = code_layout == PP_DUAL_U16_BE;
  switch ((M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8) * 2 + (be ? 1 : 0)) {
    case 2: hipLaunchKernelGGL((dual_kn_kernel<1, 8, PP_DUAL_I16_OFFSET>), dim3(grid), dim3(DKN_NT), 0, st, A); break;
    case 3: hipLaunchKernelGGL((dual_kn_kernel<1, 8, PP_DUAL_U16_BE>), dim3(grid), dim3(DKN_NT), 0, st, A); break;
    case 4: hipLaunchKernelGGL((dual_kn_kernel<2, 8, PP_DUAL_I16_OFFSET>), dim3(grid), dim3(DKN_NT), 0, st, A); break;
    case 5: hipLaunchKernelGGL((dual_kn_kernel<2, 8, PP_DUAL_U16_BE>), dim3(grid), dim3(DKN_NT), 0, st, A); break;
    case 8: hipLaunchKernelGGL((dual_kn_kernel<4, 8, PP_DUAL_I16_OFFSET>), dim3(grid), dim3(DKN_NT), 0, st, A); break;
    case 9: hipLaunchKernelGGL((dual_kn_kernel<4, 8, PP_DUAL_U16_BE>), dim3(grid), dim3(DKN_NT), 0, st, A); break;
    case 16: hipLaunchKernelGGL((dual_kn_kernel<8, 4, PP_DUAL_I16_OFFSET>), dim3(grid), dim3(DKN_NT), 0, st, A); break;
    default: hipLaunchKernelGGL((dual_kn_kernel<8, 4, PP_DUAL_U16_BE>), dim3(grid), dim3(DKN_NT), 0, st, A); break;
  }
  PP_LAUNCH_CHECK();
  if (A.part != nullptr) {
    if (plug_n > 0) {
      DualKnPlugArgs P;
      P.T = A;
      P.layout = code_layout;
      P.plug_idx = plug_idx;
      P.plug_amp = reinterpret_cast<const f16*>(plug_amp);
      P.plug_n = plug_n;
      P.elem_base = elem_base;
      hipLaunchKernelGGL(dual_kn_plug_kernel, dim3((unsigned)((plug_n + 255) / 256)), dim3(256), 0, st, P);
      PP_LAUNCH_CHECK();
    }
    const int64_t total = 2 * M * N;
    hipLaunchKernelGGL(dual_kn_finish_kernel, dim3((unsigned)((total / 4 + 63) / 64)), dim3(KN_FIN_NT), 0, st, A);
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
}

}  // namespace pp
