// Fused quad-pack decode GEMV for codes laid out (K,N) with unit column stride: the
// layout pack_quad_layer returns (quad_kernels.py:35-37) and quad_bitpacked_kernel reads
// (quad_kernels.py:53-143), for 1..8 tokens per launch.
//
//   out_m[j, n] = fp16( s_m * sum_k a[j, k] * W_m[k, n] ),   m = 0..3,
//
// W_m decoded from the word [nq|q1|q2|q3] with the LDS tables of quad_lds.h
// (quad_kernels.py:103-121).  Work item = 256 columns x one slice of rows, one wavefront:
// lane l owns columns n0 + 4l .. +3 (one 16-byte load per row, a wavefront reads 1 KiB of
// one row per instruction), 8 rows per step, the next step's loads in flight while one is
// decoded.  The activations of a row are the same for every lane (one 16-byte load of 8
// rows per token).  Each lane keeps its own 4 columns' sums, so no cross-lane reduction.
// With one slice and no plug table the wave writes its fp16 outputs; otherwise every
// slice stores its float32 partial sums [slice][m][j][n], plug corrections are added to
// slice 0 by quad_kn_plug_kernel (one thread per entry) and quad_kn_finish_kernel sums the
// slices into the fp16 outputs.
#include "quad_kn.h"
#include "quad_lds.h"
#include "rows_common.h"

namespace pp {

constexpr int KN_R = 8;        // rows per step
constexpr int KN_NT = 512;     // threads per workgroup (one per CU: the tables take all of LDS)

struct QuadKnArgs {
  const uint32_t* codes;   // code of (row 0, col 0); row k at codes + k*ldk
  int64_t ldk;
  const f16* a;            // (M, K), row stride a_sm, unit column stride
  int64_t a_sm;
  f16* out[4];             // (M, N): element (j, n) at out + j*o_sm + n*o_sn
  int64_t o_sm, o_sn;
  int M, N, K;
  int slices, ks;          // K slices of ks rows (a multiple of KN_R)
  int64_t nblk;            // ceil(N / (64 * columns per lane))
  QuadLuts luts;
  float s[4];
  float* part;             // partial sums [slice][4][M][N] (slices > 1 or plug), else null
};

// CL columns (code words) per lane and row: 4 (16-byte loads) for 1-4 tokens, 2 (8-byte
// loads) for 8 tokens, where the accumulators of 4 columns would not fit in registers.
template <int CL> struct KnVec;
template <> struct KnVec<4> { typedef u32x4 T; };
template <> struct KnVec<2> { typedef u32x2 T; };

template <int MT, int CL>
struct KnStep {
  typename KnVec<CL>::T q[KN_R];   // CL words (columns) per row
  u32x4 x[MT];                      // 8 fp16 activations (the step's rows) per token
};

template <int MT, int CL>
__device__ __forceinline__ void kn_issue(const QuadKnArgs& A, int k, int kend, uint32_t voff, KnStep<MT, CL>& S) {
  // rows [k, kend) of the slice: the resource ends at row kend, so rows past it read 0
  const int rows = max(0, kend - k);
  const rsrc_t rc = make_rsrc(A.codes + (int64_t)min(k, kend) * A.ldk, 4u * (uint32_t)((int64_t)rows * A.ldk));
#pragma unroll
  for (int r = 0; r < KN_R; ++r) {
    if constexpr (CL == 4) vload128(S.q[r], voff + 4u * (uint32_t)(r * A.ldk), rc);
    else S.q[r] = __builtin_amdgcn_raw_buffer_load_b64(rc, (int)(voff + 4u * (uint32_t)(r * A.ldk)), 0, NT_AUX);
  }
#pragma unroll
  for (int j = 0; j < MT; ++j) {
    // 8 activations of the step's rows: past kend they read 0 (with the codes, they add 0)
    const rsrc_t rx = make_rsrc(A.a + (int64_t)j * A.a_sm + min(k, kend), 2u * (uint32_t)rows);
    vload128c(S.x[j], j < A.M ? 0u : OOB, rx);
  }
}

// Table entries of one code word.
struct KnTup {
  float r;
  float2 a, b, c;
};

// Activation of token j, row r of the step (fp16 -> float on use: 8 tokens' converted
// rows would not fit in registers next to their accumulators).
template <int MT>
__device__ __forceinline__ float kn_x(const u32x4 (&x)[MT], int j, int r) {
  const uint32_t w = r < 2 ? x[j].x : r < 4 ? x[j].y : r < 6 ? x[j].z : x[j].w;
  return h2f((r & 1) ? (w >> 16) : (w & 0xFFFFu));
}

template <int MT, int CL, class L>
__device__ __forceinline__ void kn_compute(const char* lds, const LaneOff& lo, const KnStep<MT, CL>& S,
                                           float (&acc)[CL][4][MT]) {
  // tuple t = row r * CL + column c; lookups two tuples ahead of the arithmetic
  auto word = [&](int t) -> uint32_t {
    const int c = t % CL;
    if constexpr (CL == 4) {
      const u32x4& q = S.q[t / 4];
      return c == 0 ? q.x : c == 1 ? q.y : c == 2 ? q.z : q.w;
    } else {
      const u32x2& q = S.q[t / 2];
      return c == 0 ? q.x : q.y;
    }
  };
  constexpr int GT = 2, NTUP = KN_R * CL, NG = NTUP / GT;
  KnTup buf[2][GT];
#pragma unroll
  for (int u = 0; u < GT; ++u) lookup<L>(lds, word(u), lo, buf[0][u].r, buf[0][u].a, buf[0][u].b, buf[0][u].c);
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (g + 1 < NG) {
#pragma unroll
      for (int u = 0; u < GT; ++u) {
        KnTup& T = buf[(g + 1) & 1][u];
        lookup<L>(lds, word((g + 1) * GT + u), lo, T.r, T.a, T.b, T.c);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < GT; ++u) {
      const int t = g * GT + u, r = t / CL, c = t % CL;
      const KnTup& T = buf[g & 1][u];
      if constexpr (MT == 1) {
        const float rx = T.r * kn_x<MT>(S.x, 0, r);
        acc[c][0][0] = fmaf(rx, T.a.x, acc[c][0][0]);
        const float t1 = rx * T.a.y;
        acc[c][1][0] = fmaf(t1, T.b.x, acc[c][1][0]);
        const float t2 = t1 * T.b.y;
        acc[c][2][0] = fmaf(t2, T.c.x, acc[c][2][0]);
        acc[c][3][0] = fmaf(t2, T.c.y, acc[c][3][0]);
      } else {
        const float rs = T.r * T.a.y;
        const float rss = rs * T.b.y;
        const float w[4] = {T.r * T.a.x, rs * T.b.x, rss * T.c.x, rss * T.c.y};
#pragma unroll
        for (int j = 0; j < MT; ++j) {
          const float xj = kn_x<MT>(S.x, j, r);
#pragma unroll
          for (int m = 0; m < 4; ++m) acc[c][m][j] = fmaf(w[m], xj, acc[c][m][j]);
        }
      }
    }
  }
}

// A wave's item: its 64 * CL columns and row slice.
struct KnItem {
  int n, k0, k1, sl;
  uint32_t voff;
};

template <int CL>
__device__ __forceinline__ KnItem kn_item(const QuadKnArgs& A, int64_t it, int lane) {
  KnItem I;
  const int blk = (int)uniform64(it / A.slices);
  I.sl = (int)uniform64(it % A.slices);
  I.n = blk * 64 * CL + CL * lane;          // the lane's first column
  I.k0 = I.sl * A.ks;
  I.k1 = min(A.K, I.k0 + A.ks);
  I.voff = I.n < A.N ? 4u * (uint32_t)I.n : OOB;
  return I;
}

// One item, its first step already issued into s0.
template <int MT, int CL, class L>
__device__ __forceinline__ void kn_run(const char* lds, const LaneOff& lo, const QuadKnArgs& A, const KnItem& I,
                                       KnStep<MT, CL>& s0, KnStep<MT, CL>& s1) {
  float acc[CL][4][MT];
#pragma unroll
  for (int c = 0; c < CL; ++c)
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int j = 0; j < MT; ++j) acc[c][m][j] = 0.f;
  for (int k = I.k0; k < I.k1; k += 2 * KN_R) {
    kn_issue<MT, CL>(A, k + KN_R, I.k1, I.voff, s1);
    kn_compute<MT, CL, L>(lds, lo, s0, acc);
    if (k + KN_R >= I.k1) break;
    kn_issue<MT, CL>(A, k + 2 * KN_R, I.k1, I.voff, s0);
    kn_compute<MT, CL, L>(lds, lo, s1, acc);
  }
  const int n = I.n;
  if (A.part == nullptr) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const rsrc_t ro = make_rsrc(A.out[m], 2u * (uint32_t)((int64_t)(A.M - 1) * A.o_sm + (int64_t)(A.N - 1) * A.o_sn + 1));
#pragma unroll
      for (int j = 0; j < MT; ++j)
#pragma unroll
        for (int c = 0; c < CL; ++c) {
          const f16 h = (f16)(acc[c][m][j] * A.s[m]);
          const bool ok = n + c < A.N && j < A.M;
          vstore16((uint32_t)__builtin_bit_cast(unsigned short, h),
                   ok ? 2u * (uint32_t)((int64_t)j * A.o_sm + (int64_t)(n + c) * A.o_sn) : OOB, ro);
        }
    }
  } else {
    // partials [sl][m][j][n .. n+CL-1] as one 16- or 8-byte store (N % 4 == 0 on this path)
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int j = 0; j < MT; ++j)
        if (n < A.N && j < A.M) {
          float* p = A.part + (((int64_t)I.sl * 4 + m) * A.M + j) * A.N + n;
          if constexpr (CL == 4)
            *reinterpret_cast<float4*>(p) = make_float4(acc[0][m][j] * A.s[m], acc[1][m][j] * A.s[m],
                                                        acc[2][m][j] * A.s[m], acc[3][m][j] * A.s[m]);
          else
            *reinterpret_cast<float2*>(p) = make_float2(acc[0][m][j] * A.s[m], acc[1][m][j] * A.s[m]);
        }
  }
}

// With 4 tokens the early loads would stay live through the table build and spill.
template <int MT>
constexpr bool kn_early() { return MT <= 2; }

template <int MT, int CL, class L>
__device__ __forceinline__ void kn_items(const char* lds, const QuadKnArgs& A, int64_t gw, int64_t nw, int lane,
                                         KnItem I, KnStep<MT, CL>& s0, KnStep<MT, CL>& s1) {
  const LaneOff lo = L::lane(lane);
  const int64_t items = A.nblk * A.slices;
  for (int64_t it = gw; it < items; it += nw) {
    if (it != gw || !kn_early<MT>()) {
      I = kn_item<CL>(A, it, lane);
      kn_issue<MT, CL>(A, I.k0, I.k1, I.voff, s0);
    }
    kn_run<MT, CL, L>(lds, lo, A, I, s0, s1);
  }
}

template <int MT, int CL>
__global__ __launch_bounds__(KN_NT) void quad_kn_kernel(const QuadKnArgs A) {
  __shared__ __attribute__((aligned(16))) uint32_t T[QLDS_BYTES / 4];
  const char* lds = reinterpret_cast<const char*>(T);
  constexpr int WAVES = KN_NT / 64;
  const int lane = threadIdx.x & 63;
  // items dealt round-robin over the workgroups, so a launch with fewer items than
  // wavefronts still spreads them over every CU
  const int64_t gw = (int64_t)uniform(threadIdx.x >> 6) * gridDim.x + blockIdx.x;
  const int64_t nw = (int64_t)gridDim.x * WAVES;
  const int64_t items = A.nblk * A.slices;
  // the first item's first loads travel while the tables are built (1-2 tokens)
  KnStep<MT, CL> s0, s1;
  const KnItem I = kn_item<CL>(A, gw < items ? gw : 0, lane);
  if (kn_early<MT>() && gw < items) kn_issue<MT, CL>(A, I.k0, I.k1, I.voff, s0);
  if (quad_tables<KN_NT>(T, A.luts)) kn_items<MT, CL, LayShared>(lds, A, gw, nw, lane, I, s0, s1);
  else kn_items<MT, CL, LaySplit>(lds, A, gw, nw, lane, I, s0, s1);
}

// Plug corrections, one entry per thread, added to slice 0's partial sums after the
// tile kernel: x * (plug - decoded) * s_m for every token (the entry's tuple decoded with
// the same tables, so the correction cancels its term up to float32 rounding;
// quaternion_packer.py:187-193 replaces the tuple).  Positions are relative to elem_base
// in the (K,N) storage, row stride ldk.
struct QuadKnPlugArgs {
  QuadKnArgs T;
  const uint32_t* plug_idx;
  const f16* plug_vals;   // (P, 4), normalised
  int64_t plug_n, elem_base;
};

template <typename E>
__device__ __forceinline__ void kn_decode(const QuadLuts& L, uint32_t cw, float (&w)[4]) {
  const float r = lut_val<E>(L, 0, cw >> 24);
  const float c1 = lut_val<E>(L, 1, (cw >> 16) & 255u), s1 = lut_val<E>(L, 2, (cw >> 16) & 255u);
  const float c2 = lut_val<E>(L, 3, (cw >> 8) & 255u), s2 = lut_val<E>(L, 4, (cw >> 8) & 255u);
  const float c3 = lut_val<E>(L, 5, cw & 255u), s3 = lut_val<E>(L, 6, cw & 255u);
  const float rs = r * s1, rss = rs * s2;
  w[0] = r * c1;
  w[1] = rs * c2;
  w[2] = rss * c3;
  w[3] = rss * s3;
}

__global__ __launch_bounds__(256) void quad_kn_plug_kernel(const QuadKnPlugArgs P) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= P.plug_n) return;
  const QuadKnArgs& A = P.T;
  const int64_t pos = (int64_t)P.plug_idx[e] - P.elem_base;
  if (pos < 0) return;
  const int64_t k = pos / A.ldk, n = pos % A.ldk;
  if (k >= A.K || n >= A.N) return;
  float w[4];
  const uint32_t cw = A.codes[pos];
  if (A.luts.dtype == PP_F16) kn_decode<f16>(A.luts, cw, w);
  else kn_decode<float>(A.luts, cw, w);
  const f16x4 pv = *reinterpret_cast<const f16x4*>(P.plug_vals + 4 * e);
  const float d[4] = {(float)pv.x - w[0], (float)pv.y - w[1], (float)pv.z - w[2], (float)pv.w - w[3]};
  for (int j = 0; j < A.M; ++j) {
    const float x = (float)A.a[(int64_t)j * A.a_sm + k];
#pragma unroll
    for (int m = 0; m < 4; ++m)
      atomicAdd(A.part + ((int64_t)m * A.M + j) * A.N + n, x * d[m] * A.s[m]);
  }
}

// out_m[j, n] = fp16(sum over slices of part[sl][m][j][n]): a workgroup takes 64 runs of
// 4 consecutive columns (N % 4 == 0 on this path), its 8 wavefronts every 8th slice each,
// summed through LDS, so the slices' loads are in flight together.
constexpr int KN_FIN_NT = 512;

__global__ __launch_bounds__(KN_FIN_NT) void quad_kn_finish_kernel(const QuadKnArgs A) {
  __shared__ float4 red[KN_FIN_NT / 64][64];
  const int lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int64_t total = 4ll * A.M * A.N;
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
  f16* o = m == 0 ? A.out[0] : m == 1 ? A.out[1] : m == 2 ? A.out[2] : A.out[3];
  const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int c = 0; c < 4; ++c) o[(int64_t)j * A.o_sm + (int64_t)(n + c) * A.o_sn] = (f16)vv[c];
}

// Codes (K,N), row stride ldk  ->  (N,K) rows (out[n*K + k]): the layout the matrix-core
// batch decode reads.  64 x 64 tiles through LDS (a padded row so the column reads of the
// transposed write hit distinct banks); reads run along n, writes along k.
constexpr int KN_TT = 64;

__global__ __launch_bounds__(256) void quad_codes_nk_kernel(const uint32_t* codes, int64_t ldk, int K, int N,
                                                            uint32_t* out) {
  __shared__ uint32_t tile[KN_TT][KN_TT + 1];
  const int n0 = blockIdx.x * KN_TT, k0 = blockIdx.y * KN_TT;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;   // 64 x 4 threads
#pragma unroll
  for (int i = 0; i < KN_TT; i += 4) {
    const int k = k0 + ty + i, n = n0 + tx;
    if (k < K && n < N) tile[ty + i][tx] = codes[(int64_t)k * ldk + n];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < KN_TT; i += 4) {
    const int n = n0 + ty + i, k = k0 + tx;
    if (k < K && n < N) out[(int64_t)n * K + k] = tile[tx][ty + i];
  }
}

// ------------------------------------------------------------------ host side
#ifndef PP_KN_MIN_ROWS
#define PP_KN_MIN_ROWS 32   // slices of at least this many rows (4096x4096: 1..4 tokens measured best)
#endif

struct KnPlan {
  int slices, ks;
  int64_t nblk;
};

// Columns per lane for a block of M tokens.
static int kn_cl(int64_t M) { return M <= 4 ? 4 : 2; }

static KnPlan kn_plan(int64_t M, int64_t N, int64_t K) {
  KnPlan p;
  const int64_t cols = 64 * kn_cl(M);
  p.nblk = (N + cols - 1) / cols;
  const int64_t waves = (int64_t)device_cu_count() * (KN_NT / 64);
  // about one item per wavefront, slices of at least PP_KN_MIN_ROWS rows
  int64_t s = std::max<int64_t>(
      1, std::min<int64_t>(waves / std::max<int64_t>(p.nblk, 1), (K + PP_KN_MIN_ROWS - 1) / PP_KN_MIN_ROWS));
  int64_t ks = (K + s - 1) / s;
  ks = (ks + KN_R - 1) / KN_R * KN_R;
  p.ks = (int)std::max<int64_t>(ks, KN_R);
  p.slices = (int)((K + p.ks - 1) / p.ks);
  return p;
}

bool quad_kn_ok(const void* a, int64_t a_sm, int64_t a_sk, const uint32_t* codes, int64_t c_sk, int64_t c_sn,
                int64_t M, int64_t N, int64_t K) {
  return c_sn == 1 && c_sk >= N && c_sk % 4 == 0 && N % 4 == 0 && N > 0 && K > 0 && K % 8 == 0 && M >= 1 && M <= 8 &&
         aligned(codes, 16) && a_sk == 1 && (M == 1 || a_sm % 8 == 0) && aligned(a, 16) &&
         K < (1ll << 30) && c_sk * K < (1ll << 30);
}

int64_t quad_kn_workspace(int64_t M, int64_t N, int64_t K, int64_t plug_n) {
  const KnPlan p = kn_plan(M, N, K);
  if (p.slices == 1 && plug_n == 0) return 0;
  return (int64_t)p.slices * 4 * M * N * (int64_t)sizeof(float);
}

int quad_kn_gemm(const void* a, int64_t a_sm, const uint32_t* codes, int64_t ldk, const void* const* luts,
                 int lut_dtype, const float* scales, const uint32_t* plug_idx, const void* plug_vals, int64_t plug_n,
                 int64_t elem_base, void* const* out, int64_t o_sm, int64_t o_sn, int64_t M, int64_t N, int64_t K,
                 void* workspace, int64_t workspace_bytes, hipStream_t st) {
  const KnPlan p = kn_plan(M, N, K);
  const int64_t need = quad_kn_workspace(M, N, K, plug_n);
  PP_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need), "workspace too small: need %lld bytes",
             (long long)need);
  QuadKnArgs A = {};
  A.codes = codes;
  A.ldk = ldk;
  A.a = reinterpret_cast<const f16*>(a);
  A.a_sm = a_sm;
  for (int m = 0; m < 4; ++m) {
    A.out[m] = reinterpret_cast<f16*>(out[m]);
    A.s[m] = scales[m];
  }
  A.o_sm = o_sm;
  A.o_sn = o_sn;
  A.M = (int)M;
  A.N = (int)N;
  A.K = (int)K;
  A.slices = p.slices;
  A.ks = p.ks;
  A.nblk = p.nblk;
  for (int i = 0; i < 7; ++i) A.luts.p[i] = luts[i];
  A.luts.dtype = lut_dtype;
  A.part = need > 0 ? reinterpret_cast<float*>(workspace) : nullptr;
  const int64_t items = p.nblk * p.slices;
  const unsigned grid = (unsigned)std::min<int64_t>(device_cu_count(), (items + KN_NT / 64 - 1) / (KN_NT / 64));
  switch (M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8) {
    case 1: hipLaunchKernelGGL((quad_kn_kernel<1, 4>), dim3(grid), dim3(KN_NT), 0, st, A); break;
    case 2: hipLaunchKernelGGL((quad_kn_kernel<2, 4>), dim3(grid), dim3(KN_NT), 0, st, A); break;
    case 4: hipLaunchKernelGGL((quad_kn_kernel<4, 4>), dim3(grid), dim3(KN_NT), 0, st, A); break;
    default: hipLaunchKernelGGL((quad_kn_kernel<8, 2>), dim3(grid), dim3(KN_NT), 0, st, A); break;
  }
  PP_LAUNCH_CHECK();
  if (A.part != nullptr) {
    if (plug_n > 0) {
      QuadKnPlugArgs P;
      P.T = A;
      P.plug_idx = plug_idx;
      P.plug_vals = reinterpret_cast<const f16*>(plug_vals);
      P.plug_n = plug_n;
      P.elem_base = elem_base;
      hipLaunchKernelGGL(quad_kn_plug_kernel, dim3((unsigned)((plug_n + 255) / 256)), dim3(256), 0, st, P);
      PP_LAUNCH_CHECK();
    }
    const int64_t total = 4 * M * N;
    hipLaunchKernelGGL(quad_kn_finish_kernel, dim3((unsigned)((total / 4 + 63) / 64)), dim3(KN_FIN_NT), 0, st, A);
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
}

}  // namespace pp

extern "C" int pp_quad_codes_nk(const uint32_t* codes, int64_t ldk, int64_t K, int64_t N, uint32_t* out,
                                void* stream) {
  PP_REQUIRE(K >= 0 && N >= 0 && ldk >= N, "bad shape / row stride");
  if (K == 0 || N == 0) return PP_OK;
  PP_REQUIRE(codes != nullptr && out != nullptr, "null pointer");
  PP_REQUIRE(K < (1ll << 31) && N < (1ll << 31) && (K + pp::KN_TT - 1) / pp::KN_TT < 65536,
             "K / N out of range");
  const dim3 grid((unsigned)((N + pp::KN_TT - 1) / pp::KN_TT), (unsigned)((K + pp::KN_TT - 1) / pp::KN_TT));
  hipLaunchKernelGGL(pp::quad_codes_nk_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), codes, ldk,
                     (int)K, (int)N, out);
  PP_LAUNCH_CHECK();
  return PP_OK;
}
