// Quad-pack decode GEMM for 1..64 tokens on the matrix cores (the batch path): one
// packed pass over codes laid out (N,K) row-major produces the 4 models' outputs
//   out_m[j, n] = fp16( s_m * sum_k x[j, k] * W_m[n, k] )
// (quad_kernels.py:123-134), with W_m decoded from the codes in registers
// (quad_kernels.py:103-121, quaternion_packer.py:173-185) and the plug table patched
// into the decoded values (quaternion_packer.py:187-193).
//
// Work item = 16 weight rows x one K slice, one wavefront, v_mfma_f32_16x16x32_f16:
//  * lane l owns row n0 + l%16 and, in each 32-column step, columns k0 + 8(l/16) .. +7:
//    two 16-byte loads of 8 code words, decoded with the LDS tables of quad_lds.h into
//    8 fp32 weights per model, rounded to fp16: the A operand of model m (A[i][k] in
//    lane i + 16 (k/8), the layout the instruction takes for 16 x 32 fp16);
//  * x is the B operand as stored: lane l reads tokens 16t + l%16 at the same 8 columns
//    (16 bytes of fp16), t = 0 .. T-1;
//  * 4 models x T token tiles of 16 x 16 fp32 sums stay in registers across the slice;
//    lane l holds rows n0 + 4(l/16) + r, r = 0..3, of token 16t + l%16;
//  * the loads of the next step are in flight while a step is decoded.
// Plug entries: each row's entries of the slice, 4 at a time, in every lane of the row
// (from the host's per (row, slice) start table); a lane whose 8 columns hold an entry
// replaces the decoded tuple by the plug values before rounding.
// Slices: with one slice a wave writes its fp16 outputs; otherwise it adds its scaled
// sums into float32 accumulators [m][n][j] with device-scope atomics (no return, so
// nothing waits on them) and quad_mfma_finish_kernel, launched after, swaps the totals
// out (leaving zeros for the next launch) and writes the outputs.
#include "quad_lds.h"
#include "rows_common.h"

namespace pp {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int MF_NT = 512;   // threads per workgroup: 8 waves, one workgroup per CU (the tables take all of LDS)

struct QuadMfmaArgs {
  const uint32_t* codes;   // code of (row 0, col 0); row n at codes + n*ldc
  int64_t ldc;
  int64_t pos0;            // stream position of (row 0, col 0), for the plug positions
  const f16* x;            // (M, K), row stride x_sm
  int64_t x_sm;
  f16* out[4];             // (M, N), row stride o_sm
  int64_t o_sm;
  int N, K, M;
  int slices, ks;          // K slices of ks columns (a multiple of 32)
  int64_t tiles;           // ceil(N / 16)
  const int64_t* row_plug; // [n*slices + s]: first plug entry of (row n, slice s); n*slices+s+1 ends it
  QuadLuts luts;
  float s[4];
  const uint32_t* plug_idx;
  const f16* plug_vals;    // (P, 4), normalised
  int64_t plug_n;
  float* acc;              // slices > 1: [4][N][M] float32, zero on entry
};

template <int T>
struct MStage {
  u32x4 c0, c1;            // 8 code words of the lane's row
  u32x4 xb[T];             // 8 fp16 x of token 16t + l%16
};

template <int T>
__device__ __forceinline__ void mstage_issue(const QuadMfmaArgs& A, rsrc_t rc, rsrc_t rx, int ri, int q, bool rowok,
                                             int k0, int ke, MStage<T>& S) {
  const int kk = k0 + 8 * q;
  const bool valid = kk < ke;
  const uint32_t co = (rowok && valid) ? 4u * (uint32_t)(ri * A.ldc + kk) : OOB;
  vload128(S.c0, co, rc);
  vload128(S.c1, co == OOB ? OOB : co + 16u, rc);
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int j = 16 * t + ri;
    vload128(S.xb[t], (valid && j < A.M) ? 2u * (uint32_t)(j * A.x_sm + kk) : OOB, rx);
  }
}

// The lane's window of 4 plug entries of its row: columns (INT_MAX past the end) and values.
struct MPlug {
  int k[4];
  u32x2 v[4];
  int64_t next, end;       // next entry to load, end of the row's entries in the slice
};

__device__ __forceinline__ void mplug_fill(const QuadMfmaArgs& A, int64_t rowpos, MPlug& P) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t e = P.next + i;
    const bool has = e < P.end;
    P.k[i] = has ? (int)((int64_t)A.plug_idx[e] - rowpos) : 0x7FFFFFFF;
    P.v[i] = has ? *reinterpret_cast<const u32x2*>(A.plug_vals + 4 * e) : u32x2{0u, 0u};
  }
  P.next += 4;
}

template <class L>
__device__ __forceinline__ void decode8(const char* lds, const LaneOff& lo, const u32x4& c0, const u32x4& c1,
                                        float (&w)[4][8]) {
  const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float r;
    float2 a, b, c;
    lookup<L>(lds, cw[e], lo, r, a, b, c);
    const float rs = r * a.y, rss = rs * b.y;
    w[0][e] = r * a.x;
    w[1][e] = rs * b.x;
    w[2][e] = rss * c.x;
    w[3][e] = rss * c.y;
  }
}

template <int T, class L>
__device__ __forceinline__ void mfma_body(const char* lds, const QuadMfmaArgs& A) {
  const int lane = threadIdx.x & 63, ri = lane & 15, q = lane >> 4;
  const LaneOff lo = L::lane(lane);
  constexpr int WAVES = MF_NT / 64;
  const int64_t gw = (int64_t)blockIdx.x * WAVES + uniform(threadIdx.x >> 6);
  const int64_t nw = (int64_t)gridDim.x * WAVES;
  const int64_t items = A.tiles * A.slices;
  const rsrc_t rx = make_rsrc(A.x, 2u * (uint32_t)((int64_t)(A.M - 1) * A.x_sm + A.K));
  for (int64_t it = gw; it < items; it += nw) {
    const int tile = (int)uniform64(it / A.slices), sl = (int)uniform64(it % A.slices);
    const int n0 = tile * 16;
    const int kb = sl * A.ks, ke = min(A.K, kb + A.ks);
    const int nrows = min(16, A.N - n0);
    const int n = n0 + ri;
    const bool rowok = ri < nrows;
    const rsrc_t rc = make_rsrc(A.codes + (int64_t)n0 * A.ldc, 4u * (uint32_t)((int64_t)(nrows - 1) * A.ldc + A.K));
    MStage<T> s0, s1;
    mstage_issue<T>(A, rc, rx, ri, q, rowok, kb, ke, s0);
    // the row's plug entries in this slice
    MPlug P;
    P.next = rowok && A.plug_n > 0 ? A.row_plug[(int64_t)n * A.slices + sl] : 0;
    P.end = rowok && A.plug_n > 0 ? A.row_plug[(int64_t)n * A.slices + sl + 1] : 0;
    const int64_t rowpos = A.pos0 + (int64_t)n * A.ldc;
    mplug_fill(A, rowpos, P);
    f4 C[4][T];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int t = 0; t < T; ++t) C[m][t] = f4{0.f, 0.f, 0.f, 0.f};
    auto step = [&](const MStage<T>& cur, MStage<T>& nxt, int k0) {
      mstage_issue<T>(A, rc, rx, ri, q, rowok, k0 + 32, ke, nxt);
      float w[4][8];
      decode8<L>(lds, lo, cur.c0, cur.c1, w);
      const int kk = k0 + 8 * q;
      for (;;) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = P.k[i] - kk;
          const bool hit = e >= 0 && e < 8;
          if (__ballot(hit)) {
            const f16x4 pv = __builtin_bit_cast(f16x4, P.v[i]);
            const float v[4] = {(float)pv.x, (float)pv.y, (float)pv.z, (float)pv.w};
#pragma unroll
            for (int ee = 0; ee < 8; ++ee) {
              const bool sel = hit && e == ee;
#pragma unroll
              for (int m = 0; m < 4; ++m) w[m][ee] = sel ? v[m] : w[m][ee];
            }
          }
        }
        // the window is used up within this step: take the row's next 4 (rare) and patch
        // again (lanes that keep their window re-apply the same values: no change)
        const bool refill = P.k[3] < k0 + 32 && P.next < P.end;
        if (!__ballot(refill)) break;
        if (refill) mplug_fill(A, rowpos, P);
      }
      h8 a[4];
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int ee = 0; ee < 8; ++ee) a[m][ee] = (_Float16)w[m][ee];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const h8 b = __builtin_bit_cast(h8, cur.xb[t]);
#pragma unroll
        for (int m = 0; m < 4; ++m) C[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m], b, C[m][t], 0, 0, 0);
      }
    };
    int k0 = kb;
    for (;;) {
      if (k0 >= ke) break;
      step(s0, s1, k0);
      k0 += 32;
      if (k0 >= ke) break;
      step(s1, s0, k0);
      k0 += 32;
    }
    // epilogue: lane holds rows n0 + 4q + r of token 16t + ri
    if (A.slices == 1) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const rsrc_t ro = make_rsrc(A.out[m], 2u * (uint32_t)((int64_t)(A.M - 1) * A.o_sm + A.N));
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const int j = 16 * t + ri;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = n0 + 4 * q + r;
            const f16 h = (f16)(C[m][t][r] * A.s[m]);
            vstore16((uint32_t)__builtin_bit_cast(unsigned short, h),
                     (row < A.N && j < A.M) ? 2u * (uint32_t)((int64_t)j * A.o_sm + row) : OOB, ro);
          }
        }
      }
    } else {
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const int j = 16 * t + ri;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = n0 + 4 * q + r;
            if (row < A.N && j < A.M)
              __hip_atomic_fetch_add(A.acc + ((int64_t)m * A.N + row) * A.M + j, C[m][t][r] * A.s[m],
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
    }
  }
}

template <int T>
__global__ __launch_bounds__(MF_NT) void quad_mfma_kernel(const QuadMfmaArgs A) {
  __shared__ __attribute__((aligned(16))) uint32_t Tb[QLDS_BYTES / 4];
  const char* lds = reinterpret_cast<const char*>(Tb);
  if (quad_tables(Tb, A.luts)) mfma_body<T, LayShared>(lds, A);
  else mfma_body<T, LaySplit>(lds, A);
}

// Sliced launches: out_m[j, n] = fp16(acc[m][n][j]), acc left zero.
__global__ __launch_bounds__(256) void quad_mfma_finish_kernel(const QuadMfmaArgs A) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = 4ll * A.N * A.M;
  if (i >= total) return;
  const int j = (int)(i % A.M);
  const int64_t mn = i / A.M;
  const int row = (int)(mn % A.N), m = (int)(mn / A.N);
  const float v = __hip_atomic_exchange(A.acc + i, 0.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  f16* o = m == 0 ? A.out[0] : m == 1 ? A.out[1] : m == 2 ? A.out[2] : A.out[3];
  o[(int64_t)j * A.o_sm + row] = (f16)v;
}

static int mfma_tiles_t(int64_t M) { return M <= 16 ? 1 : M <= 32 ? 2 : 4; }

}  // namespace pp

using namespace pp;

extern "C" int64_t pp_quad_mfma_waves(void) { return (int64_t)device_cu_count() * (MF_NT / 64); }

extern "C" int64_t pp_quad_mfma_workspace_size(int64_t M, int64_t N, int64_t slices) {
  if (slices <= 1) return 0;
  return (4 * N * M * 4 + 255) / 256 * 256;
}

extern "C" int pp_quad_mfma(const uint32_t* codes, int64_t ldc, int64_t elem_base, const void* a, int64_t a_sm,
                            const void* const* luts, int lut_dtype, const float* scales, const uint32_t* plug_idx,
                            const void* plug_vals, int64_t plug_n, const int64_t* row_plug, int64_t slices,
                            int64_t slice_cols, void* const* out, int64_t o_sm, int64_t M, int64_t N, int64_t K,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  PP_REQUIRE(codes != nullptr && a != nullptr && out != nullptr && luts != nullptr && scales != nullptr,
             "null pointer argument");
  for (int m = 0; m < 4; ++m) PP_REQUIRE(out[m] != nullptr, "out[%d] is null", m);
  for (int i = 0; i < 7; ++i) PP_REQUIRE(luts[i] != nullptr, "lut %d is null", i);
  PP_REQUIRE(lut_dtype == PP_F16 || lut_dtype == PP_F32, "bad lut_dtype");
  PP_REQUIRE(M >= 1 && M <= 64, "the matrix-core path takes 1..64 tokens, got %lld", (long long)M);
  PP_REQUIRE(N >= 1 && K >= 8 && K % 8 == 0, "needs N >= 1 and K a multiple of 8 (N=%lld, K=%lld)", (long long)N,
             (long long)K);
  PP_REQUIRE(ldc >= K && ldc % 4 == 0 && aligned(codes, 16), "codes must be 16-byte aligned rows of ldc >= K words");
  PP_REQUIRE(aligned(a, 16) && (M == 1 || (a_sm >= K && a_sm % 8 == 0)),
             "activations must be 16-byte aligned with a row stride that is a multiple of 8");
  PP_REQUIRE(o_sm >= N, "o_sm must be >= N");
  PP_REQUIRE(slices >= 1 && slice_cols >= 32 && slice_cols % 32 == 0 && slices * slice_cols >= K &&
                 (slices - 1) * slice_cols < K,
             "slices x slice_cols must cover K in multiples of 32 columns");
  PP_REQUIRE(plug_n >= 0 && (plug_n == 0 || (plug_idx && plug_vals && row_plug)), "plug arrays are null");
  PP_REQUIRE(16 * ldc * 4 < (1ll << 31) && (M - 1) * a_sm + K < (1ll << 30) && (M - 1) * o_sm + N < (1ll << 30),
             "a tile of codes, the activations and the outputs must each stay below 2 GiB");
  const int64_t need = pp_quad_mfma_workspace_size(M, N, slices);
  PP_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need),
             "workspace too small: need %lld bytes", (long long)need);
  QuadMfmaArgs A = {};
  A.codes = codes;
  A.ldc = ldc;
  A.pos0 = elem_base;
  A.x = reinterpret_cast<const f16*>(a);
  A.x_sm = M > 1 ? a_sm : K;
  for (int m = 0; m < 4; ++m) A.out[m] = reinterpret_cast<f16*>(out[m]);
  A.o_sm = o_sm;
  A.N = (int)N;
  A.K = (int)K;
  A.M = (int)M;
  A.slices = (int)slices;
  A.ks = (int)slice_cols;
  A.tiles = (N + 15) / 16;
  A.row_plug = row_plug;
  for (int i = 0; i < 7; ++i) A.luts.p[i] = luts[i];
  A.luts.dtype = lut_dtype;
  for (int m = 0; m < 4; ++m) A.s[m] = scales[m];
  A.plug_idx = plug_idx;
  A.plug_vals = reinterpret_cast<const f16*>(plug_vals);
  A.plug_n = plug_n;
  A.acc = reinterpret_cast<float*>(workspace);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t items = A.tiles * slices;
  const int64_t waves = MF_NT / 64;
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(device_cu_count(), (items + waves - 1) / waves));
  switch (mfma_tiles_t(M)) {
    case 1: hipLaunchKernelGGL(quad_mfma_kernel<1>, dim3(grid), dim3(MF_NT), 0, st, A); break;
    case 2: hipLaunchKernelGGL(quad_mfma_kernel<2>, dim3(grid), dim3(MF_NT), 0, st, A); break;
    default: hipLaunchKernelGGL(quad_mfma_kernel<4>, dim3(grid), dim3(MF_NT), 0, st, A); break;
  }
  PP_LAUNCH_CHECK();
  if (slices > 1) {
    const int64_t total = 4 * N * M;
    hipLaunchKernelGGL(quad_mfma_finish_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, A);
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
}
