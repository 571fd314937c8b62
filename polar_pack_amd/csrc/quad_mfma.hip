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
// nothing waits on them) and quad_mfma_finish_kernel, launched after, reads the totals,
// writes the outputs and leaves zeros for the next launch.
#include "quad_mfma.h"

namespace pp {

// Threads per workgroup: 8 waves (one workgroup per CU: the tables take all of LDS).
// SUB: 32-column MFMA steps per stage.  A stage is what one load step brings in: SUB x 2
// KiB of codes per wave; 1 step (2 KiB) per stage left the waves waiting a full HBM round
// trip per step, 4 steps (8 KiB, as much as the row kernel keeps in flight) hide it.
// With 2 or 4 token tiles the x operands take the registers: 2 steps (measured faster
// than 4 with 2 tiles: 49.5 vs 53.3 us on an 11008x2048 Linear at 32 tokens).
// (Running the LDS lookups a group of tuples ahead of their arithmetic, as the row
// kernel does, measured no faster here.)
template <int T> struct MfCfg {
  static constexpr int NT = 512;
  static constexpr int SUB = T == 1 ? 4 : 2;
};

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
  static constexpr int SUB = MfCfg<T>::SUB;
  u32x4 c[SUB][2];         // per step: 8 code words of the lane's row
  u32x4 xb[SUB][T];        // per step: 8 fp16 x of token 16t + l%16
};

// Issue the loads of the step at column k0.  Each lane's offsets are fixed for the item
// (voc for its row's codes, vox[t] for token 16t + l%16; OOB for rows or tokens past the
// end); the buffer resources are rebased to k0 in scalar registers, so a step needs no
// vector address arithmetic.  K and the slices are multiples of 32 columns, so every
// lane's 8 columns of a step are in range (a step past the slice end reads data it never
// uses).
template <int T>
__device__ __forceinline__ void mstage_issue(const QuadMfmaArgs& A, const uint32_t* ctile, int nrows, uint32_t voc,
                                             const uint32_t (&vox)[T], int k0, MStage<T>& S) {
  constexpr int SUB = MfCfg<T>::SUB;
  k0 = min(k0, A.K);   // look-ahead past the end: rebase at K (nothing read there is used)
  const rsrc_t rc = make_rsrc(ctile + k0, 4u * (uint32_t)((int64_t)(nrows - 1) * A.ldc + (A.K - k0)));
#pragma unroll
  for (int u = 0; u < SUB; ++u) {
    vload128(S.c[u][0], voc + 128u * u, rc);
    vload128(S.c[u][1], voc + 128u * u + 16u, rc);
  }
  const rsrc_t rx = make_rsrc(A.x + k0, 2u * (uint32_t)((int64_t)(A.M - 1) * A.x_sm + (A.K - k0)));
#pragma unroll
  for (int u = 0; u < SUB; ++u)
#pragma unroll
    for (int t = 0; t < T; ++t) vload128c(S.xb[u][t], vox[t] + 64u * u, rx);
}

// The slice walk of one item: step(cur, pre, k0) issues the loads of step k0 + 32 into
// pre, decodes cur (step k0) into the MFMA operands, patches the plug entries and
// accumulates; returns false after the last step.  Called alternately on two stage
// buffers (the shape of the row kernel's walk), so every load is consumed one step after
// it was issued.  (A ring of 4 stages measured no faster: the compiler's waits still
// drained it to one step ahead.)
template <int T, class L>
struct MRun {
  const char* lds;
  LaneOff lo;
  const QuadMfmaArgs& A;
  const uint32_t* ctile;
  int nrows;
  uint32_t voc;
  uint32_t vox[T];
  int q;
  int ke;
  int64_t rowpos;
  MPlug P;
  f4 C[4][T];

  __device__ __forceinline__ bool step(const MStage<T>& cur, MStage<T>& pre, int& k0) {
    constexpr int SUB = MfCfg<T>::SUB;
    mstage_issue<T>(A, ctile, nrows, voc, vox, k0 + 32 * SUB, pre);
#pragma unroll
    for (int u = 0; u < SUB; ++u) {
      const int ks = k0 + 32 * u;
      if (ks >= ke) break;   // the slice ends inside the stage (wave-uniform)
      h8 a[4];
      decode8<L>(lds, lo, cur.c[u][0], cur.c[u][1], a);
      const int kk = ks + 8 * q;
      mplug_patch(PlugSrc{A.plug_idx, A.plug_vals, A.plug_n}, P, rowpos, kk, ks, a);
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const h8 b = __builtin_bit_cast(h8, cur.xb[u][t]);
#pragma unroll
        for (int m = 0; m < 4; ++m) C[m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[m], b, C[m][t], 0, 0, 0);
      }
    }
    k0 += 32 * MfCfg<T>::SUB;
    return k0 < ke;
  }
};

template <int T, class L>
__device__ __forceinline__ void mfma_body(const char* lds, const QuadMfmaArgs& A) {
  const int lane = threadIdx.x & 63, ri = lane & 15, q = lane >> 4;
  const LaneOff lo = L::lane(lane);
  constexpr int WAVES = MfCfg<T>::NT / 64;
  // items are dealt round-robin over the workgroups (item i to workgroup i % grid), so a
  // launch with fewer items than wavefronts still spreads them over every CU
  const int64_t gw = (int64_t)uniform(threadIdx.x >> 6) * gridDim.x + blockIdx.x;
  const int64_t nw = (int64_t)gridDim.x * WAVES;
  const int64_t items = A.tiles * A.slices;
  uint32_t vox[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const int j = 16 * t + ri;
    vox[t] = j < A.M ? 2u * (uint32_t)(j * A.x_sm + 8 * q) : OOB;
  }
  for (int64_t it = gw; it < items; it += nw) {
    const int tile = (int)uniform64(it / A.slices), sl = (int)uniform64(it % A.slices);
    const int n0 = tile * 16;
    const int kb = sl * A.ks, ke = min(A.K, kb + A.ks);
    const int nrows = min(16, A.N - n0);
    const int n = n0 + ri;
    const bool rowok = ri < nrows;
    const uint32_t* ctile = A.codes + (int64_t)n0 * A.ldc;
    const uint32_t voc = rowok ? 4u * (uint32_t)(ri * A.ldc + 8 * q) : OOB;
    // the row's plug entries in this slice: the first window, then the first step's loads
    MPlug P;
    P.next = rowok && A.plug_n > 0 ? A.row_plug[(int64_t)n * A.slices + sl] : 0;
    P.end = rowok && A.plug_n > 0 ? A.row_plug[(int64_t)n * A.slices + sl + 1] : 0;
    const int64_t rowpos = A.pos0 + (int64_t)n * A.ldc;
    uint32_t pidx[MPW];
    mplug_issue(PlugSrc{A.plug_idx, A.plug_vals, A.plug_n}, P, pidx);
    MStage<T> s0, s1;
    mstage_issue<T>(A, ctile, nrows, voc, vox, kb, s0);
    mplug_take(P, pidx, rowpos);
    MRun<T, L> R{lds, lo, A, ctile, nrows, voc, {}, q, ke, rowpos, P};
#pragma unroll
    for (int t = 0; t < T; ++t) R.vox[t] = vox[t];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int t = 0; t < T; ++t) R.C[m][t] = f4{0.f, 0.f, 0.f, 0.f};
    int k0 = kb;
    for (;;) {
      if (!R.step(s0, s1, k0)) break;
      if (!R.step(s1, s0, k0)) break;
    }
    const f4 (&C)[4][T] = R.C;
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
__global__ __launch_bounds__(MfCfg<T>::NT) void quad_mfma_kernel(const QuadMfmaArgs A) {
  __shared__ __attribute__((aligned(16))) uint32_t Tb[QLDS_BYTES / 4];
  const char* lds = reinterpret_cast<const char*>(Tb);
  if (quad_tables<MfCfg<T>::NT>(Tb, A.luts)) mfma_body<T, LayShared>(lds, A);
  else mfma_body<T, LaySplit>(lds, A);
}

// Sliced launches: out_m[j, n] = fp16(acc[m][n][j]), acc left zero (finish_tile).
__global__ __launch_bounds__(256) void quad_mfma_finish_kernel(const QuadMfmaArgs A, bool vec) {
  int m, n0, j0;
  finish_coords(A.N, A.M, m, n0, j0);
  f16* o = m == 0 ? A.out[0] : m == 1 ? A.out[1] : m == 2 ? A.out[2] : A.out[3];
  finish_tile(A.acc + (int64_t)m * A.N * A.M, o, A.o_sm, A.N, A.M, n0, j0, vec);
}

static int mfma_tiles_t(int64_t M) { return M <= 16 ? 1 : M <= 32 ? 2 : 4; }

static int mfma_nt(int64_t M) {
  switch (mfma_tiles_t(M)) {
    case 1: return MfCfg<1>::NT;
    case 2: return MfCfg<2>::NT;
    default: return MfCfg<4>::NT;
  }
}

}  // namespace pp

using namespace pp;

extern "C" int64_t pp_quad_mfma_waves(int64_t M) {
  if (M < 1 || M > 64) return 0;
  return (int64_t)device_cu_count() * (mfma_nt(M) / 64);
}

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
  PP_REQUIRE(N >= 1 && K >= 32 && K % 32 == 0, "needs N >= 1 and K a multiple of 32 (N=%lld, K=%lld)", (long long)N,
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
  PP_REQUIRE(need == 0 || aligned(workspace, 16), "the workspace must be 16-byte aligned");
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
  const int nt = mfma_nt(M);
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(device_cu_count(), items));
  switch (mfma_tiles_t(M)) {
    case 1: hipLaunchKernelGGL(quad_mfma_kernel<1>, dim3(grid), dim3(nt), 0, st, A); break;
    case 2: hipLaunchKernelGGL(quad_mfma_kernel<2>, dim3(grid), dim3(nt), 0, st, A); break;
    default: hipLaunchKernelGGL(quad_mfma_kernel<4>, dim3(grid), dim3(nt), 0, st, A); break;
  }
  PP_LAUNCH_CHECK();
  if (slices > 1) {
    hipLaunchKernelGGL(quad_mfma_finish_kernel, dim3((unsigned)finish_tiles(4, N, M)), dim3(256), 0, st, A,
                       finish_vec(out, 4, o_sm));
    PP_LAUNCH_CHECK();
  }
  return PP_OK;
}
