/*
 * polar_pack_amd -- C ABI of the MI355X (gfx950) fused dequant-matmul decode path.
 *
 * Every entry point:
 *   - takes device pointers (hipMalloc'd memory, or torch CUDA tensors' data_ptr())
 *     plus plain sizes/strides in ELEMENTS, and a hipStream_t passed as void*;
 *   - enqueues work on that stream and returns without synchronising;
 *   - returns PP_OK (0) or a nonzero pp_status; pp_last_error() then returns a
 *     thread-local message.
 *
 * Nothing here allocates device memory: entry points that need scratch memory take a
 * caller-provided workspace (see *_workspace_size), or, for pp_quad_gemm_noalloc, use a
 * fixed device array inside the library.
 *
 * Citations name the reference interface each entry point replaces
 * (file:line in everymonday100/polar_pack).
 */
#ifndef POLAR_PACK_H
#define POLAR_PACK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum pp_status {
  PP_OK = 0,
  PP_EINVAL = 1,       /* bad argument (shape, stride, pointer, enum) */
  PP_EHIP = 2,         /* a HIP runtime call failed */
  PP_ENOSUPPORT = 3    /* valid request this build does not implement */
};

enum pp_dtype { PP_F16 = 0, PP_F32 = 1 };

/* Dual code layouts:
 *   PP_DUAL_I16_OFFSET -- native int16 = ((amp << 10) | phase) - 32768, the
 *                         kernel layout of polar_kernels.py:9-11;
 *   PP_DUAL_U16_BE     -- the .dualpack file layout, big-endian uint16
 *                         (amp << 10) | phase, polar_bitpack.py:81-88. */
enum pp_dual_layout { PP_DUAL_I16_OFFSET = 0, PP_DUAL_U16_BE = 1 };

/* Thread-local message describing the last nonzero status. */
const char* pp_last_error(void);

/* Library version string, and the gfx target it was compiled for. */
const char* pp_version(void);

/* sizeof of the ABI structs, for binding checks: out[0] = sizeof(pp_quad_proj),
 * out[1] = sizeof(pp_quad_item), out[2] = sizeof(pp_quad_seg), out[3] = sizeof(pp_dual_proj).
 * Returns the number of values written. */
int pp_abi_sizes(int64_t* out, int n);

/* ------------------------------------------------------------------------ */
/* Quad pack: uint32 word [norm 8 | t1 8 | t2 8 | t3 8] -> 4 models.          */
/* ------------------------------------------------------------------------ */

/*
 * Fused decode GEMM over a (K,N) code view:
 *   out_m[i, n] = fp16( s_m * sum_k a[i, k] * W_m[k, n] ),   m = 0..3,
 * where W_m is decoded from codes[k*c_sk + n*c_sn] with the 7 LUTs
 * luts = {norm, cos1, sin1, cos2, sin2, cos3, sin3} (256 entries each,
 * lut_dtype PP_F16 or PP_F32, device memory; `luts` itself is a host array of
 * the 7 device pointers) and the host float[4] `scales`:
 *   w0 = r*c1, w1 = r*s1*c2, w2 = r*s1*s2*c3, w3 = r*s1*s2*s3.
 *
 * Replaces quad_bitpacked (quad_kernels.py:146-159) and
 * quad_bitpacked_kernel (quad_kernels.py:53-143).
 *
 * Plug table (optional, plug_n may be 0): entries with
 *   plug_idx[j] - elem_base == k*c_sk + n*c_sn
 * replace the decoded normalised tuple of element (k, n) by the fp16 values
 * plug_vals[4*j .. 4*j+3] (the semantics of quaternion_packer.py:187-193).
 * plug_idx must be ascending.  Plug entries need one unit stride
 * (c_sk == 1 or c_sn == 1).
 *
 * Fast paths: c_sk == 1 (container layout, codes rows are (N,K) row-major)
 * with K % 4 == 0, 16-byte aligned rows and M <= 8; c_sn == 1 (the contiguous
 * (K,N) tensor pack_quad_layer returns) with N % 4 == 0, K % 8 == 0, 16-byte
 * aligned rows, in blocks of 8 tokens over a K-slice workspace.  Other layouts
 * decode into `workspace` (4*K*N floats) and multiply.  The caller sizes the
 * workspace with pp_quad_gemm_workspace_size.
 */
int pp_quad_gemm(const void* a, int64_t a_sm, int64_t a_sk,
                 const uint32_t* codes, int64_t c_sk, int64_t c_sn,
                 const void* const* luts, int lut_dtype,
                 const float* scales,
                 const uint32_t* plug_idx, const void* plug_vals, int64_t plug_n, int64_t elem_base,
                 void* const* out, int64_t o_sm, int64_t o_sn,
                 int64_t M, int64_t N, int64_t K,
                 void* workspace, int64_t workspace_bytes,
                 void* stream);

/* Bytes of workspace pp_quad_gemm needs for this call (0 on the fast paths). */
int64_t pp_quad_gemm_workspace_size(const void* a, int64_t a_sm, int64_t a_sk,
                                    const uint32_t* codes, int64_t c_sk, int64_t c_sn,
                                    int64_t plug_n, int64_t M, int64_t N, int64_t K);

/* One (N,K) Linear of container rows (row n of the codes at codes + n*ldc, as a stream
 * stores a projection) on the fused row kernel, 1-8 tokens, with a plan made once per codes
 * and plug table (no reference counterpart: the reference's quad_bitpacked, quad_kernels.py:
 * 146-159, makes one call per Linear with no state; this is that call with its per-table work
 * done ahead, which the drop-in operator caches).  The plan:
 *   wave_plug  pp_quad_rows_plan_size(M) int64 plug starts from pp_quad_rows_plan (null
 *              without plug entries), for this elem_base, ldc, M, N and K;
 *   plug_code  each entry's code word from pp_quad_plug_codes (or null: read from the codes);
 *   workspace  pp_quad_rows_workspace_size(M, N, K) bytes, zero on entry and left zero by
 *              every launch (null when that is 0): rows with fewer tasks than ~1.5 per
 *              wavefront are cut into pp_quad_rows_parts(M, N, K) column slices; when that is
 *              a power of two dividing a workgroup's waves, a task's slices are waves of one
 *              workgroup and meet in LDS (no workspace), otherwise they meet there.
 * Outputs out[m][i*o_sm + n*o_sn] = fp16(s_m * sum_k a[i*a_sm + k] W_m[n][k]); launches that
 * share a workspace must not overlap. */
int64_t pp_quad_rows_plan_size(int64_t M);
int64_t pp_quad_rows_workspace_size(int64_t M, int64_t N, int64_t K);
int pp_quad_rows_parts(int64_t M, int64_t N, int64_t K);
int pp_quad_rows_plan(const uint32_t* plug_idx, int64_t plug_n, int64_t elem_base, int64_t ldc, int64_t M,
                      int64_t N, int64_t K, int64_t* wave_plug, void* stream);
int pp_quad_rows(const void* a, int64_t a_sm, const uint32_t* codes, int64_t ldc,
                 const void* const* luts, int lut_dtype, const float* scales,
                 const uint32_t* plug_idx, const void* plug_vals, const uint32_t* plug_code, int64_t plug_n,
                 const int64_t* wave_plug, int64_t elem_base, void* const* out, int64_t o_sm, int64_t o_sn,
                 int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* stream);

/* The kernel pp_quad_gemm / pp_dual_gemm runs for these operands (no reference counterpart:
 * the reference has one kernel per operator): PP_GEMM_ROWS (the fused row decode of (N,K)
 * rows), PP_GEMM_KN (the fused decode of (K,N) rows with unit column stride), PP_GEMM_GENERIC
 * (decode into the workspace, then a plain GEMV), 0 for an empty problem.  No device work;
 * the Python operators' routing table is checked against it. */
enum pp_gemm_kernel { PP_GEMM_ROWS = 1, PP_GEMM_KN = 2, PP_GEMM_GENERIC = 3 };
int pp_quad_gemm_kernel(const void* a, int64_t a_sm, int64_t a_sk, const uint32_t* codes, int64_t c_sk,
                        int64_t c_sn, int64_t M, int64_t N, int64_t K);

/*
 * pp_quad_gemm without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference: it exists for those callers.
 * Same operands, results and fast paths as pp_quad_gemm; the workspace is a device array
 * of PP_NOALLOC_SCRATCH_BYTES inside the library (one per GPU, held until the process
 * ends).  Calls whose pp_quad_gemm_workspace_size exceeds it fail with PP_EINVAL (the
 * generic layouts above 4M weights; the fast paths need at most 32 MiB below 500K output
 * columns).  It calls no hipMalloc,
 * hipFree or allocating library routine.  Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU race.
 */
#define PP_NOALLOC_SCRATCH_BYTES (64ll << 20)
int pp_quad_gemm_noalloc(const void* a, int64_t a_sm, int64_t a_sk,
                         const uint32_t* codes, int64_t c_sk, int64_t c_sn,
                         const void* const* luts, int lut_dtype,
                         const float* scales,
                         const uint32_t* plug_idx, const void* plug_vals, int64_t plug_n, int64_t elem_base,
                         void* const* out, int64_t o_sm, int64_t o_sn,
                         int64_t M, int64_t N, int64_t K,
                         void* stream);

/*
 * Dequantise to float32: out_m[k*N + n] = s_m * W_m[k, n] (plug applied).
 * Parity / debug export; same operands as pp_quad_gemm.
 * Replaces the decode half of unpack_quad (quaternion_packer.py:169-196)
 * for one (K,N) view.
 */
int pp_quad_dequant(const uint32_t* codes, int64_t c_sk, int64_t c_sn,
                    const void* const* luts, int lut_dtype, const float* scales,
                    const uint32_t* plug_idx, const void* plug_vals, int64_t plug_n, int64_t elem_base,
                    float* const* out, int64_t N, int64_t K, void* stream);

/*
 * The same into fp16: out_m[k*N + n] = fp16(s_m * W_m[k, n]), the rounded weights the
 * reference kernel feeds its dot products (quad_kernels.py:117-126, with s_m folded in).
 * For batches large enough that the matmul is compute-bound (the reference's prefill
 * sizes, quad_kernels.py:175-189): decode once, then a library fp16 GEMM.
 */
int pp_quad_dequant_f16(const uint32_t* codes, int64_t c_sk, int64_t c_sn,
                        const void* const* luts, int lut_dtype, const float* scales,
                        const uint32_t* plug_idx, const void* plug_vals, int64_t plug_n, int64_t elem_base,
                        void* const* out, int64_t N, int64_t K, void* stream);

/*
 * The same, transposed: codes (K,N) with unit column stride and row stride c_sk (>= N, a
 * multiple of 4, 16-byte aligned rows; the layout pack_quad_layer returns) into
 * out_m[n*K + k] = fp16(s_m * W_m[k, n]), i.e. W_m^T row-major, the operand a library GEMM
 * takes fastest for x @ W_m.  N % 8 == 0, K % 8 == 0, 16-byte aligned outputs.  Plug
 * positions as for pp_quad_dequant_f16.  No counterpart in the reference: the fp16 weights
 * of its tl.dot, laid out for the prefill GEMM that replaces it (quad_kernels.py:166-189).
 */
int pp_quad_dequant_f16_t(const uint32_t* codes, int64_t c_sk, const void* const* luts, int lut_dtype,
                          const float* scales, const uint32_t* plug_idx, const void* plug_vals, int64_t plug_n,
                          int64_t elem_base, void* const* out, int64_t N, int64_t K, void* stream);

/*
 * Whole-stream decode for 1..8 tokens: one launch over many projections of one
 * .quadpack stream (the grouped whole-step launch).  All tables are device memory
 * prepared by the host once per stream (see polar_pack_amd/stream.py):
 *
 *   projs      : n_projs descriptors of pp_quad_proj;
 *   segs       : n_segs runs of rows of one projection (pp_quad_seg);
 *                wavefront w decodes segs [seg_bounds[w], seg_bounds[w+1]),
 *                n_waves = pp_quad_stream_waves(M) (the host balances them by bytes);
 *   workspace  : needed only when a segment has parts > 1: the uint32 counters (one per
 *                task number) at its start and the float32 accumulators the segments
 *                name; all zero before the first launch, and left zero by every launch
 *                (launches that share a workspace must not overlap);
 *   luts       : 7 float32 LUTs from the header (r_max, mu);
 *   scales     : host float[4], the header RMS s_k;
 *   plug_idx / plug_vals : the stream's plug table (ascending positions, plug_n entries).
 *
 * Rows touching stream positions >= n_codes (FP16 tails) are listed apart, in
 * tail_items (one row each, flags PP_ITEM_TAIL, with their plug range), and decoded
 * from tails[m] (fp16, length tail_len[m], model m's positions
 * n_codes .. n_codes+tail_len[m]-1) by a second, small kernel.
 * Replaces the per-projection quad_bitpacked calls of a decode step and the
 * tail restore of unpack_quad (quaternion_packer.py:201-210).
 */
typedef struct pp_quad_proj {
  const uint32_t* codes;   /* code of (row 0, col 0); row r starts at codes + r*ldc */
  int64_t ldc;             /* row stride of codes in elements (K for a packed stream) */
  int64_t pos0;            /* stream position of (row 0, col 0) */
  const void* x;           /* fp16 activations (M, K), row stride x_sm */
  int64_t x_sm;
  void* out[4];            /* fp16 outputs (M, N), row stride o_sm, unit column stride */
  int64_t o_sm;
  int32_t N, K;
} pp_quad_proj;

/* A run of rows [row0, row1) of projection `proj`, columns [k0, k1), decoded by one
 * wavefront.  plug_lo = first plug entry whose position is >= the position of
 * (row0, 0).  task0 = number of the run's first task (the runs' tasks, groups of
 * pp_*_stream_rows(M) rows, numbered over the whole launch in stream order; the parts of
 * one split task share its number).
 * A run with parts == 1 covers whole rows (k0 = 0, k1 = K) and writes its outputs.
 * A run with parts > 1 is one of `parts` column slices of its rows (split-K for
 * projections with few rows): its float32 partial sums (scaled as the outputs are) are
 * added into the workspace at acc_off + (m*M + j)*N + row (model m, token j), and the
 * last of the parts of a task (counted in the workspace's uint32 counter [task]) writes
 * the fp16 outputs and leaves the accumulators and the counter at zero. */
typedef struct pp_quad_seg {
  int32_t proj;
  int32_t row0;
  int32_t row1;
  int32_t task0;
  int64_t plug_lo;
  int32_t k0, k1;          /* column range */
  int32_t parts;           /* column slices of these rows: 1 = whole rows */
  int32_t reserved;        /* 0 */
  int64_t acc_off;         /* parts > 1: float offset of the projection's accumulators */
} pp_quad_seg;

enum pp_item_flags { PP_ITEM_TAIL = 1, PP_ITEM_FP16 = 2 };

/* Rows that reach the FP16 tails.  PP_ITEM_TAIL: one row, decoded element by element,
 * with its plug range [plug_lo, plug_hi).  PP_ITEM_FP16 (dual stream only): 1..8 rows
 * wholly past n_codes that, for each model, lie wholly inside or wholly past its tail;
 * they need n_codes % 8 == 0, K % 8 == 0 and 16-byte aligned tails. */
typedef struct pp_quad_item {
  int32_t proj;            /* index into projs */
  int32_t row0;            /* first row */
  int32_t nrows;           /* 1 (PP_ITEM_TAIL) or 1..8 (PP_ITEM_FP16) */
  int32_t flags;           /* PP_ITEM_TAIL or PP_ITEM_FP16 */
  int64_t plug_lo;
  int64_t plug_hi;
} pp_quad_item;

/*
 * Batch decode GEMM on the matrix cores (1..64 tokens; used for more than 8):
 *   out_m[i, n] = fp16( s_m * sum_k a[i, k] * W_m[n, k] ),   m = 0..3,
 * for codes laid out (N,K) row-major (row n at codes + n*ldc: the container stream
 * layout, the reference's (K,N) view of it with c_sk == 1), K % 32 == 0.  Each 16-row
 * tile is decoded into fp16 MFMA operands in registers; plug entries (normalised tuples,
 * positions relative to elem_base like pp_quad_gemm) are patched into the decoded
 * tile.  K is cut into `slices` column ranges of slice_cols (a multiple of 32) columns;
 * row_plug[n*slices + s] (n*slices+s+1 entries follow, the last one past the end) is the
 * first plug entry at or after position elem_base + n*ldc + s*slice_cols (searchsorted of
 * those keys, and of elem_base + N*ldc for the last).  With slices > 1 the workspace
 * (pp_quad_mfma_workspace_size bytes) holds float32 partial sums: zero before the first
 * call, left zero by every call; calls that share it must not overlap.  Two launches
 * then (the tiles, and the reduction to fp16).  No counterpart kernel in the reference
 * (its quad_bitpacked_kernel runs every batch size through tl.dot, quad_kernels.py:53-143);
 * this replaces that for M > 8.
 */
int pp_quad_mfma(const uint32_t* codes, int64_t ldc, int64_t elem_base, const void* a, int64_t a_sm,
                 const void* const* luts, int lut_dtype, const float* scales,
                 const uint32_t* plug_idx, const void* plug_vals, int64_t plug_n, const int64_t* row_plug,
                 int64_t slices, int64_t slice_cols, void* const* out, int64_t o_sm,
                 int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, void* stream);
int64_t pp_quad_mfma_workspace_size(int64_t M, int64_t N, int64_t slices);
/* Wavefronts the batch decode launches for M tokens (the host sizes the slices for them). */
int64_t pp_quad_mfma_waves(int64_t M);

/*
 * Fused decode GEMM on the matrix cores (any M >= 1; used for more than 64 tokens, and
 * from 9 tokens on PP_QUAD_KN storage): the same product as pp_quad_mfma, replacing the
 * reference's tl.dot path for its batch sizes (quad_kernels.py:53-67, 123-134, 166-189),
 * with no weight written to memory.  Each code word is decoded once per block of 16, 32,
 * 64 or 128 tokens (the smallest that holds M; the plan depends on M).
 *   layout PP_QUAD_NK: codes (N,K) row-major, row n at codes + n*ldc (ldc >= K, a
 *                      multiple of 4, 16-byte aligned): the container stream layout;
 *   layout PP_QUAD_KN: codes (K,N), row k at codes + k*ldc (ldc >= N): the layout
 *                      pack_quad_layer returns (quad_kernels.py:46-50).
 * K % 32 == 0.  Plug entries (sorted positions, normalised fp16 tuples) are read in an
 * (N,K) frame: the entry of (row n, column k) has position plug_pos0 + n*plug_ld + k
 * (for PP_QUAD_NK storage elem_base and ldc; for PP_QUAD_KN the host moves the positions
 * of the (K,N) storage there and sorts them).  row_plug[n*slices + s] (N*slices + 1
 * entries) is the first entry at or after plug_pos0 + n*plug_ld + s*slice_cols, the last
 * one plug_pos0 + N*plug_ld.  slices / slice_cols come from pp_quad_big_plan; with
 * slices > 1 the workspace (pp_quad_big_workspace_size bytes, 16-byte aligned) holds
 * float32 partial sums: zero before the first call, left zero by every call; calls that
 * share it must not overlap.  No counterpart kernel in the reference.
 */
enum pp_quad_layout { PP_QUAD_NK = 0, PP_QUAD_KN = 1 };
int pp_quad_big(const uint32_t* codes, int layout, int64_t ldc, const void* a, int64_t a_sm,
                const void* const* luts, int lut_dtype, const float* scales,
                const uint32_t* plug_idx, const void* plug_vals, int64_t plug_n, const int64_t* row_plug,
                int64_t plug_pos0, int64_t plug_ld, int64_t slices, int64_t slice_cols,
                void* const* out, int64_t o_sm, int64_t M, int64_t N, int64_t K,
                void* workspace, int64_t workspace_bytes, void* stream);
/* K slices for pp_quad_big at this shape and code layout on the current device (any plan
 * that covers K is valid; this one balances the launch). */
int pp_quad_big_plan(int64_t M, int64_t N, int64_t K, int layout, int64_t* slices, int64_t* slice_cols);
int64_t pp_quad_big_workspace_size(int64_t M, int64_t N, int64_t slices);


/* Rows per wavefront task the stream decode uses for M tokens (0 and an error for bad M). */
int pp_quad_stream_rows(int64_t M);
/* Columns the stream decode reads per row and step for M tokens (0 for bad M): split
 * segments (parts > 1) should cut K at multiples of it. */
int pp_quad_stream_chunk(int64_t M);

/* Number of wavefronts pp_quad_stream launches for M tokens on the current device. */
int64_t pp_quad_stream_waves(int64_t M);

int pp_quad_stream(const pp_quad_proj* projs, int64_t n_projs,
                   const pp_quad_seg* segs, int64_t n_segs, const int64_t* seg_bounds, int64_t n_waves,
                   void* workspace,
                   const pp_quad_item* tail_items, int64_t n_tail,
                   const float* const* luts, const float* scales,
                   const uint32_t* plug_idx, const void* plug_vals, const uint32_t* plug_code, int64_t plug_n,
                   int64_t n_codes, const void* const* tails, const int64_t* tail_len,
                   int64_t M, void* stream);

/*
 * Transpose quad codes from a (K,N) tensor (row stride ldk >= N, as pack_quad_layer
 * returns) to (N,K) rows: out[n*K + k] = codes[k*ldk + n].  No counterpart in the
 * reference: it lets batches of 9-64 tokens on the reference's (K,N) layout run on the
 * matrix-core decode (pp_quad_mfma), which reads (N,K) rows.
 */
int pp_quad_codes_nk(const uint32_t* codes, int64_t ldk, int64_t K, int64_t N, uint32_t* out, void* stream);

/*
 * Plug side table of a quad stream (built once per stream, on the stream's device):
 * code[j] = the code word at stream position plug_idx[j] (0 at or past n_codes).  Given to
 * pp_quad_stream as plug_code, the plug corrections read the plugged words with the plug
 * table instead of gathering them from the code stream (null: they gather).  No
 * counterpart in the reference: a cache of values of its code array
 * (quaternion_packer.py:155-157).
 */
int pp_quad_plug_codes(const uint32_t* codes, int64_t n_codes, const uint32_t* plug_idx, int64_t plug_n,
                       uint32_t* code, void* stream);

/*
 * Plug ranges of the matrix-core kernels (pp_quad_mfma, pp_quad_big, pp_dual_mfma):
 * row_plug[r*slices + s] = the first j with plug_idx[j] >= pos0 + r*pld + s*cols, and
 * row_plug[rows*slices] = the first j with plug_idx[j] >= pos0 + rows*pld (rows*slices + 1
 * entries).  plug_idx ascending.  The search the reference's unpacker makes with
 * torch.searchsorted (quaternion_packer.py:188-189), one launch for every key.
 */
int pp_plug_search(const uint32_t* plug_idx, int64_t plug_n, int64_t pos0, int64_t pld, int64_t rows,
                   int64_t slices, int64_t cols, int64_t* row_plug, void* stream);

/* ------------------------------------------------------------------------ */
/* Dual pack: 16-bit [amp 6 | phase 10] -> 2 models.                          */
/* ------------------------------------------------------------------------ */

/*
 * Fused decode GEMM over a (K,N) code view:
 *   out_1[i,n] = fp16(sum_k a[i,k] * amp(k,n) * cos_lut[ph]),
 *   out_2[i,n] = fp16(sum_k a[i,k] * amp(k,n) * sin_lut[ph]),
 *   amp(k,n)   = amp_lut[amp_q] * bmax[g(k,n)].
 * Group index:  chunk_size == 0 selects the kernel-layout rule
 * g = (k*N + n) // group_size over the logical (K,N) index, whatever the strides
 * (polar_kernels.py:70-71); chunk_size > 0 selects the container rule on the
 * stream position p = elem_base + k*c_sk + n*c_sn, where groups restart every
 * chunk_size positions: g = (p / chunk)*ceil(chunk/gs) + (p % chunk)/gs
 * (polar_bitpack.py:201-203, 224-238).
 * Replaces polar_dual_bitpacked (polar_kernels.py:98-115) and
 * polar_dual_bitpacked_kernel (polar_kernels.py:14-95).
 * Plug entries (optional) replace the amplitude of the pair at
 * plug_idx[j] - elem_base by the fp16 plug_amp[j] (polar_bitpack.py:240-243).
 * Fast paths: c_sk == 1 (container layout) with chunk_size > 0 and M <= 4;
 * c_sn == 1 (the int16 (K,N) tensor quantize_polar_bitpacked returns) with
 * chunk_size == 0, a power-of-two group_size >= 8, N % 8 == 0, K % 8 == 0, in
 * blocks of 8 tokens over a K-slice workspace.  Other layouts decode into the
 * workspace (2*K*N floats); size it with pp_dual_gemm_workspace_size.
 */
int pp_dual_gemm(const void* a, int64_t a_sm, int64_t a_sk,
                 const void* codes, int code_layout, int64_t c_sk, int64_t c_sn,
                 const void* bmax, int64_t group_size, int64_t chunk_size,
                 const void* amp_lut, int amp_lut_n, const void* cos_lut, const void* sin_lut,
                 int phase_n, int lut_dtype,
                 const uint32_t* plug_idx, const void* plug_amp, int64_t plug_n, int64_t elem_base,
                 void* out1, void* out2, int64_t o_sm, int64_t o_sn,
                 int64_t M, int64_t N, int64_t K,
                 void* workspace, int64_t workspace_bytes,
                 void* stream);

int64_t pp_dual_gemm_workspace_size(const void* a, int64_t a_sm, int64_t a_sk,
                                    const void* codes, int64_t c_sk, int64_t c_sn,
                                    int64_t group_size, int64_t chunk_size, int64_t elem_base,
                                    int64_t plug_n, int64_t M, int64_t N, int64_t K);
/* The kernel pp_dual_gemm runs for these operands (enum pp_gemm_kernel above). */
int pp_dual_gemm_kernel(const void* a, int64_t a_sm, int64_t a_sk, const void* codes, int64_t c_sk,
                        int64_t c_sn, int64_t group_size, int64_t chunk_size, int64_t elem_base,
                        int64_t M, int64_t N, int64_t K);

/*
 * Dual decode GEMM on the matrix cores for batches (used for 5-64 tokens, and to 128 on
 * rows of the layout below): the
 * product of polar_dual_bitpacked (polar_kernels.py:27-115) on the int16 (K,N) codes that
 * quantize_polar_bitpacked returns (row k at codes + k*ldk, ldk >= N; stored = code - 32768;
 * group scales bmax[(k*N + n) / group_size], group_size a power of two), each weight rounded
 * to fp16 before the product as the reference's tl.dot takes it, no weight written to
 * memory.  K % 32 == 0.  Plug entries (sorted positions, fp16 amplitudes replacing the
 * table amplitude times the group scale, polar_bitpack.py:240-243) are read in an (N,K)
 * frame: the entry of (column n, row k) has position plug_pos0 + n*plug_ld + k (the host
 * moves the (K,N) storage positions there); row_plug[n*slices + s] (N*slices + 1 entries)
 * is the first entry at or after plug_pos0 + n*plug_ld + s*slice_cols, the last one
 * plug_pos0 + N*plug_ld.  slices / slice_cols from pp_dual_mfma_plan; with slices > 1 the
 * workspace (pp_dual_mfma_workspace_size bytes) holds float32 partial sums: zero before the
 * first call, left zero by every call; calls that share it must not overlap (16-byte
 * aligned).  From 65 tokens, without plug entries, with N a multiple of 16 and of
 * group_size and 16-byte aligned rows, the product runs on producer/consumer workgroups;
 * pp_dual_mfma_plan then returns their plan (any valid plan is accepted either way).
 */
int pp_dual_mfma(const void* codes, int64_t ldk, const void* a, int64_t a_sm, const void* bmax,
                 int64_t group_size, const void* amp_lut, int amp_n, const void* cos_lut,
                 const void* sin_lut, int phase_n, int lut_dtype, const uint32_t* plug_idx,
                 const void* plug_amp, int64_t plug_n, const int64_t* row_plug, int64_t plug_pos0,
                 int64_t plug_ld, int64_t slices, int64_t slice_cols, void* out1, void* out2,
                 int64_t o_sm, int64_t M, int64_t N, int64_t K, void* workspace,
                 int64_t workspace_bytes, void* stream);
/* K slices for pp_dual_mfma at this shape on the current device. */
int pp_dual_mfma_plan(int64_t M, int64_t N, int64_t K, int64_t* slices, int64_t* slice_cols);
int64_t pp_dual_mfma_workspace_size(int64_t M, int64_t N, int64_t slices);

/*
 * The same product over (N,K) rows of a .dualpack stream (the reference's (K,N) view of
 * the container with c_sk == 1, polar_kernels.py:27-115 over unpack_dual_models' layout,
 * polar_bitpack.py:228-247): row n at codes + n*ldc (ldc >= K, a multiple of 8, codes
 * 16-byte aligned), pairs in the file's byte order (PP_DUAL_U16_BE) or the int16 layout;
 * group scales by the container rule on the stream position p = elem_base + n*ldc + k:
 * g = (p / chunk_size) * ceil(chunk_size / group_size) + (p % chunk_size) / group_size,
 * scales[0 .. n_groups).  elem_base % 8 == 0, group_size a power of two >= 8, chunk_size a
 * multiple of 8 in [32, 2^30), K % 32 == 0.  Plug entries are stream positions (sorted);
 * row_plug[n*slices + s] (N*slices + 1 entries) is the first entry at or after elem_base +
 * n*ldc + s*slice_cols, the last one at or after elem_base + N*ldc.  slices / slice_cols
 * from pp_dual_mfma_plan, workspace as pp_dual_mfma's (pp_dual_mfma_workspace_size).  No
 * counterpart kernel in the reference (its container path unpacks to fp16 weights first);
 * used for 5-64 tokens.
 */
int pp_dual_nk_mfma(const void* codes, int code_layout, int64_t ldc, int64_t elem_base, const void* a,
                    int64_t a_sm, const void* scales, int64_t n_groups, int64_t group_size, int64_t chunk_size,
                    const void* amp_lut, int amp_n, const void* cos_lut, const void* sin_lut, int phase_n,
                    int lut_dtype, const uint32_t* plug_idx, const void* plug_amp, int64_t plug_n,
                    const int64_t* row_plug, int64_t slices, int64_t slice_cols, void* out1, void* out2,
                    int64_t o_sm, int64_t M, int64_t N, int64_t K, void* workspace, int64_t workspace_bytes,
                    void* stream);

/* Dequantise to float32 (w1, w2) over a (K,N) view; parity / debug export.
 * Replaces the decode of unpack_dual_models (polar_bitpack.py:228-247). */
int pp_dual_dequant(const void* codes, int code_layout, int64_t c_sk, int64_t c_sn,
                    const void* bmax, int64_t group_size, int64_t chunk_size,
                    const void* amp_lut, int amp_lut_n, const void* cos_lut, const void* sin_lut,
                    int phase_n, int lut_dtype,
                    const uint32_t* plug_idx, const void* plug_amp, int64_t plug_n, int64_t elem_base,
                    float* out1, float* out2, int64_t N, int64_t K, void* stream);

/* The same into fp16 (w1, w2): the rounded weights polar_dual_bitpacked_kernel feeds its
 * dot products (polar_kernels.py:78-82), for a library GEMM at prefill batch sizes
 * (polar_kernels.py:165-184). */
int pp_dual_dequant_f16(const void* codes, int code_layout, int64_t c_sk, int64_t c_sn,
                        const void* bmax, int64_t group_size, int64_t chunk_size,
                        const void* amp_lut, int amp_lut_n, const void* cos_lut, const void* sin_lut,
                        int phase_n, int lut_dtype,
                        const uint32_t* plug_idx, const void* plug_amp, int64_t plug_n, int64_t elem_base,
                        void* out1, void* out2, int64_t N, int64_t K, void* stream);

/* The same, transposed: codes (K,N) with unit column stride and row stride c_sk (>= N, a
 * multiple of 8, 16-byte aligned rows; the layout quantize_polar_bitpacked returns), the
 * kernel's group rule (k*N + n) / group_size with a power-of-two group_size >= 8, into
 * out1[n*K + k] = w1[k, n] and out2 likewise (W^T row-major fp16, for the prefill GEMM
 * that replaces polar_dual_bitpacked_kernel at large batches, polar_kernels.py:165-184).
 * N % 8 == 0, K % 8 == 0, 16-byte aligned outputs.  No counterpart in the reference. */
int pp_dual_dequant_f16_t(const void* codes, int code_layout, int64_t c_sk, const void* bmax, int64_t group_size,
                          const void* amp_lut, int amp_lut_n, const void* cos_lut, const void* sin_lut,
                          int phase_n, int lut_dtype, const uint32_t* plug_idx, const void* plug_amp,
                          int64_t plug_n, int64_t elem_base, void* out1, void* out2, int64_t N, int64_t K,
                          void* stream);

/*
 * Whole-stream dual decode for 1..4 tokens: every projection of a .dualpack stream in
 * one launch.  Same segment / tail-item planning as pp_quad_stream (the structs are
 * shared); projections are described by pp_dual_proj.  Codes are the stream's 16-bit
 * pairs in `code_layout`; scales are the fp16 group maxima (n_groups of them) with the
 * group rule of the file (group_size, chunk_size: groups restart every chunk);
 * amp_lut / cos_lut / sin_lut are float32 tables from the header (64 / 1024 / 1024
 * entries); plug entries replace the amplitude of a pair by an exact fp16 amplitude.
 * plug_ent (2 words per entry, from pp_dual_plug_table for the same projections,
 * pp_dual_stream_rows(M), code layout and amp_lut) is each entry's record, read with the
 * plug window instead of gathering the entry's code and scale from the stream; the
 * kernel takes the amplitude corrections from it (plug_amp is read by the tail rows).
 * Projections need K < 2^19 when plug_n > 0.
 * Positions >= n_codes come from the per-model fp16 tails (tails[m], tail_len[m]): a
 * build-defined extension for streams whose models have different lengths (the file
 * format itself zero-pads the shorter model).
 * The segments' tasks (runs of pp_dual_stream_rows(M) rows, in stream order) are
 * numbered 0 .. n_tasks-1; segs[i].task0 is the number of the segment's first task and
 * task_plug[2t], task_plug[2t+1] are the first plug entry at or after task t's first
 * position and the first one past its last position.  plug_windows (1 or 2) is the
 * number of 64-entry plug windows each decode step takes (2 for dense plug tables).
 * Split segments (parts > 1, columns cut at multiples of pp_dual_stream_chunk(M)) work
 * as in pp_quad_stream: their float32 partial sums go to the workspace (uint32 counter
 * per task, accumulators at acc_off + (m*M + j)*N + row for model m = 0, 1), which must
 * be zero before the first launch and is left zero by each; launches that share it must
 * not overlap.  A null workspace skips split segments.
 * scale_tab (optional, n_tab fp16 entries from pp_dual_scale_table for the same
 * projections and R = pp_dual_stream_rows(M)): with chunk_size % group_size == 0 the row
 * kernel reads each decode step's group scales from it (one load for the R rows of a
 * task) instead of from scales; it requires every projection to have K % group_size == 0,
 * N % R == 0 and pos0 % (R * group_size) == 0.  Null: scales only.
 * Replaces the per-projection polar_dual_bitpacked calls of a decode step
 * (polar_kernels.py:98-115) and the decode of unpack_dual_models
 * (polar_bitpack.py:194-260).
 */
typedef struct pp_dual_proj {
  const void* codes;       /* 16-bit code of (row 0, col 0); row r starts at codes + r*ldc */
  int64_t ldc;             /* row stride in pairs */
  int64_t pos0;            /* stream position of (row 0, col 0) */
  const void* x;           /* fp16 activations (M, K), row stride x_sm */
  int64_t x_sm;
  void* out[2];            /* fp16 outputs (M, N) of the two models, row stride o_sm */
  int64_t o_sm;
  int32_t N, K;
} pp_dual_proj;

int pp_dual_stream_rows(int64_t M);
/* One (N,K) Linear of a dual stream on the stream kernel's one-Linear launch (no reference
 * counterpart: the reference's polar_dual_bitpacked, polar_kernels.py:98-115, makes one call
 * per Linear; this is that call with the per-stream plan of pp_dual_stream done ahead).
 * proj: the Linear (its codes, stream position, activations and outputs, as a pp_dual_proj
 * of pp_dual_stream); task_plug, plug_ent, scale_tab: as pp_dual_stream takes them, for this
 * one projection (tasks of pp_dual_stream_rows(M) rows numbered from its first row); no
 * segments and no tails.  The waves find their rows and column slice from the launch shape;
 * rows with fewer tasks than ~1.5 per wavefront are cut into column slices whose sums meet in
 * the workspace: pp_dual_rows_workspace_size(M, N, K) bytes, zero on entry, left zero by every
 * launch (launches sharing it must not overlap). */
int64_t pp_dual_rows_workspace_size(int64_t M, int64_t N, int64_t K);
/* K parts of pp_dual_rows at this shape (1: whole rows).  When a power of two that divides a
 * workgroup's waves, a task's parts are waves of one workgroup and their sums meet in LDS
 * (no workspace: pp_dual_rows_workspace_size is 0); otherwise they meet in the workspace. */
int pp_dual_rows_parts(int64_t M, int64_t N, int64_t K);
/* The one-Linear launch's per-task plug records (no reference counterpart: a re-layout of
 * pp_dual_plug_table's records): task t's records plug_ent[task_plug[2t] .. task_plug[2t+1])
 * copied to out[t * task_cap ..] (8 bytes each), null records after them; task_cap must be
 * at least every task's entry count.  out holds n_tasks * task_cap records. */
int pp_dual_task_entries(const uint32_t* plug_ent, int64_t plug_n, const int64_t* task_plug, int64_t n_tasks,
                         int64_t task_cap, uint32_t* out, void* stream);
/* task_cap 0: plug_ent holds pp_dual_plug_table's records and task_plug their ranges per task;
 * task_cap > 0: plug_ent holds pp_dual_task_entries' task_cap records per task (task_plug
 * may be null), so a wave loads its task's records without first loading their range. */
int pp_dual_rows(const pp_dual_proj* proj, const int64_t* task_plug, int64_t task_cap, int plug_windows,
                 int code_layout, const void* scales, int64_t n_groups, int64_t group_size, int64_t chunk_size,
                 const void* scale_tab, int64_t n_tab, const float* amp_lut, const float* cos_lut,
                 const float* sin_lut, const uint32_t* plug_idx, const void* plug_amp,
                 const uint32_t* plug_ent, int64_t plug_n, int64_t M, void* workspace,
                 int64_t workspace_bytes, void* stream);
/* Pairs the dual stream decode reads per row and step for M tokens (0 for bad M). */
int pp_dual_stream_chunk(int64_t M);
int64_t pp_dual_stream_waves(int64_t M);

int pp_dual_stream(const pp_dual_proj* projs, int64_t n_projs,
                   const pp_quad_seg* segs, int64_t n_segs, const int64_t* seg_bounds, int64_t n_waves,
                   void* workspace, const int64_t* task_plug, int64_t n_tasks, int plug_windows,
                   const pp_quad_item* tail_items, int64_t n_tail,
                   int code_layout, const void* scales, int64_t n_groups, int64_t group_size, int64_t chunk_size,
                   const void* scale_tab, int64_t n_tab,
                   const float* amp_lut, const float* cos_lut, const float* sin_lut,
                   const uint32_t* plug_idx, const void* plug_amp, const uint32_t* plug_ent, int64_t plug_n,
                   int64_t n_codes, const void* const* tails, const int64_t* tail_len,
                   int64_t M, void* stream);

/*
 * Group scales of a dual stream regrouped for pp_dual_stream's scale_tab (built once per
 * stream plan, on the stream's device): projection i covers stream positions
 * proj_pos0[i] .. proj_pos0[i] + proj_n[i] * proj_k[i] - 1 (rows of proj_k[i] columns;
 * proj_pos0 ascending, n_projs entries).  With R = rows_per_task (8, 4 or 2:
 * pp_dual_stream_rows(M)), for the rows Rb .. Rb+R-1 of projection i, which start at
 * position P = proj_pos0[i] + R b proj_k[i],
 *   tab[P / group_size + R j + q] = scales[(P + q proj_k[i]) / group_size + j]
 * (row Rb + q, column group j); entries outside every projection are copied from scales
 * (0 at or past n_groups).  n_tab >= the end of the last projection / group_size.
 * Requirements as for scale_tab above.  No counterpart in the reference: a reordering of
 * its scale array (polar_bitpack.py:205-211) for the decode's loads.
 */
int pp_dual_scale_table(const void* scales, int64_t n_groups, int64_t group_size, const int64_t* proj_pos0,
                        const int32_t* proj_n, const int32_t* proj_k, int64_t n_projs, int64_t rows_per_task,
                        void* tab, int64_t n_tab, void* stream);

/*
 * Plug records of a dual stream (built once per stream plan, on the stream's device):
 * for entry j at stream position p = plug_idx[j], with c the pair's 16-bit code
 * (amp << 10 | phase, read from codes in code_layout) and s its group scale (group rule
 * of pp_dual_stream),
 *   ent[2j]   = column of p | (row of p in its task of rows_per_task <= 8 rows) << 19 |
 *               phase << 22, where projection i covers [proj_pos0[i], proj_pos0[i+1])
 *               with rows of proj_k[i] < 2^19 columns (proj_pos0 has n_projs + 1
 *               entries; column and row 0 outside);
 *   ent[2j+1] = the float32 bits of d = plug_amp[j] - amp_lut[amp] * s (one rounding),
 *               the correction the decode adds to the pair's amplitude (0 at or past
 *               n_codes).
 * amp_lut is the stream's float32 amplitude table (64 entries, device memory).
 * No counterpart in the reference: an index over its code, scale and plug arrays
 * (polar_bitpack.py:205-211) for the plug correction.
 */
int pp_dual_plug_table(const void* codes, int64_t n_codes, int code_layout, const void* scales, int64_t n_groups,
                       int64_t group_size, int64_t chunk_size, const float* amp_lut, const uint32_t* plug_idx,
                       const void* plug_amp, int64_t plug_n, const int64_t* proj_pos0, const int32_t* proj_k,
                       int64_t n_projs, int64_t rows_per_task, uint32_t* ent, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* POLAR_PACK_H */
