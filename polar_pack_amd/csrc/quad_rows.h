// Host-side entry into the fused quad decode kernel (quad_rows.hip), shared with the
// single-projection operator in quad.hip.
#pragma once

#include "pp_common.h"

namespace pp {

// True when the fused row kernel can serve this (M, K) view: codes rows (N,K)
// row-major with 16-byte aligned rows, contiguous fp16 activations, M <= 8.
bool quad_rows_ok(const void* a, int64_t a_sm, int64_t a_sk, const uint32_t* codes, int64_t c_sk, int64_t c_sn,
                  int64_t M, int64_t N, int64_t K);

// Workspace bytes quad_rows_single needs (per-wave plug starts), 0 without a plug table.
int64_t quad_rows_workspace(int64_t M, int64_t N, int64_t plug_n);

// out_m[i, n*o_sn + i*o_sm] = fp16(s_m * sum_k a[i,k] W_m[n,k]) over codes rows (N,K).
int quad_rows_single(const void* a, int64_t a_sm, const uint32_t* codes, int64_t ldc, const void* const* luts,
                     int lut_dtype, const float* scales, const uint32_t* plug_idx, const void* plug_vals,
                     int64_t plug_n, int64_t elem_base, void* const* out, int64_t o_sm, int64_t o_sn, int64_t M,
                     int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, hipStream_t st);

}  // namespace pp
