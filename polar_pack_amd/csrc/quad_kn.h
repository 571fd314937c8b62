// Host-side entry into the fused decode of (K,N) codes with unit column stride
// (quad_kn.hip), used by the single-projection operator in quad.hip.
#pragma once

#include "pp_common.h"

namespace pp {

// True when quad_kn_gemm can serve this view for M (1..8) tokens: codes (K,N) with
// c_sn == 1, rows of a multiple of 4 words, 16-byte aligned; N % 4 == 0, K % 8 == 0;
// contiguous, 16-byte aligned fp16 activations.
bool quad_kn_ok(const void* a, int64_t a_sm, int64_t a_sk, const uint32_t* codes, int64_t c_sk, int64_t c_sn,
                int64_t M, int64_t N, int64_t K);

// Workspace bytes quad_kn_gemm needs (the K slices' float32 partial sums), 0 when the
// launch writes its outputs directly.
int64_t quad_kn_workspace(int64_t M, int64_t N, int64_t K, int64_t plug_n);

// out_m[j*o_sm + n*o_sn] = fp16(s_m * sum_k a[j,k] W_m[k,n]) over codes (K,N), row stride ldk.
int quad_kn_gemm(const void* a, int64_t a_sm, const uint32_t* codes, int64_t ldk, const void* const* luts,
                 int lut_dtype, const float* scales, const uint32_t* plug_idx, const void* plug_vals, int64_t plug_n,
                 int64_t elem_base, void* const* out, int64_t o_sm, int64_t o_sn, int64_t M, int64_t N, int64_t K,
                 void* workspace, int64_t workspace_bytes, hipStream_t st);

}  // namespace pp
