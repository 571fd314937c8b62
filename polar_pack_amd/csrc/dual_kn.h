// Host-side entry into the fused dual decode of (K,N) codes with unit column stride
// (dual_kn.hip), used by the single-projection operator in dual.hip.
#pragma once

#include "pp_common.h"

namespace pp {

struct DualLuts;

// True when dual_kn_gemm can serve this view for M (1..8) tokens: codes (K,N) with
// c_sn == 1, rows of a multiple of 8 codes, 16-byte aligned; N % 8 == 0, K % 8 == 0;
// groups by the kernel rule (k*N + n) / gs (chunk_size 0) with gs a power of two >= 8;
// contiguous, 16-byte aligned fp16 activations.
bool dual_kn_ok(const void* a, int64_t a_sm, int64_t a_sk, const void* codes, int64_t c_sk, int64_t c_sn,
                int64_t group_size, int64_t chunk_size, int64_t M, int64_t N, int64_t K);

// Workspace bytes dual_kn_gemm needs (the K slices' float32 partial sums), 0 when the
// launch writes its outputs directly.
int64_t dual_kn_workspace(int64_t M, int64_t N, int64_t K, int64_t plug_n);

// out_m[j*o_sm + n*o_sn] = fp16(sum_k a[j,k] W_m[k,n]), m = 0, 1, over codes (K,N) with
// row stride ldk; plug entries (positions relative to elem_base in that storage) replace
// the amplitude of their pair.
int dual_kn_gemm(const void* a, int64_t a_sm, const void* codes, int code_layout, int64_t ldk, const void* bmax,
                 int64_t group_size, const DualLuts& luts, const uint32_t* plug_idx, const void* plug_amp,
                 int64_t plug_n, int64_t elem_base, void* const* out, int64_t o_sm, int64_t o_sn, int64_t M,
                 int64_t N, int64_t K, void* workspace, int64_t workspace_bytes, hipStream_t st);

}  // namespace pp
