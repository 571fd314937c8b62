// LDS decode tables of the dual-pack kernels (dual_rows.hip, dual_kn.hip) and their
// lookups.
//
// (cos, sin) of the 1024 phases in 128-byte rows of 16 replicas (lane l reads replica
// l % 16, so a wavefront's 64 reads of 8 bytes spread over the banks), the 64 amplitudes
// one per 4-byte bank (a wave's 64 reads hit distinct banks or share one address, so no
// replicas).  For the int16 layout (stored = code ^ 0x8000, polar_kernels.py:9-11) the
// amplitude entry a holds amp_lut[a ^ 32], so the stored bits index it directly.
#pragma once

#include "pp_common.h"

namespace pp {

// The decode tables as the caller holds them: amp_lut[amp_n], cos_lut / sin_lut[phase_n],
// fp16 or float32 (dtype); indices past amp_n / phase_n decode to 0.
struct DualLuts {
  const void* amp;
  const void* cs[2];  // cos, sin
  int amp_n, phase_n, dtype;
};

constexpr uint32_t DLDS_AMP = 0;               // the 64 amplitudes, 4 bytes each: one per LDS bank
constexpr uint32_t DLDS_CS = 0x400;            // (cos, sin) rows: phase p at DLDS_CS + p*128 + 8*(lane % 16)
constexpr uint32_t DLDS_BYTES = 0x400 + 1024 * 128;

// Stored 32-bit word (two pairs) -> two codes in the table-index form: the file layout is
// byte-swapped per half, the int16 layout is used as stored.
template <int LAYOUT>
__device__ __forceinline__ uint32_t dual_word(uint32_t w) {
  if constexpr (LAYOUT == PP_DUAL_U16_BE) return __builtin_amdgcn_perm(w, w, 0x02030001u);
  else return w;
}
template <int LAYOUT>
__device__ __forceinline__ uint32_t dual_half(uint32_t h16) {
  if constexpr (LAYOUT == PP_DUAL_U16_BE) return ((h16 & 0xFFu) << 8) | ((h16 >> 8) & 0xFFu);
  else return h16 & 0xFFFFu;
}

struct DualLane {
  uint32_t cs;        // the lane's replica inside a (cos, sin) row
};

__device__ __forceinline__ DualLane dual_lane(int l) {
  DualLane o;
  o.cs = 8u * (l & 15);
  return o;
}

// Amplitude and (cos, sin) of both codes of a stored 32-bit word.  The amplitude table
// needs no replicas (a wave's 64 reads hit distinct banks or share one address), so its
// byte offset, 4 * amp bits, comes straight out of the stored word: byte 0 / byte 2 of
// a big-endian word, byte 1 / byte 3 of the int16 layout, masked with 0xFC.
template <int LAYOUT>
__device__ __forceinline__ void dual_lookup2(const char* lds, uint32_t raw, const DualLane& o, float (&an)[2],
                                             float2 (&cs)[2]) {
  const uint32_t a0 = (LAYOUT == PP_DUAL_U16_BE ? raw : raw >> 8) & 0xFCu;
  const uint32_t a1 = (raw >> (LAYOUT == PP_DUAL_U16_BE ? 16 : 24)) & 0xFCu;
  const uint32_t w = dual_word<LAYOUT>(raw);
  const uint32_t c0 = ((w << 7) & 0x1FF80u) | o.cs;
  const uint32_t c1 = ((w >> 9) & 0x1FF80u) | o.cs;
  an[0] = *reinterpret_cast<const float*>(lds + DLDS_AMP + a0);
  an[1] = *reinterpret_cast<const float*>(lds + DLDS_AMP + a1);
  cs[0] = *reinterpret_cast<const float2*>(lds + DLDS_CS + c0);
  cs[1] = *reinterpret_cast<const float2*>(lds + DLDS_CS + c1);
}

// The same for one code in the table-index form (amp bits 10..15, phase 0..9).
__device__ __forceinline__ void dual_lookup1(const char* lds, uint32_t c, const DualLane& o, float& an, float2& cs) {
  an = *reinterpret_cast<const float*>(lds + DLDS_AMP + ((c >> 8) & 0xFCu));
  cs = *reinterpret_cast<const float2*>(lds + DLDS_CS + (((c << 7) & 0x1FF80u) | o.cs));
}

// Build the tables of a workgroup of NT threads (a multiple of 64) from the caller's LUTs
// (entries of type E): every LUT load of a thread is issued before its stores, the
// (cos, sin) rows written as 16-byte units in address order.  For the int16 layout
// (stored = code ^ 0x8000) amplitude entry a holds amp_lut[a ^ 32].  Ends with a barrier.
template <int NT, int LAYOUT, typename E>
__device__ __forceinline__ void dual_tables_of(char* lds, const DualLuts& L) {
  constexpr int KU = (8192 + NT - 1) / NT;
  const E* cp = reinterpret_cast<const E*>(L.cs[0]);
  const E* sp = reinterpret_cast<const E*>(L.cs[1]);
  float c[KU], s[KU];
#pragma unroll
  for (int k = 0; k < KU; ++k) {
    const int p = (threadIdx.x + k * NT) >> 3;
    c[k] = p < L.phase_n ? (float)cp[p] : 0.f;
    s[k] = p < L.phase_n ? (float)sp[p] : 0.f;
  }
  if (threadIdx.x < 64) {
    const int e = LAYOUT == PP_DUAL_I16_OFFSET ? (threadIdx.x ^ 32) : threadIdx.x;
    *reinterpret_cast<float*>(lds + DLDS_AMP + 4 * threadIdx.x) =
        e < L.amp_n ? (float)reinterpret_cast<const E*>(L.amp)[e] : 0.f;
  }
#pragma unroll
  for (int k = 0; k < KU; ++k)
    if (threadIdx.x + k * NT < 8192)
      *reinterpret_cast<float4*>(lds + DLDS_CS + 16 * (threadIdx.x + k * NT)) = make_float4(c[k], s[k], c[k], s[k]);
  __syncthreads();
}

}  // namespace pp
