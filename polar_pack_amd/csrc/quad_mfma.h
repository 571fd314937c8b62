// Device helpers shared by the matrix-core quad decode kernels (quad_mfma.hip: 1..64
// tokens, quad_big.hip: larger batches): the decode of 8 code words into the fp16 A
// operands of v_mfma_f32_16x16x32_f16 for the 4 models, and the per-lane window of plug
// entries patched into those operands (quaternion_packer.py:187-193).
#pragma once

#include "quad_lds.h"
#include "finish_tile.h"
#include "rows_common.h"

namespace pp {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// The plug table: sorted stream positions and (P, 4) normalised fp16 values.
struct PlugSrc {
  const uint32_t* idx;
  const f16* vals;
  int64_t n;
};

// The lane's window of MPW plug entries of its row: columns (INT_MAX past the end, INT_MIN
// once applied) and values.
#ifndef PP_MPW
#define PP_MPW 4
#endif
constexpr int MPW = PP_MPW;
struct MPlug {
  int k[MPW];
  u32x2 v[MPW];
  int64_t next, end;       // next entry to load, end of the row's entries in the slice
};

// Load the next MPW entries of the row (bounds-checked buffer loads, nothing past `end`).
__device__ __forceinline__ void mplug_issue(const PlugSrc& S, MPlug& P, uint32_t (&idx)[MPW]) {
  const rsrc_t ri = make_rsrc(S.idx, 4u * (uint32_t)S.n);
  const rsrc_t rv = make_rsrc(S.vals, 8u * (uint32_t)S.n);
#pragma unroll
  for (int i = 0; i < MPW; ++i) {
    const int64_t e = P.next + i;
    const bool has = e < P.end;
    vload32(idx[i], has ? 4u * (uint32_t)e : OOB, ri);
    vload64(P.v[i], has ? 8u * (uint32_t)e : OOB, rv);
  }
}
__device__ __forceinline__ void mplug_take(MPlug& P, const uint32_t (&idx)[MPW], int64_t rowpos) {
#pragma unroll
  for (int i = 0; i < MPW; ++i) P.k[i] = P.next + i < P.end ? (int)((int64_t)idx[i] - rowpos) : 0x7FFFFFFF;
  P.next += MPW;
}

// Decode 8 code words into the fp16 A operands of the 4 models (each tuple rounded
// once, as soon as it is decoded: the fp32 values are not kept).  The table reads of a
// group of GT tuples are issued before the arithmetic of the previous group (scheduling
// fences keep them there), so a wave has up to 8 GT reads in flight instead of waiting
// for each tuple's four reads in turn.
#ifndef PP_MFMA_GT
#define PP_MFMA_GT 2
#endif
template <class L>
__device__ __forceinline__ void decode8(const char* lds, const LaneOff& lo, const u32x4& c0, const u32x4& c1,
                                        h8 (&a)[4]) {
  const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  constexpr int GT = PP_MFMA_GT, NG = 8 / GT;
  static_assert(8 % GT == 0, "the group must divide 8 tuples");
  float r[2][GT];
  float2 ta[2][GT], tb[2][GT], tc[2][GT];
#pragma unroll
  for (int u = 0; u < GT; ++u) lookup<L>(lds, cw[u], lo, r[0][u], ta[0][u], tb[0][u], tc[0][u]);
#pragma unroll
  for (int g = 0; g < NG; ++g) {
    if (g + 1 < NG) {
#pragma unroll
      for (int u = 0; u < GT; ++u) {
        const int b = (g + 1) & 1;
        lookup<L>(lds, cw[(g + 1) * GT + u], lo, r[b][u], ta[b][u], tb[b][u], tc[b][u]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < GT; ++u) {
      const int b = g & 1, e = g * GT + u;
      const float rs = r[b][u] * ta[b][u].y, rss = rs * tb[b][u].y;
      a[0][e] = (_Float16)(r[b][u] * ta[b][u].x);
      a[1][e] = (_Float16)(rs * tb[b][u].x);
      a[2][e] = (_Float16)(rss * tc[b][u].x);
      a[3][e] = (_Float16)(rss * tc[b][u].y);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Patch the plug entries of the lane's 8 columns kk .. kk+7 (step columns ks .. ks+31)
// into its operands: the decoded tuple is replaced by the plug values, one entry per
// pass (two in one lane's 8 columns of one step are rare); a window used up within the
// step is refilled.  Wave-uniform control flow: the common case is one compare per
// window entry and one ballot.
__device__ __forceinline__ void mplug_patch_loop(const PlugSrc& S, MPlug& P, int64_t rowpos, int kk, int ks,
                                                 h8 (&a)[4]) {
  for (;;) {
    int hit = -1;
#pragma unroll
    for (int i = MPW - 1; i >= 0; --i) hit = (unsigned)(P.k[i] - kk) < 8u ? i : hit;
    if (__ballot(hit >= 0)) {
      int kh = kk - 1;
      u32x2 pv2 = P.v[0];
#pragma unroll
      for (int i = 0; i < MPW; ++i) {
        kh = hit == i ? P.k[i] : kh;
        pv2 = hit == i ? P.v[i] : pv2;
      }
      const int e = kh - kk;   // -1 in a lane without a hit
      const f16x4 pv = __builtin_bit_cast(f16x4, pv2);
      const _Float16 v[4] = {(_Float16)pv.x, (_Float16)pv.y, (_Float16)pv.z, (_Float16)pv.w};
#pragma unroll
      for (int ee = 0; ee < 8; ++ee)
#pragma unroll
        for (int m = 0; m < 4; ++m) a[m][ee] = e == ee ? v[m] : a[m][ee];
#pragma unroll
      for (int i = 0; i < MPW; ++i) P.k[i] = hit == i ? (int)0x80000000 : P.k[i];
      continue;
    }
    const bool refill = P.k[MPW - 1] < ks + 32 && P.next < P.end;
    if (!__ballot(refill)) break;
    // rare: load and wait here, so no load is left in flight past this branch (a
    // possibly pending load would make every later wait drain the prefetch too)
    uint32_t idx[MPW];
    MPlug R = P;
    mplug_issue(S, R, idx);
#pragma unroll
    for (int i = 0; i < MPW; ++i) asm volatile("" : : "v"(idx[i]), "v"(R.v[i]));
    mplug_take(R, idx, rowpos);
    if (refill) P = R;
  }
}

// The common case outside the loop (no entry in the step, no refill due), so the step
// does not enter a loop that carries the operands.
__device__ __forceinline__ void mplug_patch(const PlugSrc& S, MPlug& P, int64_t rowpos, int kk, int ks, h8 (&a)[4]) {
  bool any = P.k[MPW - 1] < ks + 32 && P.next < P.end;
#pragma unroll
  for (int i = 0; i < MPW; ++i) any = any || (unsigned)(P.k[i] - kk) < 8u;
  if (__ballot(any)) mplug_patch_loop(S, P, rowpos, kk, ks, a);
}

// The same patch for operands already written to LDS (the producer waves of the large-batch
// kernel): model m's 8 fp16 values of the lane at base + m * mstride.  A lane whose columns
// hold an entry stores its 4 values there, 2 bytes each, after the operand stores (the
// same wave's LDS operations complete in order), so the common step keeps no operands in
// registers across a branch; entries are applied in table order (a duplicate position
// keeps the last entry) and re-applying an entry stores the same values again.
__device__ __forceinline__ void mplug_apply_lds(const MPlug& P, int kk, char* base, uint32_t mstride) {
  bool any = false;
#pragma unroll
  for (int i = 0; i < MPW; ++i) any = any || (unsigned)(P.k[i] - kk) < 8u;
  if (!__ballot(any)) return;
#pragma unroll
  for (int i = 0; i < MPW; ++i) {
    const int e = P.k[i] - kk;
    if ((unsigned)e < 8u) {
      const f16x4 pv = __builtin_bit_cast(f16x4, P.v[i]);
#pragma unroll
      for (int m = 0; m < 4; ++m) *reinterpret_cast<f16*>(base + m * mstride + 2 * e) = pv[m];
    }
  }
}
__device__ __forceinline__ void mplug_patch_lds(const PlugSrc& S, MPlug& P, int64_t rowpos, int kk, int ks, char* base,
                                                uint32_t mstride) {
  mplug_apply_lds(P, kk, base, mstride);
  // the refill loop only when a lane needs one, so the common step carries no window
  // state through a loop
  if (!__ballot(P.k[MPW - 1] < ks + 32 && P.next < P.end)) return;
  for (;;) {
    const bool refill = P.k[MPW - 1] < ks + 32 && P.next < P.end;
    if (!__ballot(refill)) break;
    // rare: load and wait here (as in mplug_patch_loop)
    uint32_t idx[MPW];
    MPlug R = P;
    mplug_issue(S, R, idx);
#pragma unroll
    for (int i = 0; i < MPW; ++i) asm volatile("" : : "v"(idx[i]), "v"(R.v[i]));
    mplug_take(R, idx, rowpos);
    if (refill) P = R;
    mplug_apply_lds(P, kk, base, mstride);
  }
}

}  // namespace pp
