// pp_quad_gemm_noalloc: pp_quad_gemm for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// pp_quad_gemm's kernels take a caller-provided workspace: the per-wavefront plug starts of
// the row kernel (container (N,K) rows with plug entries), the K-slice partial sums of the
// (K,N) kernel, or the float32 decode of the generic layouts.  Here that workspace is the
// file-scope device array `scratch` (PP_NOALLOC_SCRATCH_BYTES, held by every GPU the library
// runs on until the process ends).  Its device address is looked up once per device with
// hipGetSymbolAddress and cached; host code never passes the array's name to a kernel.
//
// Every kernel of those paths writes each workspace slot it later reads, within the call,
// so nothing has to start at zero and no clearing pass is needed.  Calls on one GPU share
// its array: two calls whose work overlaps on that GPU (different streams, or one stream
// used from several threads without ordering) race on it.
#include "pp_common.h"

#include <mutex>

namespace pp {

static __device__ __align__(256) unsigned char scratch[PP_NOALLOC_SCRATCH_BYTES];

static constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on the first call on each device).
static int scratch_address(void** out) {
  int dev = 0;
  PP_HIP(hipGetDevice(&dev));
  PP_REQUIRE(dev >= 0 && dev < kMaxDevices, "device %d is beyond the %d devices the scratch table holds", dev,
             kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    PP_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    PP_REQUIRE(p != nullptr, "hipGetSymbolAddress returned a null scratch address on device %d", dev);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PP_OK;
}

}  // namespace pp

extern "C" int pp_quad_gemm_noalloc(const void* a, int64_t a_sm, int64_t a_sk, const uint32_t* codes, int64_t c_sk,
                                    int64_t c_sn, const void* const* luts, int lut_dtype, const float* scales,
                                    const uint32_t* plug_idx, const void* plug_vals, int64_t plug_n,
                                    int64_t elem_base, void* const* out, int64_t o_sm, int64_t o_sn, int64_t M,
                                    int64_t N, int64_t K, void* stream) {
  PP_REQUIRE(M >= 0 && N >= 0 && K >= 0, "negative shape");
  PP_REQUIRE(plug_n >= 0, "negative plug count");
  const int64_t need = pp_quad_gemm_workspace_size(a, a_sm, a_sk, codes, c_sk, c_sn, plug_n, M, N, K);
  PP_REQUIRE(need <= PP_NOALLOC_SCRATCH_BYTES,
             "this call needs %lld bytes of scratch; pp_quad_gemm_noalloc holds %lld (use pp_quad_gemm with a "
             "workspace)",
             (long long)need, (long long)PP_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0 && M > 0 && N > 0)
    if (int rc = pp::scratch_address(&ws)) return rc;
  return pp_quad_gemm(a, a_sm, a_sk, codes, c_sk, c_sn, luts, lut_dtype, scales, plug_idx, plug_vals, plug_n,
                      elem_base, out, o_sm, o_sn, M, N, K, ws, ws != nullptr ? PP_NOALLOC_SCRATCH_BYTES : 0, stream);
}
