// Library-wide C-ABI pieces: thread-local error text, version, cached device facts.
#include "pp_common.h"

#include <mutex>
#include <vector>

namespace pp {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

// The current device's side stream and its fork / join events, created on first use and
// kept until the process ends; default priority.  side_lock serialises the enqueue of a
// fork / side launch / join sequence, so that concurrent callers do not cross events.
std::mutex& side_lock() {
  static std::mutex mu;
  return mu;
}

int side_stream(hipStream_t* side, hipEvent_t* fork, hipEvent_t* join) {
  struct Side {
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
  };
  static std::mutex mu;
  static std::vector<Side> cache;
  int dev = 0;
  PP_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1);
  Side& c = cache[dev];
  if (c.s == nullptr) {
    PP_HIP(hipStreamCreateWithFlags(&c.s, hipStreamNonBlocking));
    PP_HIP(hipEventCreateWithFlags(&c.fork, hipEventDisableTiming));
    PP_HIP(hipEventCreateWithFlags(&c.join, hipEventDisableTiming));
  }
  *side = c.s;
  *fork = c.fork;
  *join = c.join;
  return PP_OK;
}

int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace pp

extern "C" const char* pp_last_error(void) { return pp::g_last_error.c_str(); }

extern "C" const char* pp_version(void) { return "polar_pack_amd 0.1 gfx950"; }

extern "C" int pp_abi_sizes(int64_t* out, int n) {
  const int64_t v[4] = {(int64_t)sizeof(pp_quad_proj), (int64_t)sizeof(pp_quad_item),
                        (int64_t)sizeof(pp_quad_seg), (int64_t)sizeof(pp_dual_proj)};
  int k = 0;
  for (; k < n && k < 4; ++k) out[k] = v[k];
  return k;
}
