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
