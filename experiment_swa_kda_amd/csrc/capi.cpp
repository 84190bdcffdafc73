// Thread-local error state and version of libkda_mi355x.
#include <mutex>
#include <set>
#include <string>
#include <tuple>

#include "kda_host.hpp"

namespace kda {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

hipError_t ensure_lds_limit(const void* kernel, int bytes) {
  static std::mutex mu;
  static std::set<std::tuple<const void*, int, int>> done;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(kernel, dev, bytes);
  if (done.count(key)) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.insert(key);
  return e;
}

}  // namespace kda

extern "C" const char* kda_last_error(void) { return kda::g_last_error.c_str(); }

extern "C" const char* kda_version(void) { return "kda_mi355x 0.1 gfx950"; }
