// Thread-local error state and version of libkda_mi355x.
#include <string>

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

}  // namespace kda

extern "C" const char* kda_last_error(void) { return kda::g_last_error.c_str(); }

extern "C" const char* kda_version(void) { return "kda_mi355x 0.1 gfx950"; }
