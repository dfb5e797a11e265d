// Error plumbing and library identity for the C ABI.
#include <cstdarg>
#include <cstdio>
#include <string>

#include "common.hpp"

namespace sm {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

}  // namespace sm

extern "C" int sm_version(void) { return 1; }

extern "C" const char* sm_last_error(void) { return sm::g_last_error.c_str(); }
