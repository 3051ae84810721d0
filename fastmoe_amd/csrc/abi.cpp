// Version and thread-local error string of the C ABI (host code only).
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/fastmoe_amd.h"

namespace fmoe_host {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

}  // namespace fmoe_host

extern "C" int fmoe_abi_version(void) { return FMOE_ABI_VERSION; }

extern "C" const char* fmoe_last_error(void) { return fmoe_host::g_last_error.c_str(); }
