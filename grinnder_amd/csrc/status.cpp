// Thread-local error reporting for the C ABI.
#include "gr_internal.h"

namespace gr {

static thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

const char* last_error_cstr() { return g_last_error.c_str(); }

}  // namespace gr

extern "C" const char* gr_last_error(void) { return gr::last_error_cstr(); }

extern "C" int gr_abi_version(void) { return 100; }

#ifndef GR_SOURCE_HASH
#error "GR_SOURCE_HASH must be defined by the build (grinnder_amd/build.py)"
#endif

extern "C" const char* gr_source_hash(void) { return GR_SOURCE_HASH; }
