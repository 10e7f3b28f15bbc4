// Library-wide pieces of libttlhip.so: thread-local error text and version.
// The error convention mirrors the reference's boundary, where validation
// failures surface as ValueError / RuntimeError with a message
// (python/ttl/ttl_api.py:733-737); here a status code plus
// ttlh_last_error(), which the Python layer turns into those exceptions.

#include "ttlh_common.h"

namespace ttlh {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error.assign(buf);
}

void clear_error() { g_last_error.clear(); }

}  // namespace ttlh

extern "C" const char* ttlh_last_error(void) { return ttlh::g_last_error.c_str(); }

extern "C" int ttlh_version(void) { return TTLH_ABI_VERSION; }
