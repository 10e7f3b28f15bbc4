#include "ttlh_common.h"
extern "C" int ttlh_matmul(const void*, int, int64_t, const void*, int, int64_t, void*, int,
                           int64_t, int64_t, int64_t, int64_t, int, void*) {
  ttlh::set_error("ttlh_matmul: not built yet");
  return TTLH_EUNSUPPORTED;
}
