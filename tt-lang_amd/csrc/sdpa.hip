#include "ttlh_common.h"
extern "C" int ttlh_sdpa_fwd(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t, int64_t, float, int, void*) { ttlh::set_error("not built"); return TTLH_EUNSUPPORTED; }
