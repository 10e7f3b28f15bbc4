#include "ttlh_common.h"
extern "C" int ttlh_bfp8_pack_host(const float*, void*, int64_t, int64_t) { ttlh::set_error("not built"); return TTLH_EUNSUPPORTED; }
extern "C" int ttlh_bfp8_unpack_host(const void*, uint16_t*, int64_t, int64_t) { ttlh::set_error("not built"); return TTLH_EUNSUPPORTED; }
extern "C" int ttlh_bfp8_unpack(const void*, void*, int64_t, int64_t, void*) { ttlh::set_error("not built"); return TTLH_EUNSUPPORTED; }
extern "C" int ttlh_matmul_bfp8w(const void*, int64_t, const void*, void*, int64_t, int64_t, int64_t, int64_t, void*) { ttlh::set_error("not built"); return TTLH_EUNSUPPORTED; }
