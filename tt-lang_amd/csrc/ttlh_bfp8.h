// Device decode of bfloat8_b element bytes (format: bfp8.hip header).
#pragma once

#include "ttlh_common.h"

namespace ttlh {

// 8 element bytes sharing exponent e -> 8 bf16 packed in 4 dwords (element 0
// in the low half of dword 0).  value = (-1)^s * m * 2^(e - 133): m is
// converted to fp32 (exact), scaled by v_ldexp_f32 (exact, the result has at
// most 7 significant bits and, for e < 7, is an fp32 subnormal whose low 16
// bits are zero), and the top half of the fp32 pattern is the exact bf16.
__device__ __forceinline__ uint32_t bfp8_decode1(uint32_t b, int sh) {
  const float f = __builtin_amdgcn_ldexpf(static_cast<float>(b & 0x7fu), sh);
  return (__float_as_uint(f) >> 16) | ((b & 0x80u) << 8);
}

__device__ __forceinline__ u32x4 bfp8_decode8(uint64_t bytes, uint8_t e) {
  const int sh = static_cast<int>(e) - 133;
  const uint32_t lo = static_cast<uint32_t>(bytes), hi = static_cast<uint32_t>(bytes >> 32);
  u32x4 r;
  r.x = bfp8_decode1(lo & 0xff, sh) | (bfp8_decode1((lo >> 8) & 0xff, sh) << 16);
  r.y = bfp8_decode1((lo >> 16) & 0xff, sh) | (bfp8_decode1(lo >> 24, sh) << 16);
  r.z = bfp8_decode1(hi & 0xff, sh) | (bfp8_decode1((hi >> 8) & 0xff, sh) << 16);
  r.w = bfp8_decode1((hi >> 16) & 0xff, sh) | (bfp8_decode1(hi >> 24, sh) << 16);
  return r;
}

// One bfloat4_b nibble (bit 3 sign, bits 2..0 magnitude m) with shift
// sh = e - 129 -> bf16 bits of (-1)^s * m * 2^sh: converted and scaled
// exactly as for bfloat8_b (at most 3 significant bits).
__device__ __forceinline__ uint32_t bfp4_decode1(uint32_t n, int sh) {
  const float f = __builtin_amdgcn_ldexpf(static_cast<float>(n & 7u), sh);
  return (__float_as_uint(f) >> 16) | ((n & 8u) << 12);
}

}  // namespace ttlh
