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

// 16 bfloat4_b nibbles (element c in bits 4c..4c+3) sharing exponent e ->
// 16 bf16 in two u32x4.  value = (-1)^s * m * 2^(e - 129): converted and
// scaled exactly as for bfloat8_b (at most 3 significant bits).
__device__ __forceinline__ uint32_t bfp4_decode1(uint32_t n, int sh) {
  const float f = __builtin_amdgcn_ldexpf(static_cast<float>(n & 7u), sh);
  return (__float_as_uint(f) >> 16) | ((n & 8u) << 12);
}

__device__ __forceinline__ void bfp4_decode16(uint64_t nib, uint8_t e, u32x4& lo, u32x4& hi) {
  const int sh = static_cast<int>(e) - 129;
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t b = static_cast<uint32_t>(nib >> (8 * i)) & 0xffu;
    w[i] = bfp4_decode1(b & 0xfu, sh) | (bfp4_decode1(b >> 4, sh) << 16);
  }
  lo = u32x4{w[0], w[1], w[2], w[3]};
  hi = u32x4{w[4], w[5], w[6], w[7]};
}

}  // namespace ttlh
