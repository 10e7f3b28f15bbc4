// Shared helpers for the gfx950 kernels of libttlhip.so: bf16 bit
// conversions, error reporting and launch checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <string>

#include "../../include/ttlhip.h"

namespace ttlh {

// native clang vectors (usable with the nontemporal / buffer builtins)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---- error reporting (thread-local message, returned by ttlh_last_error) --
void set_error(const char* fmt, ...);
void clear_error();

#define TTLH_REQUIRE(cond, code, ...)     \
  do {                                    \
    if (!(cond)) {                        \
      ::ttlh::set_error(__VA_ARGS__);     \
      return (code);                      \
    }                                     \
  } while (0)

#define TTLH_HIP_CHECK(expr)                                                  \
  do {                                                                        \
    hipError_t _e = (expr);                                                   \
    if (_e != hipSuccess) {                                                   \
      ::ttlh::set_error("%s failed: %s", #expr, hipGetErrorString(_e));       \
      return TTLH_EHIP;                                                       \
    }                                                                         \
  } while (0)

// Checks the launch that was just enqueued.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("launch of %s failed: %s", what, hipGetErrorString(e));
    return TTLH_EHIP;
  }
  return TTLH_OK;
}

// ---- bf16 <-> fp32 ----------------------------------------------------
// bf16 is the upper half of an IEEE fp32.  Rounding is round-to-nearest-even,
// NaN stays a quiet NaN: the conversion torch applies when it materialises a
// bfloat16 tensor (the simulator's rounding point after every tile op).
__host__ __device__ inline float bf16_to_f32(uint16_t h) {
  union {
    uint32_t u;
    float f;
  } v;
  v.u = static_cast<uint32_t>(h) << 16;
  return v.f;
}

__host__ __device__ inline uint16_t f32_to_bf16(float f) {
  union {
    uint32_t u;
    float f;
  } v;
  v.f = f;
  uint32_t u = v.u;
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__host__ __device__ inline float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// packs two fp32 into two RNE bf16 in one dword (lo = a, hi = b)
__device__ inline uint32_t pack_bf16x2(float a, float b) {
  return static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
}

// (lo, hi) -> two bf16 in one dword (lo in the low half), round to nearest
// even, NaN -> quiet NaN: one v_cvt_pk_bf16_f32 (a vector conversion; two
// scalar conversions would cost a conversion each plus a shift and an or).
__device__ __forceinline__ uint32_t cvt_pk_bf16x2(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

inline int num_cus() {
  static int n = [] {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
      hipDeviceProp_t p;
      if (hipGetDeviceProperties(&p, dev) == hipSuccess) cus = p.multiProcessorCount;
    }
    return cus;
  }();
  return n;
}

}  // namespace ttlh
