// bfloat8_b tiles: host codec and device dequantisation.
//
// The reference fixes only the tile size, 32*32 + 64 = 1088 bytes
// (python/ttl/dtype_utils.py:174-175); the packing lives in un-vendored
// tt-metal.  This build's format (also documented in include/ttlhip.h):
//   one 32x32 tile = 64 exponent bytes, then 1024 element bytes;
//   faces f0..f3 = (rows 0-15, cols 0-15), (0-15, 16-31), (16-31, 0-15),
//   (16-31, 16-31); exponent byte 16*f + r is shared by the 16 elements of
//   face f, row r; element byte 64 + 256*f + 16*r + c holds sign (bit 7) and
//   magnitude m (bits 6..0) of face f, row r, col c;
//   value = (-1)^sign * m * 2^(e - 133), exactly (every such value is a
//   bfloat16, normal or subnormal, because m has at most 7 significant bits).
// Pack: e = largest biased fp32 exponent among the 16 values (0 when they are
// all zero / subnormal), m = round-half-even(|x| * 2^(133 - e)) saturated at
// 127.  Tiles are stored row-major over the tile grid of the matrix.

#include <algorithm>
#include <cmath>
#include <cstring>

#include "ttlh_common.h"

namespace ttlh {

// byte offset of element (r, c) inside a tile and of its exponent
__host__ __device__ inline int bfp8_elem_off(int r, int c) {
  const int f = ((r >> 4) << 1) | (c >> 4);
  return 64 + 256 * f + 16 * (r & 15) + (c & 15);
}
__host__ __device__ inline int bfp8_exp_off(int r, int c) {
  const int f = ((r >> 4) << 1) | (c >> 4);
  return 16 * f + (r & 15);
}

// exact bf16 bits of (-1)^s * m * 2^(e - 133)
inline uint16_t bfp8_decode_host(uint8_t e, uint8_t b) {
  const int m = b & 0x7f;
  const double v = std::ldexp(static_cast<double>(m), static_cast<int>(e) - 133);
  const float f = static_cast<float>(v);  // exact: m has <= 7 significant bits
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return static_cast<uint16_t>((u >> 16) | ((b & 0x80u) << 8));
}

}  // namespace ttlh

using namespace ttlh;

namespace {

bool finite_all(const float* p, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    if (!std::isfinite(p[i])) return false;
  return true;
}

// round-half-to-even of a non-negative double
double rne(double x) {
  const double f = std::floor(x);
  const double d = x - f;
  if (d > 0.5) return f + 1.0;
  if (d < 0.5) return f;
  return std::fmod(f, 2.0) == 0.0 ? f : f + 1.0;
}

}  // namespace

extern "C" int ttlh_bfp8_pack_host(const float* src, void* dst, int64_t rows, int64_t cols) {
  clear_error();
  TTLH_REQUIRE(src && dst, TTLH_EINVAL, "ttlh_bfp8_pack_host: null pointer");
  TTLH_REQUIRE(rows > 0 && cols > 0 && rows % 32 == 0 && cols % 32 == 0, TTLH_EINVAL,
               "ttlh_bfp8_pack_host: rows and cols must be positive multiples of 32");
  TTLH_REQUIRE(finite_all(src, rows * cols), TTLH_EINVAL,
               "ttlh_bfp8_pack_host: input holds inf or NaN (not representable in bfloat8_b)");
  uint8_t* out = static_cast<uint8_t*>(dst);
  const int64_t nt_c = cols / 32;
  for (int64_t tr = 0; tr < rows / 32; ++tr)
    for (int64_t tc = 0; tc < nt_c; ++tc) {
      uint8_t* tile = out + (tr * nt_c + tc) * TTLH_BFP8_TILE_BYTES;
      for (int r = 0; r < 32; ++r)
        for (int half = 0; half < 2; ++half) {
          const float* row = src + (tr * 32 + r) * cols + tc * 32 + half * 16;
          int e = 0;
          for (int c = 0; c < 16; ++c) {
            uint32_t u;
            std::memcpy(&u, &row[c], 4);
            e = std::max(e, static_cast<int>((u >> 23) & 0xff));
          }
          tile[bfp8_exp_off(r, half * 16)] = static_cast<uint8_t>(e);
          const double scale = std::ldexp(1.0, 133 - e);
          for (int c = 0; c < 16; ++c) {
            const double a = std::fabs(static_cast<double>(row[c])) * scale;
            const int m = static_cast<int>(std::min(127.0, rne(a)));
            const uint8_t sign = std::signbit(row[c]) ? 0x80 : 0x00;
            tile[bfp8_elem_off(r, half * 16 + c)] = static_cast<uint8_t>(sign | m);
          }
        }
    }
  return TTLH_OK;
}

extern "C" int ttlh_bfp8_unpack_host(const void* src, uint16_t* dst, int64_t rows, int64_t cols) {
  clear_error();
  TTLH_REQUIRE(src && dst, TTLH_EINVAL, "ttlh_bfp8_unpack_host: null pointer");
  TTLH_REQUIRE(rows > 0 && cols > 0 && rows % 32 == 0 && cols % 32 == 0, TTLH_EINVAL,
               "ttlh_bfp8_unpack_host: rows and cols must be positive multiples of 32");
  const uint8_t* in = static_cast<const uint8_t*>(src);
  const int64_t nt_c = cols / 32;
  for (int64_t tr = 0; tr < rows / 32; ++tr)
    for (int64_t tc = 0; tc < nt_c; ++tc) {
      const uint8_t* tile = in + (tr * nt_c + tc) * TTLH_BFP8_TILE_BYTES;
      for (int r = 0; r < 32; ++r)
        for (int c = 0; c < 32; ++c)
          dst[(tr * 32 + r) * cols + tc * 32 + c] =
              bfp8_decode_host(tile[bfp8_exp_off(r, c)], tile[bfp8_elem_off(r, c)]);
    }
  return TTLH_OK;
}

// ---------------------------------------------------------------------------
// device dequantisation (the same decode the bfp8-weight matmul runs in LDS
// staging, see bfp8_decode8 in ttlh_bfp8.h)

#include "ttlh_bfp8.h"

namespace {

// A workgroup takes up to kUnpackTiles consecutive tiles of one tile row:
// their packed bytes (one contiguous range) reach LDS in 16-byte loads, then
// each lane decodes 8-element chunks of whole output rows, so every store
// instruction of a wave writes two rows' 512 contiguous bytes (one wave per
// tile writing 64-byte pieces of 32 rows measured 36 us at 4096 x 11008,
// 3.8 TB/s; this 25 us, 5.4 TB/s, with the same output bits).  The stores
// are temporal: alone the kernel runs 25% faster with non-temporal ones, but
// the GEMM that reads the output next then misses the Infinity Cache (the
// C4 step, unpack + GEMM, 327 us temporal against 337 non-temporal and 332
// with one wave per tile, alternating on one box).
constexpr int kUnpackTiles = 8;

__global__ __launch_bounds__(256) void bfp8_unpack_kernel(const uint8_t* __restrict__ q,
                                                          uint16_t* __restrict__ out,
                                                          int64_t cols, int64_t nt_c,
                                                          int64_t groups_per_row) {
  constexpr int kW = TTLH_BFP8_TILE_BYTES / 16;  // 16-byte words per tile
  __shared__ __attribute__((aligned(16))) uint8_t lds[kUnpackTiles * TTLH_BFP8_TILE_BYTES];
  const int64_t g = blockIdx.x;
  const int64_t tr = g / groups_per_row;
  const int64_t tc0 = (g - tr * groups_per_row) * kUnpackTiles;
  const int nt = static_cast<int>(min(static_cast<int64_t>(kUnpackTiles), nt_c - tc0));
  const u32x4* src = reinterpret_cast<const u32x4*>(q + (tr * nt_c + tc0) * TTLH_BFP8_TILE_BYTES);
#pragma unroll
  for (int i0 = 0; i0 < kUnpackTiles * kW; i0 += 256) {
    const int i = i0 + static_cast<int>(threadIdx.x);
    if (i < nt * kW) *reinterpret_cast<u32x4*>(lds + 16 * i) = src[i];
  }
  __syncthreads();
  // chunk i of the group: row i / 32, tile (i % 32) / 4, columns 8 (i % 4)
  uint16_t* const orow = out + tr * 32 * cols + tc0 * 32;
#pragma unroll
  for (int i0 = 0; i0 < 32 * 4 * kUnpackTiles; i0 += 256) {
    const int i = i0 + static_cast<int>(threadIdx.x);
    const int r = i >> 5, c = i & 31;
    const int t = c >> 2, col = (c & 3) * 8;
    if (t >= nt) continue;  // a short last group of the tile row
    const int f = ((r >> 4) << 1) | (col >> 4);
    const uint8_t* tb = lds + t * TTLH_BFP8_TILE_BYTES;
    const uint8_t e = tb[16 * f + (r & 15)];
    const uint64_t m =
        *reinterpret_cast<const uint64_t*>(tb + 64 + 256 * f + 16 * (r & 15) + (col & 15));
    *reinterpret_cast<u32x4*>(orow + r * cols + c * 8) = bfp8_decode8(m, e);
  }
}

}  // namespace

extern "C" int ttlh_bfp8_unpack(const void* src, void* dst_bf16, int64_t rows, int64_t cols,
                                void* stream) {
  clear_error();
  TTLH_REQUIRE(src && dst_bf16, TTLH_EINVAL, "ttlh_bfp8_unpack: null pointer");
  TTLH_REQUIRE(rows > 0 && cols > 0 && rows % 32 == 0 && cols % 32 == 0, TTLH_EINVAL,
               "ttlh_bfp8_unpack: rows and cols must be positive multiples of 32");
  TTLH_REQUIRE((reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(dst_bf16) & 15) == 0,
               TTLH_EINVAL, "ttlh_bfp8_unpack: src and dst must be 16-byte aligned");
  const int64_t nt_c = cols / 32;
  const int64_t groups_per_row = (nt_c + kUnpackTiles - 1) / kUnpackTiles;
  const int64_t blocks = (rows / 32) * groups_per_row;
  TTLH_REQUIRE(blocks < (int64_t(1) << 31), TTLH_EUNSUPPORTED, "ttlh_bfp8_unpack: too large");
  hipLaunchKernelGGL(bfp8_unpack_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(src),
                     static_cast<uint16_t*>(dst_bf16), cols, nt_c, groups_per_row);
  return check_launch("bfp8_unpack_kernel");
}

// ---------------------------------------------------------------------------
// bfloat4_b (format in include/ttlhip.h): the same face / shared-exponent
// structure with 4-bit sign-magnitude elements, two per byte.

namespace {

int bfp4_elem_byte(int r, int c) {
  const int f = ((r >> 4) << 1) | (c >> 4);
  return 64 + 128 * f + 8 * (r & 15) + ((c & 15) >> 1);
}

uint16_t bfp4_decode_host(uint8_t e, uint32_t n) {
  const double v = std::ldexp(static_cast<double>(n & 7u), static_cast<int>(e) - 129);
  const float f = static_cast<float>(v);  // exact: at most 3 significant bits
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return static_cast<uint16_t>((u >> 16) | ((n & 8u) << 12));
}

// The bfloat8_b unpack's layout (see bfp8_unpack_kernel): kUnpackTiles
// consecutive tiles of a tile row per workgroup, staged in LDS (in 8-byte
// loads: the tile array need only be 8-byte aligned, 576 = 72 x 8), then
// 8-element chunks of whole output rows, each from 4 nibble bytes and the
// face row's exponent.
__global__ __launch_bounds__(256) void bfp4_unpack_kernel(const uint8_t* __restrict__ q,
                                                          uint16_t* __restrict__ out,
                                                          int64_t cols, int64_t nt_c,
                                                          int64_t groups_per_row) {
  constexpr int kW = TTLH_BFP4_TILE_BYTES / 8;  // 8-byte words per tile
  __shared__ __attribute__((aligned(16))) uint8_t lds[kUnpackTiles * TTLH_BFP4_TILE_BYTES];
  const int64_t g = blockIdx.x;
  const int64_t tr = g / groups_per_row;
  const int64_t tc0 = (g - tr * groups_per_row) * kUnpackTiles;
  const int nt = static_cast<int>(min(static_cast<int64_t>(kUnpackTiles), nt_c - tc0));
  const uint64_t* src =
      reinterpret_cast<const uint64_t*>(q + (tr * nt_c + tc0) * TTLH_BFP4_TILE_BYTES);
#pragma unroll
  for (int i0 = 0; i0 < kUnpackTiles * kW; i0 += 256) {
    const int i = i0 + static_cast<int>(threadIdx.x);
    if (i < nt * kW) *reinterpret_cast<uint64_t*>(lds + 8 * i) = src[i];
  }
  __syncthreads();
  // chunk i of the group: row i / 32, tile (i % 32) / 4, columns 8 (i % 4)
  uint16_t* const orow = out + tr * 32 * cols + tc0 * 32;
#pragma unroll
  for (int i0 = 0; i0 < 32 * 4 * kUnpackTiles; i0 += 256) {
    const int i = i0 + static_cast<int>(threadIdx.x);
    const int r = i >> 5, c = i & 31;
    const int t = c >> 2, col = (c & 3) * 8;
    if (t >= nt) continue;  // a short last group of the tile row
    const int f = ((r >> 4) << 1) | (col >> 4);
    const uint8_t* tb = lds + t * TTLH_BFP4_TILE_BYTES;
    const int sh = static_cast<int>(tb[16 * f + (r & 15)]) - 129;
    const uint32_t nib =
        *reinterpret_cast<const uint32_t*>(tb + 64 + 128 * f + 8 * (r & 15) + (col & 15) / 2);
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t b = (nib >> (8 * k)) & 0xffu;
      w[k] = bfp4_decode1(b & 0xfu, sh) | (bfp4_decode1(b >> 4, sh) << 16);
    }
    *reinterpret_cast<u32x4*>(orow + r * cols + c * 8) = u32x4{w[0], w[1], w[2], w[3]};
  }
}

}  // namespace

extern "C" int ttlh_bfp4_pack_host(const float* src, void* dst, int64_t rows, int64_t cols) {
  clear_error();
  TTLH_REQUIRE(src && dst, TTLH_EINVAL, "ttlh_bfp4_pack_host: null pointer");
  TTLH_REQUIRE(rows > 0 && cols > 0 && rows % 32 == 0 && cols % 32 == 0, TTLH_EINVAL,
               "ttlh_bfp4_pack_host: rows and cols must be positive multiples of 32");
  TTLH_REQUIRE(finite_all(src, rows * cols), TTLH_EINVAL,
               "ttlh_bfp4_pack_host: input holds inf or NaN (not representable in bfloat4_b)");
  uint8_t* out = static_cast<uint8_t*>(dst);
  const int64_t nt_c = cols / 32;
  std::memset(out, 0, static_cast<size_t>((rows / 32) * nt_c * TTLH_BFP4_TILE_BYTES));
  for (int64_t tr = 0; tr < rows / 32; ++tr)
    for (int64_t tc = 0; tc < nt_c; ++tc) {
      uint8_t* tile = out + (tr * nt_c + tc) * TTLH_BFP4_TILE_BYTES;
      for (int r = 0; r < 32; ++r)
        for (int half = 0; half < 2; ++half) {
          const float* row = src + (tr * 32 + r) * cols + tc * 32 + half * 16;
          int e = 0;
          for (int c = 0; c < 16; ++c) {
            uint32_t u;
            std::memcpy(&u, &row[c], 4);
            e = std::max(e, static_cast<int>((u >> 23) & 0xff));
          }
          tile[bfp8_exp_off(r, half * 16)] = static_cast<uint8_t>(e);
          const double scale = std::ldexp(1.0, 129 - e);
          for (int c = 0; c < 16; ++c) {
            const double a = std::fabs(static_cast<double>(row[c])) * scale;
            const uint32_t m = static_cast<uint32_t>(std::min(7.0, rne(a)));
            const uint32_t nib = (std::signbit(row[c]) ? 8u : 0u) | m;
            const int cc = half * 16 + c;
            tile[bfp4_elem_byte(r, cc)] |= static_cast<uint8_t>(nib << (4 * (cc & 1)));
          }
        }
    }
  return TTLH_OK;
}

extern "C" int ttlh_bfp4_unpack_host(const void* src, uint16_t* dst, int64_t rows, int64_t cols) {
  clear_error();
  TTLH_REQUIRE(src && dst, TTLH_EINVAL, "ttlh_bfp4_unpack_host: null pointer");
  TTLH_REQUIRE(rows > 0 && cols > 0 && rows % 32 == 0 && cols % 32 == 0, TTLH_EINVAL,
               "ttlh_bfp4_unpack_host: rows and cols must be positive multiples of 32");
  const uint8_t* in = static_cast<const uint8_t*>(src);
  const int64_t nt_c = cols / 32;
  for (int64_t tr = 0; tr < rows / 32; ++tr)
    for (int64_t tc = 0; tc < nt_c; ++tc) {
      const uint8_t* tile = in + (tr * nt_c + tc) * TTLH_BFP4_TILE_BYTES;
      for (int r = 0; r < 32; ++r)
        for (int c = 0; c < 32; ++c) {
          const uint32_t nib = (tile[bfp4_elem_byte(r, c)] >> (4 * (c & 1))) & 0xfu;
          dst[(tr * 32 + r) * cols + tc * 32 + c] = bfp4_decode_host(tile[bfp8_exp_off(r, c)], nib);
        }
    }
  return TTLH_OK;
}

extern "C" int ttlh_bfp4_unpack(const void* src, void* dst_bf16, int64_t rows, int64_t cols,
                                void* stream) {
  clear_error();
  TTLH_REQUIRE(src && dst_bf16, TTLH_EINVAL, "ttlh_bfp4_unpack: null pointer");
  TTLH_REQUIRE(rows > 0 && cols > 0 && rows % 32 == 0 && cols % 32 == 0, TTLH_EINVAL,
               "ttlh_bfp4_unpack: rows and cols must be positive multiples of 32");
  TTLH_REQUIRE((reinterpret_cast<uintptr_t>(src) & 7) == 0 &&
                   (reinterpret_cast<uintptr_t>(dst_bf16) & 15) == 0,
               TTLH_EINVAL, "ttlh_bfp4_unpack: src must be 8-byte and dst 16-byte aligned");
  const int64_t nt_c = cols / 32;
  const int64_t groups_per_row = (nt_c + kUnpackTiles - 1) / kUnpackTiles;
  const int64_t blocks = (rows / 32) * groups_per_row;
  TTLH_REQUIRE(blocks < (int64_t(1) << 31), TTLH_EUNSUPPORTED, "ttlh_bfp4_unpack: too large");
  hipLaunchKernelGGL(bfp4_unpack_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(src),
                     static_cast<uint16_t*>(dst_bf16), cols, nt_c, groups_per_row);
  return check_launch("bfp4_unpack_kernel");
}

extern "C" int ttlh_matmul_bfp4w_ws(const void* A, int64_t lda, const void* Bq4, void* C,
                                    int64_t ldc, int64_t M, int64_t N, int64_t K,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  TTLH_REQUIRE(workspace, TTLH_EINVAL, "ttlh_matmul_bfp4w_ws: null workspace");
  TTLH_REQUIRE(K > 0 && N > 0 && workspace_bytes >= K * N * 2, TTLH_EINVAL,
               "ttlh_matmul_bfp4w_ws: workspace of %lld bytes is smaller than K*N*2 = %lld",
               (long long)workspace_bytes, (long long)(K > 0 && N > 0 ? K * N * 2 : 0));
  TTLH_REQUIRE(A && Bq4 && C, TTLH_EINVAL, "ttlh_matmul_bfp4w_ws: null pointer");
  TTLH_REQUIRE(M > 0 && M % 32 == 0 && N % 32 == 0 && K % 32 == 0, TTLH_EINVAL,
               "ttlh_matmul_bfp4w_ws: M, N, K must be positive multiples of 32");
  TTLH_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15) == 0, TTLH_EINVAL,
               "ttlh_matmul_bfp4w_ws: workspace must be 16-byte aligned");
  int st = ttlh_bfp4_unpack(Bq4, workspace, K, N, stream);
  if (st != TTLH_OK) return st;
  return ttlh_matmul(A, TTLH_BF16, lda, workspace, TTLH_BF16, N, C, TTLH_BF16, ldc, M, N, K, 0,
                     stream);
}
