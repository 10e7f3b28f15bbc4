// Row-major <-> tilized element order (ttlh_tilize / ttlh_untilize), and the
// bf16 transpose that stages a K^T operand as K for fused attention
// (ttlh_transpose_bf16).
//
// A tilized 2-D tensor (the TILE_LAYOUT storage of ttnn tensors the
// reference's compiled path requires, python/ttl/ttl_api.py:489-506) holds
// its 32x32 tiles row-major over the tile grid; each tile is four 16x16 faces
// (f0 rows 0-15 / cols 0-15, f1 rows 0-15 / cols 16-31, f2 rows 16-31 /
// cols 0-15, f3 rows 16-31 / cols 16-31), each face row-major.  The face
// split is the one the bfloat8_b / bfloat4_b tiles of this library use.
//
// A byte permutation, HBM-bound: every lane moves one 16-byte chunk (8 bf16
// or 4 f32 elements, always inside one face row) with a 16-byte load and a
// 16-byte store.  On the tilized side a wave's 64 chunks are 1 KB
// contiguous; on the row-major side every 16-byte chunk belongs to a 32-byte
// (bf16) or 64-byte (f32) run of a face row, and lanes of a wave cover whole
// 64-byte tile rows.

#include "ttlh_common.h"

namespace ttlh {
namespace {

// The kernel takes these as scalar arguments (layout.hip is built with
// kernarg preloading, so they are in SGPRs when a wave starts).
struct LayoutArgs {
  const char* src;
  char* dst;
  int64_t ld_bytes;       // row stride of the row-major side, bytes
  uint32_t tiles_per_row; // cols / 32
  uint32_t chunks;        // total 16-byte chunks
};

// Chunk k of the tilized buffer -> byte offset of the same 16 bytes on the
// row-major side.  E = element bytes (chunks per face row: 32 / (16 / E)).
template <int E>
__device__ __forceinline__ int64_t rowmajor_offset(const LayoutArgs& a, uint32_t k) {
  constexpr uint32_t kPerChunk = 16 / E;          // elements per chunk
  const uint32_t e = k * kPerChunk;               // element index in tilized order
  const uint32_t t = e >> 10, w = e & 1023u;      // tile, position in the tile
  const uint32_t f = w >> 8, r = (w >> 4) & 15u, c = w & 15u;
  const uint32_t tr = t / a.tiles_per_row, tc = t - tr * a.tiles_per_row;
  const int64_t row = int64_t(tr) * 32 + (f >> 1) * 16 + r;
  const int64_t col = int64_t(tc) * 32 + (f & 1u) * 16 + c;
  return row * a.ld_bytes + col * E;
}

template <int E, bool TILIZE>
__global__ __launch_bounds__(256) void layout_kernel(const char* src, char* dst, int64_t ld_bytes,
                                                     uint32_t tiles_per_row, uint32_t chunks) {
  const LayoutArgs a{src, dst, ld_bytes, tiles_per_row, chunks};
  const uint32_t k = blockIdx.x * 256u + threadIdx.x;
  if (k >= a.chunks) return;
  const int64_t rm = rowmajor_offset<E>(a, k);
  const int64_t tl = int64_t(k) * 16;
  const u32x4 v = *reinterpret_cast<const u32x4*>(a.src + (TILIZE ? rm : tl));
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(a.dst + (TILIZE ? tl : rm)));
}

int run_layout(const char* who, bool tilize, const void* src, void* dst, int64_t ld, int64_t rows,
               int64_t cols, int elem_bytes, void* stream) {
  clear_error();
  TTLH_REQUIRE(src && dst, TTLH_EINVAL, "%s: null pointer", who);
  TTLH_REQUIRE(elem_bytes == 2 || elem_bytes == 4, TTLH_EINVAL,
               "%s: elem_bytes must be 2 (bf16) or 4 (f32)", who);
  TTLH_REQUIRE(rows >= 0 && cols >= 0 && rows % 32 == 0 && cols % 32 == 0, TTLH_EINVAL,
               "%s: rows and cols must be multiples of 32 (got %lld x %lld)", who,
               (long long)rows, (long long)cols);
  TTLH_REQUIRE(ld >= cols, TTLH_EINVAL, "%s: row stride %lld below the %lld columns", who,
               (long long)ld, (long long)cols);
  TTLH_REQUIRE((reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(dst) & 15) == 0 && (ld * elem_bytes) % 16 == 0,
               TTLH_EINVAL, "%s: buffers and the row stride must be 16-byte aligned", who);
  const int64_t chunks = rows * cols * elem_bytes / 16;
  TTLH_REQUIRE(chunks < (int64_t(1) << 31) / 4, TTLH_EUNSUPPORTED, "%s: tensor too large", who);
  if (chunks == 0) return TTLH_OK;
  LayoutArgs a;
  a.src = static_cast<const char*>(src);
  a.dst = static_cast<char*>(dst);
  a.ld_bytes = ld * elem_bytes;
  a.tiles_per_row = static_cast<uint32_t>(cols / 32);
  a.chunks = static_cast<uint32_t>(chunks);
  const dim3 grid(static_cast<uint32_t>((chunks + 255) / 256)), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (elem_bytes == 2) {
    if (tilize) hipLaunchKernelGGL((layout_kernel<2, true>), grid, block, 0, s, a.src, a.dst, a.ld_bytes,
                                  a.tiles_per_row, a.chunks);
    else hipLaunchKernelGGL((layout_kernel<2, false>), grid, block, 0, s, a.src, a.dst, a.ld_bytes,
                                  a.tiles_per_row, a.chunks);
  } else {
    if (tilize) hipLaunchKernelGGL((layout_kernel<4, true>), grid, block, 0, s, a.src, a.dst, a.ld_bytes,
                                  a.tiles_per_row, a.chunks);
    else hipLaunchKernelGGL((layout_kernel<4, false>), grid, block, 0, s, a.src, a.dst, a.ld_bytes,
                                  a.tiles_per_row, a.chunks);
  }
  return check_launch("layout_kernel");
}

// Transpose of a bf16 matrix through LDS: a 256-thread workgroup moves one
// 64 x 64 tile.  Loads: 16-byte chunks along source rows (eight lanes cover
// one 128-byte row run).  Stores: each lane gathers eight source rows of one
// source column into one 16-byte chunk of a destination row.  The LDS row
// pitch of 66 elements (33 dwords) spreads those column reads over the banks.
constexpr int kTr = 64;
constexpr int kTrPitch = kTr + 2;

struct TransposeArgs {
  const uint16_t* src;
  uint16_t* dst;
  int64_t src_ld, dst_ld;   // row strides, elements
  int32_t rows, cols;       // of the source
};

__global__ __launch_bounds__(256) void transpose_bf16_kernel(TransposeArgs a) {
  __shared__ uint16_t t[kTr * kTrPitch];
  const int r0 = blockIdx.y * kTr, c0 = blockIdx.x * kTr;
  for (int i = threadIdx.x; i < kTr * kTr / 8; i += 256) {
    const int r = i >> 3, ch = i & 7;
    const int gr = r0 + r, gc = c0 + 8 * ch;
    if (gr < a.rows && gc < a.cols) {
      const uint4 v = *reinterpret_cast<const uint4*>(a.src + int64_t(gr) * a.src_ld + gc);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        t[r * kTrPitch + 8 * ch + 2 * e] = uint16_t(w[e] & 0xffffu);
        t[r * kTrPitch + 8 * ch + 2 * e + 1] = uint16_t(w[e] >> 16);
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < kTr * kTr / 8; i += 256) {
    const int c = i >> 3, ch = i & 7;           // destination row c0 + c
    const int gr = r0 + 8 * ch, gc = c0 + c;    // first source row of the chunk
    if (gr < a.rows && gc < a.cols) {
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = uint32_t(t[(8 * ch + 2 * e) * kTrPitch + c]) |
               (uint32_t(t[(8 * ch + 2 * e + 1) * kTrPitch + c]) << 16);
      *reinterpret_cast<uint4*>(a.dst + int64_t(gc) * a.dst_ld + gr) =
          uint4{w[0], w[1], w[2], w[3]};
    }
  }
}

}  // namespace
}  // namespace ttlh

extern "C" int ttlh_transpose_bf16(const void* src, int64_t src_ld, void* dst, int64_t dst_ld,
                                   int64_t rows, int64_t cols, void* stream) {
  using namespace ttlh;
  clear_error();
  TTLH_REQUIRE(src && dst, TTLH_EINVAL, "ttlh_transpose_bf16: null pointer");
  TTLH_REQUIRE(rows >= 0 && cols >= 0 && rows % 8 == 0 && cols % 8 == 0, TTLH_EINVAL,
               "ttlh_transpose_bf16: rows and cols must be multiples of 8 (got %lld x %lld)",
               (long long)rows, (long long)cols);
  TTLH_REQUIRE(src_ld >= cols && dst_ld >= rows && src_ld % 8 == 0 && dst_ld % 8 == 0,
               TTLH_EINVAL, "ttlh_transpose_bf16: row strides must cover the rows and be "
               "multiples of 8 elements");
  TTLH_REQUIRE((reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(dst) & 15) == 0,
               TTLH_EINVAL, "ttlh_transpose_bf16: buffers must be 16-byte aligned");
  TTLH_REQUIRE((rows + kTr - 1) / kTr <= 65535 && (cols + kTr - 1) / kTr <= (int64_t(1) << 24),
               TTLH_EUNSUPPORTED, "ttlh_transpose_bf16: matrix too large");
  const char* s0 = static_cast<const char*>(src);
  const char* d0 = static_cast<const char*>(dst);
  const int64_t sbytes = (rows ? (rows - 1) * src_ld + cols : 0) * 2;
  const int64_t dbytes = (cols ? (cols - 1) * dst_ld + rows : 0) * 2;
  TTLH_REQUIRE(d0 + dbytes <= s0 || s0 + sbytes <= d0, TTLH_EINVAL,
               "ttlh_transpose_bf16: source and destination overlap");
  if (rows == 0 || cols == 0) return TTLH_OK;
  TransposeArgs a;
  a.src = static_cast<const uint16_t*>(src);
  a.dst = static_cast<uint16_t*>(dst);
  a.src_ld = src_ld;
  a.dst_ld = dst_ld;
  a.rows = static_cast<int32_t>(rows);
  a.cols = static_cast<int32_t>(cols);
  const dim3 grid(static_cast<uint32_t>((cols + kTr - 1) / kTr),
                  static_cast<uint32_t>((rows + kTr - 1) / kTr));
  hipLaunchKernelGGL(transpose_bf16_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     a);
  return check_launch("transpose_bf16_kernel");
}

extern "C" int ttlh_tilize(const void* src, int64_t src_ld, void* dst, int64_t rows, int64_t cols,
                           int elem_bytes, void* stream) {
  return ttlh::run_layout("ttlh_tilize", true, src, dst, src_ld, rows, cols, elem_bytes, stream);
}

extern "C" int ttlh_untilize(const void* src, void* dst, int64_t dst_ld, int64_t rows,
                             int64_t cols, int elem_bytes, void* stream) {
  return ttlh::run_layout("ttlh_untilize", false, src, dst, dst_ld, rows, cols, elem_bytes,
                          stream);
}
