// Row-major <-> tilized element order (ttlh_tilize / ttlh_untilize).
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
__global__ __launch_bounds__(256) void layout_kernel(const LayoutArgs a) {
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
    if (tilize) hipLaunchKernelGGL((layout_kernel<2, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((layout_kernel<2, false>), grid, block, 0, s, a);
  } else {
    if (tilize) hipLaunchKernelGGL((layout_kernel<4, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((layout_kernel<4, false>), grid, block, 0, s, a);
  }
  return check_launch("layout_kernel");
}

}  // namespace
}  // namespace ttlh

extern "C" int ttlh_tilize(const void* src, int64_t src_ld, void* dst, int64_t rows, int64_t cols,
                           int elem_bytes, void* stream) {
  return ttlh::run_layout("ttlh_tilize", true, src, dst, src_ld, rows, cols, elem_bytes, stream);
}

extern "C" int ttlh_untilize(const void* src, void* dst, int64_t dst_ld, int64_t rows,
                             int64_t cols, int elem_bytes, void* stream) {
  return ttlh::run_layout("ttlh_untilize", false, src, dst, dst_ld, rows, cols, elem_bytes,
                          stream);
}
