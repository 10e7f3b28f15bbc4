// Tile matmul for gfx950: C[M,N] (=|+=) A[M,K] . B[K,N], fp32 accumulation.
//
// What it replaces: the tile matmul of a TTL compute thread
// (Block.__matmul__ + store(acc=True), python/sim/block.py:805-868,1012-1013)
// and the Tensix loop that runs it, one 32x32 output tile per core with
// matmul_tiles into DST and a K-tile loop fed through circular buffers
// (examples/metal_examples/singlecore_matmul/metal/kernels/mm_compute.cpp:28-68,
// mm_reader.cpp:8-55; blocked variant bmm_large_block_zm.cpp:41-120).
//
// MI355X design (bf16):
//  - one workgroup computes a 128x128 output block (4x4 tiles of 32x32), four
//    waves in a 2x2 arrangement, each owning 64x64 = 2x2 MFMA tiles of
//    v_mfma_f32_32x32x16_bf16 with fp32 accumulators (64 per lane);
//  - K advances 64 at a time through a double-buffered LDS stage (the CB
//    ring analogue): A is stored as loaded (row-major, K contiguous); B is
//    transposed in registers (4x8 bf16 blocks) on its way into LDS so both
//    MFMA operands are one ds_read_b128 per lane; rows are padded to 72
//    elements (36 dwords) so the 32 rows an MFMA operand read touches fall
//    in distinct bank groups;
//  - the next K-step's global loads are issued before the current step's
//    MFMAs, and one barrier per K-step separates the LDS ping-pong;
//  - the workgroup -> output-block mapping is XCD-aware: consecutive
//    workgroup ids land on different XCDs (round-robin dispatch), so ids are
//    regrouped to give each XCD a compact band of output blocks whose A rows
//    and B columns stay in that XCD's L2;
//  - the epilogue rounds once to the output dtype (RNE).
// fp32 inputs take a simpler v_mfma_f32_32x32x2f32 kernel (64x64 blocks).

#include <atomic>
#include <type_traits>

#include "ttlh_bfp8.h"
#include "ttlh_common.h"
#include "ttlh_eltprog.h"

namespace ttlh {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef const __attribute__((address_space(1))) u32x4 gu32x4;

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDP = BK + 8;  // padded LDS row pitch (elements)
constexpr int kThreads = 256;

struct MmArgs {
  const uint16_t* A;
  const uint16_t* B;
  const uint8_t* Bq;       // bfloat8_b tiles of B (weight-quantised variant)
  int32_t bq_tiles_n;      // tiles per tile-row of Bq (N / 32)
  void* C;
  int64_t lda, ldb, ldc;
  int32_t M, N, K;
  int32_t c_dtype, accumulate;
  int32_t grid_m, grid_n;  // output blocks along M / N
};

// XCD-aware block order: MI355X dispatches workgroup i to XCD i % 8.  Regroup
// ids so XCD x gets the contiguous range [x * per, (x + 1) * per) of a
// row-band-major walk over output blocks (bands of 8 block-rows).
__device__ __forceinline__ void block_coords(const MmArgs& a, int& bm, int& bn) {
  const int nblk = a.grid_m * a.grid_n;
  int id = blockIdx.x;
  constexpr int kXcd = 8;
  if (nblk % kXcd == 0) {
    const int per = nblk / kXcd;
    id = (id % kXcd) * per + id / kXcd;
  }
  constexpr int kBand = 8;
  const int band_size = kBand * a.grid_n;
  const int band = id / band_size;
  const int in_band = id - band * band_size;
  const int rows = min(kBand, a.grid_m - band * kBand);
  bm = band * kBand + in_band % rows;
  bn = in_band / rows;
}

// Global -> register loads of one K-step.  A: 128 rows x 64 k = 1024 chunks
// of 8 bf16, 4 per thread.  B: 64 k x 128 n, each thread a 4 (k) x 8 (n)
// block as 4 chunks.  Out-of-range rows / columns / k read as zero.
struct Stage {
  u32x4 a[4];
  u32x4 b[4];
  uint64_t bq[4];  // bfloat8_b: 8 element bytes per k row (decoded in store_stage)
  uint32_t be[4];  // and their shared exponents
};

__device__ __forceinline__ u32x4 zero4() { return u32x4{0u, 0u, 0u, 0u}; }

template <bool BQ>
__device__ __forceinline__ void load_stage(const MmArgs& p, int bm, int bn, int k0, Stage& s) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = t + i * kThreads;  // chunk id 0..1023
    const int r = c >> 3;            // row within block
    const int kc = (c & 7) * 8;      // k offset within step
    const int gr = bm * BM + r, gk = k0 + kc;
    s.a[i] = (gr < p.M && gk < p.K)
                 ? *reinterpret_cast<gu32x4*>(reinterpret_cast<uintptr_t>(p.A + static_cast<int64_t>(gr) * p.lda + gk))
                 : zero4();
  }
  // lanes 16 apart share an n column group; the 16 lanes of a group take the
  // 16 k quads, so their 8-byte transposed LDS stores cover all 32 banks
  const int kq = (t & 15) * 4;  // 0..60
  const int n8 = (t >> 4) * 8;  // 0..120
  const int gn = bn * BN + n8;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int gk = k0 + kq + i;
    const bool ok = gk < p.K && gn < p.N;
    if constexpr (BQ) {
      // 8 consecutive columns of one k row sit in one half face row
      const int64_t tile = static_cast<int64_t>(gk >> 5) * p.bq_tiles_n + (gn >> 5);
      const uint8_t* t8 = p.Bq + tile * TTLH_BFP8_TILE_BYTES;
      const int r = gk & 31, c = gn & 31;
      const int f = ((r >> 4) << 1) | (c >> 4);
      s.bq[i] = ok ? *reinterpret_cast<const uint64_t*>(t8 + 64 + 256 * f + 16 * (r & 15) + (c & 15))
                   : 0ull;
      s.be[i] = ok ? t8[16 * f + (r & 15)] : 0u;
    } else {
      s.b[i] = ok ? *reinterpret_cast<gu32x4*>(reinterpret_cast<uintptr_t>(
                        p.B + static_cast<int64_t>(gk) * p.ldb + gn))
                  : zero4();
    }
  }
}

__device__ __forceinline__ uint32_t lo16(uint32_t w) { return w & 0xffffu; }
__device__ __forceinline__ uint32_t hi16(uint32_t w) { return w >> 16; }

// Register -> LDS.  A chunks go straight in; the 4x8 B block is transposed to
// 8 rows of Bt (n-major) with 4 consecutive k each (one 8-byte store per n).
template <bool BQ>
__device__ __forceinline__ void store_stage(Stage& s, uint16_t* As, uint16_t* Bts) {
  const int t = threadIdx.x;
  if constexpr (BQ) {  // dequantise the bfloat8_b rows to bf16 on their way into LDS
#pragma unroll
    for (int i = 0; i < 4; ++i) s.b[i] = bfp8_decode8(s.bq[i], static_cast<uint8_t>(s.be[i]));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = t + i * kThreads;
    const int r = c >> 3, kc = (c & 7) * 8;
    *reinterpret_cast<u32x4*>(As + r * LDP + kc) = s.a[i];
  }
  const int kq = (t & 15) * 4;
  const int n8 = (t >> 4) * 8;
  // b[i] = row k = kq + i, 8 values n8..n8+7 (2 per dword)
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int d = j >> 1;
    uint32_t e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = (j & 1) ? hi16(s.b[i][d]) : lo16(s.b[i][d]);
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = {e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
    *reinterpret_cast<u32x2*>(Bts + (n8 + j) * LDP + kq) = v;
  }
}

template <bool BQ>
__global__ __launch_bounds__(kThreads, 2) void mm_bf16_kernel(const MmArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][BM * LDP];  // [buf][A/Bt]
  int bm, bn;
  block_coords(p, bm, bn);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 64;  // wave's row offset in the block
  const int wn = (wave & 1) * 64;   // wave's col offset
  const int l32 = lane & 31;
  const int kg = (lane >> 5) * 8;   // this lane's k group inside an MFMA

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nk = (p.K + BK - 1) / BK;
  Stage st;
  load_stage<BQ>(p, bm, bn, 0, st);
  store_stage<BQ>(st, lds[0][0], lds[0][1]);
  __syncthreads();

  for (int ks = 0; ks < nk; ++ks) {
    const int cur = ks & 1;
    if (ks + 1 < nk) load_stage<BQ>(p, bm, bn, (ks + 1) * BK, st);
    const uint16_t* As = lds[cur][0];
    const uint16_t* Bts = lds[cur][1];
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      bf16x8 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const bf16x8*>(As + (wm + i * 32 + l32) * LDP + kk + kg);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const bf16x8*>(Bts + (wn + j * 32 + l32) * LDP + kk + kg);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (ks + 1 < nk) store_stage<BQ>(st, lds[cur ^ 1][0], lds[cur ^ 1][1]);
    __syncthreads();
  }

  // epilogue: lane holds column (l32) of each 32x32 tile, rows
  // 8*(r/4) + 4*(lane/32) + r%4 for accumulator r
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int gc = bn * BN + wn + j * 32 + l32;
      if (gc >= p.N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gr = bm * BM + wm + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (gr >= p.M) continue;
        const int64_t off = static_cast<int64_t>(gr) * p.ldc + gc;
        float v = acc[i][j][r];
        if (p.c_dtype == TTLH_BF16) {
          uint16_t* c = static_cast<uint16_t*>(p.C) + off;
          if (p.accumulate) v += bf16_to_f32(*c);
          *c = f32_to_bf16(v);
        } else {
          float* c = static_cast<float*>(p.C) + off;
          if (p.accumulate) v += *c;
          *c = v;
        }
      }
    }
}

// ---------------------------------------------------------------------------
// Large-problem kernel: 256x256 output block per workgroup, four waves each
// owning a 128x128 quadrant (4x4 MFMA tiles, 256 fp32 accumulators per lane,
// which the compiler places in the accumulation registers; one wave per
// SIMD).  A wave re-uses every A fragment 4 times and every B fragment 4
// times, which halves the LDS read traffic per MFMA of the 128x128 kernel:
// per 64-k step a CU reads 128 KB and writes 64 KB of LDS for 256 MFMAs.
// Staging per 64-k step: A = 256 rows x 64 k (8 chunks of 8 per thread,
// stored as loaded); B = 64 k x 256 n, each thread an 8 (k) x 8 (n) block
// transposed in registers (v_perm_b32) to 8 Bt rows of 8 k (one 16-byte LDS
// store each).  With one wave per SIMD nothing else hides a stall, so the
// steady-state 64-k step is a single basic block in which every LDS store,
// global load and transpose is interleaved between MFMAs, and the fragments
// of the next 16-k substep are read while the current substep's MFMAs run.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (N > 0) {
    static_for<N - 1>(f);
    f(std::integral_constant<int, N - 1>());
  }
}

// Writes one 32x32 accumulator tile at (r0, c0): the lane holds column
// c0 + lane % 32, rows r0 + 8 (r / 4) + 4 (lane / 32) + r % 4.
__device__ __forceinline__ void store_acc_tile(const MmArgs& p, const f32x16& t, int r0, int c0,
                                               int lane) {
  const int gc = c0 + (lane & 31);
  if (gc >= p.N) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int gr = r0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    if (gr >= p.M) continue;
    const int64_t off = static_cast<int64_t>(gr) * p.ldc + gc;
    float v = t[r];
    if (p.c_dtype == TTLH_BF16) {
      uint16_t* c = static_cast<uint16_t*>(p.C) + off;
      if (p.accumulate) v += bf16_to_f32(*c);
      *c = f32_to_bf16(v);
    } else {
      float* c = static_cast<float*>(p.C) + off;
      if (p.accumulate) v += *c;
      *c = v;
    }
  }
}

// Writes one 32x32 accumulator tile lying wholly inside C, two columns per
// store.  Lanes 2c and 2c + 1 hold columns 2c and 2c + 1 of the same 16
// rows; DPP swaps of each row pair give the even lane rows 8 (r / 4) +
// 4 (lane / 32) + r % 4 for even r and the odd lane those for odd r, both as
// (column 2c, column 2c + 1) pairs: 8 packed stores per lane instead of 16
// 2-byte ones.  Offsets are 32-bit (the launcher checks M * ldc < 2^31).
template <bool BF16OUT, bool ACC>
__device__ __forceinline__ void store_acc_tile_pairs(const MmArgs& p, const f32x16& t, int r0,
                                                     int c0, int lane) {
  const bool odd = lane & 1;
  const int col = c0 + ((lane & 31) & ~1);
  const int rbase = r0 + 4 * (lane >> 5) + (odd ? 1 : 0);
  static_for<8>([&](auto mm) {
    constexpr int m = decltype(mm)::value;
    // quad_perm [1, 0, 3, 2]: the neighbouring lane's value (selecting on
    // the DPP results, not on t's index, keeps t's elements in registers)
    const float e0 = t[2 * m], e1 = t[2 * m + 1];
    const float n0 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(e0), 0xB1, 0xF, 0xF, false));
    const float n1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(e1), 0xB1, 0xF, 0xF, false));
    const float lo = odd ? n1 : e0;  // column 2c
    const float hi = odd ? e1 : n0;  // column 2c + 1
    const int row = rbase + 8 * (m >> 1) + 2 * (m & 1);
    const uint32_t off = static_cast<uint32_t>(row) * static_cast<uint32_t>(p.ldc) +
                         static_cast<uint32_t>(col);
    if constexpr (BF16OUT) {
      uint32_t* c = reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p.C) + off);
      float a = lo, b = hi;
      if constexpr (ACC) {
        const uint32_t old = *c;
        a += __uint_as_float(old << 16);
        b += __uint_as_float(old & 0xffff0000u);
      }
      *c = cvt_pk_bf16x2(a, b);
    } else {
      typedef float f32x2 __attribute__((ext_vector_type(2)));
      f32x2* c = reinterpret_cast<f32x2*>(static_cast<float*>(p.C) + off);
      f32x2 v = {lo, hi};
      if constexpr (ACC) v += *c;
      *c = v;
    }
  });
}

constexpr int LM = 256, LN = 256, LK = 64, LP = LK + 8;

// Per-thread staging geometry of the 256x256 kernel.  A: chunks of 8 k at
// rows ar0 + 32 i (i < 8), k offset akc.  B: an 8 (k) x 8 (n) block at k rows
// kb + i, columns n8..n8+7.  Rows past M and columns past N are clamped to the
// last valid one: they only feed output rows / columns that are never stored.
struct Stage2 {
  u32x4 a[8];
  u32x4 b[8];
  uint64_t bq[8];  // bfloat8_b: 8 element bytes of each of the 8 k rows
  uint64_t be;     // and the 8 rows' shared exponents (consecutive bytes)
};

struct Geo2 {
  const uint16_t* a_row[8];  // A + row * lda + akc, per chunk
  int akc, kb, gn;           // gn: first staged column (clamped)
  int64_t b_col;             // bf16 B: element offset of (k = kb, column gn)
};

template <bool BQ>
__device__ __forceinline__ Geo2 make_geo2(const MmArgs& p, int bm, int bn) {
  const int t = threadIdx.x;
  Geo2 g;
  g.akc = (t & 7) * 8;
  g.kb = (t & 7) * 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = min(bm * LM + (t >> 3) + 32 * i, p.M - 1);
    g.a_row[i] = p.A + static_cast<int64_t>(row) * p.lda + g.akc;
  }
  g.gn = min(bn * LN + (t >> 3) * 8, p.N - 8);
  g.b_col = static_cast<int64_t>(g.kb) * p.ldb + g.gn;
  return g;
}

// FULL: the whole 64-k step lies inside K (no k bounds checks, no branches);
// otherwise k rows at or past K read as zero (K % 64 == 32 tail step).
template <bool BQ, bool FULL>
__device__ __forceinline__ void load_a2(const MmArgs& p, const Geo2& g, int k0, Stage2& s) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (FULL || k0 + g.akc < p.K)
      s.a[i] = *reinterpret_cast<gu32x4*>(reinterpret_cast<uintptr_t>(g.a_row[i] + k0));
    else
      s.a[i] = zero4();
  }
}

template <bool BQ, bool FULL>
__device__ __forceinline__ void load_b2(const MmArgs& p, const Geo2& g, int k0, Stage2& s) {
  if constexpr (BQ) {
    // the 8 k rows kb..kb+7 share a face (kb is a multiple of 8): their
    // exponents are 8 consecutive bytes and their element bytes 16 apart
    const int gk = k0 + g.kb;
    const int64_t tile = static_cast<int64_t>(gk >> 5) * p.bq_tiles_n + (g.gn >> 5);
    const uint8_t* t8 = p.Bq + tile * TTLH_BFP8_TILE_BYTES;
    const int r = gk & 31, c = g.gn & 31;
    const int f = ((r >> 4) << 1) | (c >> 4);
    const uint8_t* el = t8 + 64 + 256 * f + 16 * (r & 15) + (c & 15);
    if (FULL || gk < p.K) {
      s.be = *reinterpret_cast<const uint64_t*>(t8 + 16 * f + (r & 15));
#pragma unroll
      for (int i = 0; i < 8; ++i) s.bq[i] = *reinterpret_cast<const uint64_t*>(el + 16 * i);
    } else {
      s.be = 0ull;
#pragma unroll
      for (int i = 0; i < 8; ++i) s.bq[i] = 0ull;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (FULL || k0 + g.kb + i < p.K)
        s.b[i] = *reinterpret_cast<gu32x4*>(reinterpret_cast<uintptr_t>(
            p.B + g.b_col + static_cast<int64_t>(k0 + i) * p.ldb));
      else
        s.b[i] = zero4();
    }
  }
}

// lo16(x) | lo16(y) << 16 and hi16(x) | hi16(y) << 16
__device__ __forceinline__ uint32_t pack_lo(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x07060302u);
}

__device__ __forceinline__ void store_a2(const Stage2& s, uint16_t* As) {
  const int t = threadIdx.x;
  uint16_t* d = As + (t >> 3) * LP + (t & 7) * 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) *reinterpret_cast<u32x4*>(d + i * 32 * LP) = s.a[i];
}

// b[i] = k row kb + i, columns n8..n8+7 (dword d = columns 2d, 2d + 1);
// Bt row n8 + j receives the 8 k values of column j
template <bool BQ>
__device__ __forceinline__ void store_b2(Stage2& s, uint16_t* Bts) {
  const int t = threadIdx.x;
  if constexpr (BQ) {
#pragma unroll
    for (int i = 0; i < 8; ++i) s.b[i] = bfp8_decode8(s.bq[i], static_cast<uint8_t>(s.be >> (8 * i)));
  }
  uint16_t* d = Bts + ((t >> 3) * 8) * LP + (t & 7) * 8;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int w = j >> 1;
    u32x4 v;
    if (j & 1) {
      v.x = pack_hi(s.b[0][w], s.b[1][w]);
      v.y = pack_hi(s.b[2][w], s.b[3][w]);
      v.z = pack_hi(s.b[4][w], s.b[5][w]);
      v.w = pack_hi(s.b[6][w], s.b[7][w]);
    } else {
      v.x = pack_lo(s.b[0][w], s.b[1][w]);
      v.y = pack_lo(s.b[2][w], s.b[3][w]);
      v.z = pack_lo(s.b[4][w], s.b[5][w]);
      v.w = pack_lo(s.b[6][w], s.b[7][w]);
    }
    *reinterpret_cast<u32x4*>(d + j * LP) = v;
  }
}

__device__ __forceinline__ void block_coords2(const MmArgs& a, int& bm, int& bn) {
  const int nblk = a.grid_m * a.grid_n;
  int id = blockIdx.x;
  constexpr int kXcd = 8;
  if (nblk % kXcd == 0) {
    const int per = nblk / kXcd;
    id = (id % kXcd) * per + id / kXcd;
  }
  constexpr int kBand = 4;
  const int band_size = kBand * a.grid_n;
  const int band = id / band_size;
  const int in_band = id - band * band_size;
  const int rows = min(kBand, a.grid_m - band * kBand);
  bm = band * kBand + in_band % rows;
  bn = in_band / rows;
}

struct Frags {
  bf16x8 a[4], b[4];
};

__device__ __forceinline__ void read_frags(const uint16_t* As, const uint16_t* Bts, int fa_off,
                                           int fb_off, int kk, Frags& f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f.a[i] = *reinterpret_cast<const bf16x8*>(As + fa_off + i * 32 * LP + kk);
    f.b[i] = *reinterpret_cast<const bf16x8*>(Bts + fb_off + i * 32 * LP + kk);
  }
}

__device__ __forceinline__ void mfma16(const Frags& f, f32x16 (&acc)[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
}

// scheduling-group masks (LLVM AMDGPU): MFMA, VALU, VMEM read, DS read, DS write
constexpr int kSgMfma = 0x008, kSgValu = 0x002, kSgVmemRd = 0x020, kSgDsRd = 0x100,
              kSgDsWr = 0x200;
#define TTLH_SG(mask, n) __builtin_amdgcn_sched_group_barrier((mask), (n), 0)

// Single-instruction pieces of a 64-k step, so a substep can be written as
// an explicit sequence: MFMA, then the memory / transpose work that issues
// while it executes.
__device__ __forceinline__ void mfma_one(const Frags& f, f32x16 (&acc)[4][4], int q) {
  acc[q >> 2][q & 3] =
      __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[q >> 2], f.b[q & 3], acc[q >> 2][q & 3], 0, 0, 0);
}
__device__ __forceinline__ void read_one(const uint16_t* As, const uint16_t* Bts, int fa_off,
                                         int fb_off, int kk, Frags& f, int q) {
  if (q < 4) f.a[q] = *reinterpret_cast<const bf16x8*>(As + fa_off + q * 32 * LP + kk);
  else f.b[q - 4] = *reinterpret_cast<const bf16x8*>(Bts + fb_off + (q - 4) * 32 * LP + kk);
}
__device__ __forceinline__ void store_a_one(const Stage2& s, uint16_t* As, int i) {
  const int t = threadIdx.x;
  *reinterpret_cast<u32x4*>(As + (t >> 3) * LP + (t & 7) * 8 + i * 32 * LP) = s.a[i];
}
// Bt row n8 + j <- the 8 k values of staged column j (b[i] = k row kb + i)
__device__ __forceinline__ void store_b_one(const Stage2& s, uint16_t* Bts, int j) {
  const int t = threadIdx.x;
  const int w = j >> 1;
  u32x4 v;
  if (j & 1) {
    v.x = pack_hi(s.b[0][w], s.b[1][w]);
    v.y = pack_hi(s.b[2][w], s.b[3][w]);
    v.z = pack_hi(s.b[4][w], s.b[5][w]);
    v.w = pack_hi(s.b[6][w], s.b[7][w]);
  } else {
    v.x = pack_lo(s.b[0][w], s.b[1][w]);
    v.y = pack_lo(s.b[2][w], s.b[3][w]);
    v.z = pack_lo(s.b[4][w], s.b[5][w]);
    v.w = pack_lo(s.b[6][w], s.b[7][w]);
  }
  *reinterpret_cast<u32x4*>(Bts + ((t >> 3) * 8 + j) * LP + (t & 7) * 8) = v;
}
__device__ __forceinline__ void load_a_one(const Geo2& g, int k0, Stage2& s, int i) {
  s.a[i] = *reinterpret_cast<gu32x4*>(reinterpret_cast<uintptr_t>(g.a_row[i] + k0));
}
template <bool BQ>
__device__ __forceinline__ void load_b_one(const MmArgs& p, const Geo2& g, int k0, Stage2& s,
                                           int i) {
  if constexpr (BQ) {
    const int gk = k0 + g.kb;
    const int64_t tile = static_cast<int64_t>(gk >> 5) * p.bq_tiles_n + (g.gn >> 5);
    const uint8_t* t8 = p.Bq + tile * TTLH_BFP8_TILE_BYTES;
    const int r = gk & 31, c = g.gn & 31;
    const int f = ((r >> 4) << 1) | (c >> 4);
    if (i == 0) s.be = *reinterpret_cast<const uint64_t*>(t8 + 16 * f + (r & 15));
    s.bq[i] = *reinterpret_cast<const uint64_t*>(t8 + 64 + 256 * f + 16 * (r & 15) + (c & 15) + 16 * i);
  } else {
    s.b[i] = *reinterpret_cast<gu32x4*>(reinterpret_cast<uintptr_t>(
        p.B + g.b_col + static_cast<int64_t>(k0 + i) * p.ldb));
  }
}

#define TTLH_FENCE() __builtin_amdgcn_sched_barrier(0)

// One 64-k step in four 16-k substeps.  Buffer X (= ks & 1) holds step ks,
// whose substep-0 fragments are already in f0; Y (the other) receives step
// ks + 1 from the staging registers, which then fetch step ks + 2.
//   s0: MFMAs(f0) | read X s1 fragments, store A -> Y, load A of step ks + 2
//       (bfloat8_b: dequantise B)
//   s1: MFMAs(f1) | read X s2 fragments, transpose + store B -> Y, load B of
//       step ks + 2
//   barrier (Y complete)
//   s2: MFMAs(f0) | read X s3 fragments
//   s3: MFMAs(f1) | read Y s0 fragments of step ks + 1
//   barrier (X no longer read: step ks + 1 may overwrite it)
// With one wave per SIMD nothing else hides a stall, so the STEADY form
// (steps ks + 1 and ks + 2 exist and are full: one basic block) is written as
// an explicit instruction sequence, fenced against reordering, with the
// memory and transpose work after each MFMA, where it issues while the MFMA
// executes.  Edge steps run the same work without the interleave.
template <bool BQ, bool STEADY>
__device__ __forceinline__ void k_step(const MmArgs& p, const Geo2& g, uint16_t* lds, int ks,
                                       int nk, int nfull, int fa_off, int fb_off, Frags& f0,
                                       f32x16 (&acc)[4][4], Stage2& st) {
  constexpr int kBuf = 2 * LM * LP;
  const uint16_t* As = lds + (ks & 1) * kBuf;
  const uint16_t* Bts = As + LM * LP;
  uint16_t* nA = lds + ((ks + 1) & 1) * kBuf;
  uint16_t* nB = nA + LM * LP;
  const int k2 = (ks + 2) * LK;
  Frags f1;
  if constexpr (STEADY) {
    // s0: A stores, each followed by the A load of step ks + 2 into the
    // same registers (a full step for that load to land); bfloat8_b: the B
    // dequantisation as well
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      mfma_one(f0, acc, q);
      if (q < 8) {
        read_one(As, Bts, fa_off, fb_off, 16, f1, q);
        store_a_one(st, nA, q);
        load_a_one(g, k2, st, q);
      } else if (BQ) {
        st.b[q - 8] = bfp8_decode8(st.bq[q - 8], static_cast<uint8_t>(st.be >> (8 * (q - 8))));
      }
      TTLH_FENCE();
    }
    // s1: B transposes and stores, then the B loads of step ks + 2
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      mfma_one(f1, acc, q);
      if (q < 8) {
        read_one(As, Bts, fa_off, fb_off, 32, f0, q);
        store_b_one(st, nB, q);
      } else {
        load_b_one<BQ>(p, g, k2, st, q - 8);
      }
      TTLH_FENCE();
    }
    __syncthreads();
    // s2
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      mfma_one(f0, acc, q);
      if (q < 8) read_one(As, Bts, fa_off, fb_off, 48, f1, q);
      TTLH_FENCE();
    }
    // s3
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      mfma_one(f1, acc, q);
      if (q < 8) read_one(nA, nB, fa_off, fb_off, 0, f0, q);
      TTLH_FENCE();
    }
    __syncthreads();
  } else {
    const bool has1 = ks + 1 < nk;
    const bool has2 = ks + 2 < nk;
    read_frags(As, Bts, fa_off, fb_off, 16, f1);
    if (has1) {
      store_a2(st, nA);
      store_b2<BQ>(st, nB);
    }
    mfma16(f0, acc);
    read_frags(As, Bts, fa_off, fb_off, 32, f0);
    if (has2) {
      load_a2<BQ, false>(p, g, k2, st);
      load_b2<BQ, false>(p, g, k2, st);
    }
    mfma16(f1, acc);
    __syncthreads();
    read_frags(As, Bts, fa_off, fb_off, 48, f1);
    mfma16(f0, acc);
    if (has1) read_frags(nA, nB, fa_off, fb_off, 0, f0);
    mfma16(f1, acc);
    __syncthreads();
  }
}

template <bool BQ, bool OUT_BF16, bool ACC>
__global__ __launch_bounds__(kThreads, 1) void mm256_kernel(const MmArgs p) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds2[];  // [2][A | Bt][256 * LP]
  int bm, bn;
  block_coords2(p, bm, bn);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 128;
  const int wn = (wave & 1) * 128;
  const int fa_off = (wm + (lane & 31)) * LP + (lane >> 5) * 8;
  const int fb_off = (wn + (lane & 31)) * LP + (lane >> 5) * 8;

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const Geo2 g = make_geo2<BQ>(p, bm, bn);
  const int nfull = p.K / LK;
  const int nk = (p.K + LK - 1) / LK;
  Stage2 st;
  if (nfull > 0) {
    load_a2<BQ, true>(p, g, 0, st);
    load_b2<BQ, true>(p, g, 0, st);
  } else {
    load_a2<BQ, false>(p, g, 0, st);
    load_b2<BQ, false>(p, g, 0, st);
  }
  store_a2(st, lds2);
  store_b2<BQ>(st, lds2 + LM * LP);
  if (nk > 1) {
    if (nfull > 1) {
      load_a2<BQ, true>(p, g, LK, st);
      load_b2<BQ, true>(p, g, LK, st);
    } else {
      load_a2<BQ, false>(p, g, LK, st);
      load_b2<BQ, false>(p, g, LK, st);
    }
  }
  __syncthreads();
  Frags f0;
  read_frags(lds2, lds2 + LM * LP, fa_off, fb_off, 0, f0);

  int ks = 0;
  // (two steps per iteration: the second step's waits for its staged data
  // are then counted exactly instead of conservatively across the back edge)
  for (; ks + 3 < nfull; ks += 2) {
    k_step<BQ, true>(p, g, lds2, ks, nk, nfull, fa_off, fb_off, f0, acc, st);
    k_step<BQ, true>(p, g, lds2, ks + 1, nk, nfull, fa_off, fb_off, f0, acc, st);
  }
  for (; ks + 2 < nfull; ++ks) k_step<BQ, true>(p, g, lds2, ks, nk, nfull, fa_off, fb_off, f0, acc, st);
  for (; ks < nk; ++ks) k_step<BQ, false>(p, g, lds2, ks, nk, nfull, fa_off, fb_off, f0, acc, st);

  // (a compile-time loop: with a runtime (i, j) index the accumulators
  // would be kept in scratch memory)
  // M and N are multiples of 32, so every 32x32 tile is wholly inside C or
  // wholly outside it
  const int r0 = bm * LM + wm, c0 = bn * LN + wn;
  static_for<16>([&](auto ij) {
    constexpr int i = decltype(ij)::value / 4, j = decltype(ij)::value % 4;
    if (r0 + i * 32 < p.M && c0 + j * 32 < p.N)
      store_acc_tile_pairs<OUT_BF16, ACC>(p, acc[i][j], r0 + i * 32, c0 + j * 32, lane);
  });
}

constexpr size_t kLds256 = 2ull * 2 * LM * LP * sizeof(uint16_t);  // 147,456 bytes

template <bool BQ, bool OUT_BF16, bool ACC>
bool launch_mm256_as(const MmArgs& a, hipStream_t s, int* status) {
  // raise the kernel's dynamic LDS limit once per device
  static std::atomic<uint64_t> attr_set{0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev >= 64) return false;
  if (!(attr_set.load() & (uint64_t(1) << dev))) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&mm256_kernel<BQ, OUT_BF16, ACC>),
                            hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(kLds256)) != hipSuccess)
      return false;
    attr_set.fetch_or(uint64_t(1) << dev);
  }
  hipLaunchKernelGGL((mm256_kernel<BQ, OUT_BF16, ACC>), dim3(a.grid_m * a.grid_n), dim3(kThreads),
                     kLds256, s, a);
  *status = check_launch(BQ ? "mm256_kernel<bfp8>" : "mm256_kernel");
  return true;
}

// ---------------------------------------------------------------------------
// bf16 x bf16 large-problem kernel with a four-stage direct-to-LDS pipeline.
// Same 256x256 block / 128x128-per-wave MFMA tiling as mm256_kernel, but:
//  - operands reach LDS through global_load_lds_dwordx4 (lane l's 16 bytes
//    land at the wave's LDS base + 16 l): no staging registers, no LDS store
//    instructions;
//  - B stays row-major (k rows, n contiguous) in LDS and its MFMA operand
//    (8 consecutive k of one column) is read with ds_read_b64_tr_b16 (within
//    16 lanes, output lane i, element k = element i % 4 of the 8 bytes lane
//    4k + i / 4 addresses), so no register transposes;
//  - 32-k stages in four LDS buffers (4 x 32 KB): a stage's loads are issued
//    two and a half stages before its data is needed;
//  - rows are unpadded; 16-byte chunk c of A row r sits at chunk c ^ ((r >> 2) & 3)
//    and of B row r at c ^ (4 (r & 3)).  gfx950's LDS serves 256 bytes (64
//    banks) per cycle: a ds_read_b128 is conflict-free when each 16 lanes hit
//    16 distinct 16-byte bank groups, a ds_read_b64 when each 32 lanes do.
//    The A fragment reads (16 rows, one chunk) and the B transpose reads (4
//    rows x 4 chunks per 32 lanes) both meet that;
//  - one barrier per stage, between its two 16-k substeps: before it each
//    wave waits for its own loads of the next stage, after it the next
//    stage's first fragments are read and the stage four ahead is fetched
//    into the buffer just released.
// Every buffer is a separate LDS variable so the compiler can tell a load
// into one buffer from reads of another.
constexpr int DK = 32;  // k per stage

struct DmaGeo {
  const uint16_t* a_src[4];  // per A load: row (clamped to M - 1) and chunk, at k = 0
  const uint16_t* b_src[4];  // per B load: k row and chunk (column clamped), at k = 0
  int fa_off;                // A fragment byte offset of this lane (row, substep 0)
  int fa_off1;               // ... substep 1
  int fb[4];                 // B transpose-read byte offsets of the 4 n tiles
};

__device__ __forceinline__ DmaGeo make_dma_geo(const MmArgs& p, int bm, int bn, int wm, int wn,
                                               int lane) {
  DmaGeo g;
  const int t = threadIdx.x;
  const int wbase = (t & ~63);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int pos = i * kThreads + wbase + (t & 63);  // 16-byte position in the stage buffer
    // A: 4 chunks per 64-byte row
    const int ar = pos >> 2;
    const int alc = (pos & 3) ^ ((ar >> 2) & 3);
    const int grow = min(bm * LM + ar, p.M - 1);
    g.a_src[i] = p.A + static_cast<int64_t>(grow) * p.lda + alc * 8;
    // B: 32 chunks per 512-byte k row
    const int br = pos >> 5;
    const int blc = (pos & 31) ^ ((br & 3) << 2);
    const int gcol = min(bn * LN + blc * 8, p.N - 8);
    g.b_src[i] = p.B + static_cast<int64_t>(br) * p.ldb + gcol;
  }
  const int l32 = lane & 31, h = lane >> 5;
  const int xa = (l32 >> 2) & 3;
  const int arow = wm + l32;
  g.fa_off = arow * 64 + ((0 + h) ^ xa) * 16;
  g.fa_off1 = arow * 64 + ((2 + h) ^ xa) * 16;
  // B operand of n tile j, k rows kb.. (kb multiple of 4): lane addresses
  // row kb + (lane & 15) / 4, column wn + 32 j + 16 ((lane >> 4) & 1) + 4 (lane & 3),
  // i.e. chunk wn / 8 + 4 j + e stored at chunk wn / 8 + 4 (j ^ brow) + e
  const int brow = (lane & 15) >> 2;
  const int e = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const int base = brow * 512 + (wn / 8 + e) * 16 + 8 * (lane & 1);
#pragma unroll
  for (int j = 0; j < 4; ++j) g.fb[j] = base + 64 * (j ^ brow);
  return g;
}

typedef __attribute__((address_space(3))) void lds_void;
typedef short i16x4m __attribute__((ext_vector_type(4)));
typedef short i16x8m __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4m lds_i16x4m;

// DMA of stage k0 into (A, B) buffers
__device__ __forceinline__ void dma_stage(const MmArgs& p, const DmaGeo& g, int k0, uint16_t* Ab,
                                          uint16_t* Bb) {
  const int wbase = threadIdx.x & ~63;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    __builtin_amdgcn_global_load_lds(g.a_src[i] + k0, (lds_void*)(Ab + (i * kThreads + wbase) * 8), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(g.b_src[i] + static_cast<int64_t>(k0) * p.ldb,
                                     (lds_void*)(Bb + (i * kThreads + wbase) * 8), 16, 0, 0);
  }
}

struct DFrags {
  bf16x8 a[4], b[4];
};

// fragments of substep `sub` (0 or 1) of the stage in (Ab, Bb)
__device__ __forceinline__ void dma_read_frags(const uint16_t* Ab, const uint16_t* Bb,
                                               const DmaGeo& g, int sub, int lane, DFrags& f) {
  const char* ab = reinterpret_cast<const char*>(Ab);
  const char* bb = reinterpret_cast<const char*>(Bb);
  const int aoff = sub ? g.fa_off1 : g.fa_off;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    f.a[i] = *reinterpret_cast<const bf16x8*>(ab + aoff + i * 32 * 64);
  const int kb = 16 * sub + 8 * (lane >> 5);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int off = g.fb[j];
    const i16x4m lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4m*)(bb + off + kb * 512));
    const i16x4m hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4m*)(bb + off + (kb + 4) * 512));
    const i16x8m w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    f.b[j] = __builtin_bit_cast(bf16x8, w);
  }
}

__device__ __forceinline__ void dma_mfma16(const DFrags& f, f32x16 (&acc)[4][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
}

// Single-instruction pieces, for explicitly sequenced substeps.
// Fragment piece q of substep `sub`: q < 4 -> A fragment q (ds_read_b128);
// q >= 4 -> half (q & 1) of B fragment (q - 4) / 2 (a transpose read).
struct DFragParts {
  bf16x8 a[4];
  i16x4m b[8];
  __device__ __forceinline__ void to_frags(DFrags& f) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const i16x8m w = {b[2 * j][0], b[2 * j][1], b[2 * j][2], b[2 * j][3],
                        b[2 * j + 1][0], b[2 * j + 1][1], b[2 * j + 1][2], b[2 * j + 1][3]};
      f.b[j] = __builtin_bit_cast(bf16x8, w);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) f.a[i] = a[i];
  }
};

__device__ __forceinline__ void dma_read_piece(const uint16_t* Ab, const uint16_t* Bb,
                                               const DmaGeo& g, int sub, int lane, DFragParts& f,
                                               int q) {
  const char* ab = reinterpret_cast<const char*>(Ab);
  const char* bb = reinterpret_cast<const char*>(Bb);
  if (q < 4) {
    f.a[q] = *reinterpret_cast<const bf16x8*>(ab + (sub ? g.fa_off1 : g.fa_off) + q * 32 * 64);
  } else {
    const int j = (q - 4) >> 1, half = q & 1;
    const int kb = 16 * sub + 8 * (lane >> 5) + 4 * half;
    const int off = g.fb[j];
    f.b[q - 4] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4m*)(bb + off + kb * 512));
  }
}

// load i of the 8 (4 A, 4 B) that fetch stage k0 into (Ab, Bb)
__device__ __forceinline__ void dma_piece(const MmArgs& p, const DmaGeo& g, int k0, uint16_t* Ab,
                                          uint16_t* Bb, int i) {
  const int wbase = threadIdx.x & ~63;
  if (i < 4)
    __builtin_amdgcn_global_load_lds(g.a_src[i] + k0, (lds_void*)(Ab + (i * kThreads + wbase) * 8),
                                     16, 0, 0);
  else
    __builtin_amdgcn_global_load_lds(g.b_src[i - 4] + static_cast<int64_t>(k0) * p.ldb,
                                     (lds_void*)(Bb + ((i - 4) * kThreads + wbase) * 8), 16, 0, 0);
}

__device__ __forceinline__ void dma_mfma_one(const DFrags& f, f32x16 (&acc)[4][4], int q) {
  acc[q >> 2][q & 3] =
      __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[q >> 2], f.b[q & 3], acc[q >> 2][q & 3], 0, 0, 0);
}

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8): wait until at most n global loads are outstanding
constexpr int vmcnt_imm(int n) { return 0x0F70 | (n & 0xF) | ((n >> 4) << 14); }

// at most `stages` stages (8 loads per thread each) still in flight
__device__ __forceinline__ void wait_stages(int stages) {
  if (stages >= 3) __builtin_amdgcn_s_waitcnt(vmcnt_imm(24));
  else if (stages == 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(16));
  else if (stages == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(8));
  else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
}

// the four stage buffers, each its own LDS variable (see above)
__shared__ __attribute__((aligned(16))) uint16_t dmaA0[LM * DK], dmaA1[LM * DK], dmaA2[LM * DK],
    dmaA3[LM * DK];
__shared__ __attribute__((aligned(16))) uint16_t dmaB0[DK * LN], dmaB1[DK * LN], dmaB2[DK * LN],
    dmaB3[DK * LN];

template <int Q>
__device__ __forceinline__ uint16_t* dma_abuf() {
  if constexpr (Q == 0) return dmaA0;
  else if constexpr (Q == 1) return dmaA1;
  else if constexpr (Q == 2) return dmaA2;
  else return dmaA3;
}
template <int Q>
__device__ __forceinline__ uint16_t* dma_bbuf() {
  if constexpr (Q == 0) return dmaB0;
  else if constexpr (Q == 1) return dmaB1;
  else if constexpr (Q == 2) return dmaB2;
  else return dmaB3;
}

// Barrier without a memory fence: the waits it needs are explicit (LDS reads
// done, this thread's loads of the next stage landed), so the loads of later
// stages stay in flight across it.
__device__ __forceinline__ void stage_barrier() { __builtin_amdgcn_s_barrier(); }

// The main loop of the DMA kernel for block (bm, bn): acc = this wave's
// 128x128 quadrant (rows bm * 256 + wm, columns bn * 256 + wn) of A . B.
__device__ __forceinline__ void dma_gemm_main(const MmArgs& p, int bm, int bn, int wm, int wn,
                                              int lane, f32x16 (&acc)[4][4]) {
  const DmaGeo g = make_dma_geo(p, bm, bn, wm, wn, lane);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nk = p.K / DK;
  // prologue: stages 0..3 in flight, stage 0 visible, its substep-0 fragments
  dma_stage(p, g, 0, dma_abuf<0>(), dma_bbuf<0>());
  if (1 < nk) dma_stage(p, g, DK, dma_abuf<1>(), dma_bbuf<1>());
  if (2 < nk) dma_stage(p, g, 2 * DK, dma_abuf<2>(), dma_bbuf<2>());
  if (3 < nk) dma_stage(p, g, 3 * DK, dma_abuf<3>(), dma_bbuf<3>());
  wait_stages(min(nk - 1, 3));  // stage 0 landed; stages 1..3 may be in flight
  stage_barrier();
  DFrags f0, f1;
  dma_read_frags(dma_abuf<0>(), dma_bbuf<0>(), g, 0, lane, f0);

  // STEADY: stages s + 1 .. s + 4 exist (fixed waits, no branches)
  auto stage = [&](auto qq, auto steady, int s) {
    constexpr int q = decltype(qq)::value;  // buffer of stage s
    constexpr bool STEADY = decltype(steady)::value;
    uint16_t* Ab = dma_abuf<q>();
    uint16_t* Bb = dma_bbuf<q>();
    uint16_t* An = dma_abuf<(q + 1) & 3>();
    uint16_t* Bn = dma_bbuf<(q + 1) & 3>();
    if constexpr (STEADY) {
      // substep 0: one MFMA on f0, then one piece of this stage's substep-1
      // fragments, fenced so the order holds
      DFragParts parts;
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        dma_mfma_one(f0, acc, x);
        if (x < 12) dma_read_piece(Ab, Bb, g, 1, lane, parts, x);
        __builtin_amdgcn_sched_barrier(0);
      }
      parts.to_frags(f1);
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of the buffer done
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(16));  // own loads of stage s + 1 landed
      stage_barrier();
      // substep 1: one MFMA on f1, then a piece of the next stage's substep-0
      // fragments, and after every second MFMA one load of stage s + 4 into
      // the buffer just released: the eight loads spread over the substep
      // (issued back to back they reach the texture path at twice the rate it
      // drains and stall the wave; spread, the workgroup takes 8% fewer cycles
      // per tile, though at the power cap the clock gives part of it back)
      DFragParts nparts;
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        dma_mfma_one(f1, acc, x);
        if (x < 12) dma_read_piece(An, Bn, g, 0, lane, nparts, x);
        if (x & 1) dma_piece(p, g, (s + 4) * DK, Ab, Bb, x >> 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      nparts.to_frags(f0);
    } else {
      // substep 0: MFMAs on f0, read this stage's substep-1 fragments
      dma_read_frags(Ab, Bb, g, 1, lane, f1);
      dma_mfma16(f0, acc);
      __builtin_amdgcn_sched_barrier(0);
      // this wave's LDS reads are done (the buffer may be refilled after the
      // barrier) and its loads of stage s + 1 landed (later stages may still
      // be in flight)
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      if (s + 1 < nk) wait_stages(min(nk - 2 - s, 2));
      stage_barrier();
      // substep 1: MFMAs on f1, read the next stage's substep-0 fragments and
      // fetch stage s + 4 into the buffer this stage no longer reads
      if (s + 1 < nk) dma_read_frags(An, Bn, g, 0, lane, f0);
      if (s + 4 < nk) dma_stage(p, g, (s + 4) * DK, Ab, Bb);
      dma_mfma16(f1, acc);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  int s = 0;
  for (; s + 8 <= nk; s += 4) {
    stage(I0(), std::true_type(), s);
    stage(I1(), std::true_type(), s + 1);
    stage(I2(), std::true_type(), s + 2);
    stage(I3(), std::true_type(), s + 3);
  }
  for (; s + 4 <= nk; s += 4) {
    stage(I0(), std::false_type(), s);
    stage(I1(), std::false_type(), s + 1);
    stage(I2(), std::false_type(), s + 2);
    stage(I3(), std::false_type(), s + 3);
  }
  if (s < nk) stage(I0(), std::false_type(), s);
  if (s + 1 < nk) stage(I1(), std::false_type(), s + 1);
  if (s + 2 < nk) stage(I2(), std::false_type(), s + 2);
}

// Column XOR of row r of a staged 64-row half quadrant (rows at a 256-byte
// pitch): the four rows one dword store instruction writes (r, r + 1, r + 4,
// r + 5) land in four different 64-byte bank groups, and a 16-byte chunk
// stays contiguous.
__device__ __forceinline__ int epi_swz(int r) { return ((r & 1) | ((r >> 1) & 2)) << 5; }

// One 32x32 accumulator tile, rounded to bf16, into a staged half quadrant
// (rows r0 + 0..31, columns c0 + 0..31): lane pairs swap halves so each lane
// writes one dword of two adjacent columns.
__device__ __forceinline__ void epi_tile_to_lds(const f32x16& t, uint16_t* half, int r0, int c0,
                                                int lane) {
  const bool odd = lane & 1;
  const int col = c0 + ((lane & 31) & ~1);
  const int rbase = r0 + 4 * (lane >> 5) + (odd ? 1 : 0);
  static_for<8>([&](auto mm) {
    constexpr int m = decltype(mm)::value;
    const float e0 = t[2 * m], e1 = t[2 * m + 1];
    const float n0 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(e0), 0xB1, 0xF, 0xF, false));
    const float n1 = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(e1), 0xB1, 0xF, 0xF, false));
    const float lo = odd ? n1 : e0;  // column 2c
    const float hi = odd ? e1 : n0;  // column 2c + 1
    const int row = rbase + 8 * (m >> 1) + 2 * (m & 1);
    *reinterpret_cast<uint32_t*>(half + row * 128 + (col ^ epi_swz(row))) = cvt_pk_bf16x2(lo, hi);
  });
}

// The 8 staged elements of the quadrant's row `row` (0-127) from column c8.
__device__ __forceinline__ u32x4 epi_staged(const uint16_t* top, const uint16_t* bot, int row,
                                            int c8) {
  const int r = row & 63;
  return *reinterpret_cast<const u32x4*>((row < 64 ? top : bot) + r * 128 + (c8 ^ epi_swz(r)));
}

// The wave's 128x128 quadrant, rounded to bf16, into LDS (rows 0-63 in A
// stage buffer `wave`, 64-127 in B stage buffer `wave`: the main loop is done
// with them once every wave has passed the barrier); returns the two halves.
__device__ __forceinline__ void quadrant_to_lds(const f32x16 (&acc)[4][4], int wave, int lane,
                                                uint16_t*& top, uint16_t*& bot) {
  stage_barrier();  // every wave is done with the stage buffers
  top = wave == 0 ? dmaA0 : wave == 1 ? dmaA1 : wave == 2 ? dmaA2 : dmaA3;
  bot = wave == 0 ? dmaB0 : wave == 1 ? dmaB1 : wave == 2 ? dmaB2 : dmaB3;
  uint16_t* const t = top;
  uint16_t* const b = bot;
  static_for<16>([&](auto ij) {
    constexpr int i = decltype(ij)::value / 4, j = decltype(ij)::value % 4;
    epi_tile_to_lds(acc[i][j], i < 2 ? t : b, (i & 1) * 32, j * 32, lane);
  });
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the quadrant is in LDS
  asm volatile("" ::: "memory");       // (lanes read what other lanes wrote)
}

template <bool OUT_BF16, bool ACC>
__global__ __launch_bounds__(kThreads, 1) void mm_dma_kernel(const MmArgs p) {
  int bm, bn;
  block_coords2(p, bm, bn);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 128;
  const int wn = (wave & 1) * 128;
  f32x16 acc[4][4];
  dma_gemm_main(p, bm, bn, wm, wn, lane, acc);
  const int r0 = bm * LM + wm, c0 = bn * LN + wn;
  static_for<16>([&](auto ij) {
    constexpr int i = decltype(ij)::value / 4, j = decltype(ij)::value % 4;
    if (r0 + i * 32 < p.M && c0 + j * 32 < p.N)
      store_acc_tile_pairs<OUT_BF16, ACC>(p, acc[i][j], r0 + i * 32, c0 + j * 32, lane);
  });
}

// The DMA kernel with the elementwise program of the store fused into its
// epilogue: out = prog(round_bf16(A . B), operands...) over the GEMM's
// output, e.g. relu(a @ b + c).  The simulator materialises the product
// block in its dtype before the other ops read it (python/sim/block.py:
// 870-920), so the product is rounded to bf16 first; then the program runs
// with ttlh_eltwise's op definitions and per-step rounding, the product
// standing for the operand whose pointer is null.  The product never reaches
// HBM: quadrant_to_lds puts each wave's rounded quadrant in LDS and
// epi_groups walks it in chunks of 8 consecutive elements (the program's
// chunk shape) with the accumulators dead, so the program has the registers.
struct EpiArgs {
  EltArgs e;
  MmArgs p;
};


// element e (0..7) of eight bf16 values packed in q, as f32
__device__ __forceinline__ float bf16_elem(const u32x4 q, int e) {
  const uint32_t w = e < 2 ? q.x : e < 4 ? q.y : e < 6 ? q.z : q.w;
  return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
}

constexpr int kEpiG = 4;     // chunks per lane and group (8 groups per quadrant)
constexpr int kEpiProd = 3;  // Ins.arg of the step that reads the product
constexpr int kEpiSet = 0;   // pseudo-op of a K_SET step: the source value itself

// One group's operand bits: the 16-byte block holding each chunk's first
// element and that element's byte offset in it (used by broadcast operands).
struct EpiGroup {
  u32x4 q[3][kEpiG];
  uint32_t sel[3][kEpiG];
};

template <int NG>
__device__ __forceinline__ void epi_issue(const EltArgs& e, const MmArgs& p, int r0, int c0,
                                          int lane, int g0, EpiGroup& s) {
#pragma unroll
  for (int u = 0; u < kEpiG; ++u) {
    const int qi = (g0 + u) * 64 + lane, row = qi >> 4, c8 = (qi & 15) * 8;
    const int64_t y = e.y0 + min(r0 + row, p.M - 1), x = e.x0 + min(c0 + c8, p.N - 8);
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const uintptr_t a = operand_addr<true>(e.ops[j], y, x);
      s.q[j][u] = *reinterpret_cast<gu32x4*>(a & ~uintptr_t(15));
      s.sel[j][u] = static_cast<uint32_t>(a & 15u);
    }
  }
}

// a broadcast operand (one element per chunk): that element in all 8 slots
template <int NG>
__device__ __forceinline__ void epi_normalise(const EltArgs& e, EpiGroup& s) {
#pragma unroll
  for (int j = 0; j < NG; ++j) {
    if (e.ops[j].vec) continue;
#pragma unroll
    for (int u = 0; u < kEpiG; ++u) {
      const uint32_t d = pick_dword(s.q[j][u], s.sel[j][u]);
      const uint32_t h = (s.sel[j][u] & 2) ? (d >> 16) : (d & 0xffffu);
      const uint32_t w = h | (h << 16);
      s.q[j][u] = u32x4{w, w, w, w};
    }
  }
}

// acc = op(acc, src) (op(src, acc) for REV), in place, for the group
template <int OP, bool REV, class Src>
__device__ __forceinline__ void epi_apply(float (&acc)[kEpiG][8], Src src) {
#pragma unroll
  for (int u = 0; u < kEpiG; ++u) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float b = src(u, i);
      if constexpr (OP == kEpiSet) acc[u][i] = b;
      else acc[u][i] = REV ? binary1<OP>(b, acc[u][i]) : binary1<OP>(acc[u][i], b);
    }
  }
}

template <int OP, bool REV, int NG>
__device__ __forceinline__ void epi_bin_step(const Ins ins, float (&acc)[kEpiG][8],
                                             const u32x4 (&pr)[kEpiG], const EpiGroup& s) {
  if (ins.src == SRC_IMM) {
    const float c = ins.imm;
    epi_apply<OP, REV>(acc, [&](int, int) { return c; });
    return;
  }
  switch (ins.arg) {  // uniform: no dynamic register indexing
    case 0:
      if constexpr (NG > 0) epi_apply<OP, REV>(acc, [&](int u, int i) { return bf16_elem(s.q[0][u], i); });
      else __builtin_unreachable();  // the host numbers operands below NG
      break;
    case 1:
      if constexpr (NG > 1) epi_apply<OP, REV>(acc, [&](int u, int i) { return bf16_elem(s.q[1][u], i); });
      else __builtin_unreachable();  // the host numbers operands below NG
      break;
    case 2:
      if constexpr (NG > 2) epi_apply<OP, REV>(acc, [&](int u, int i) { return bf16_elem(s.q[2][u], i); });
      else __builtin_unreachable();  // the host numbers operands below NG
      break;
    default:  // kEpiProd
      epi_apply<OP, REV>(acc, [&](int u, int i) { return bf16_elem(pr[u], i); });
      break;
  }
}

template <int OP>
__device__ __forceinline__ void epi_un(float (&acc)[kEpiG][8]) {
  if constexpr (OP == TTLH_OP_EXP) {
    // the group's range check hoisted out of exp1, as vexp_uniform does
    bool ok = true;
#pragma unroll
    for (int u = 0; u < kEpiG; ++u) {
#pragma unroll
      for (int i = 0; i < 8; ++i) ok &= exp1_in_range(acc[u][i]);
    }
    if (__all(ok)) {
#pragma unroll
      for (int u = 0; u < kEpiG; ++u) {
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[u][i] = exp1_fast(acc[u][i]);
      }
      return;
    }
  }
#pragma unroll
  for (int u = 0; u < kEpiG; ++u) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[u][i] = unary1<OP>(acc[u][i]);
  }
}

template <bool REV, int NG>
__device__ __forceinline__ void epi_bin_op(const Ins ins, float (&acc)[kEpiG][8],
                                           const u32x4 (&pr)[kEpiG], const EpiGroup& s) {
  switch (ins.op) {
    case TTLH_OP_ADD: epi_bin_step<TTLH_OP_ADD, REV, NG>(ins, acc, pr, s); break;
    case TTLH_OP_SUB: epi_bin_step<TTLH_OP_SUB, REV, NG>(ins, acc, pr, s); break;
    case TTLH_OP_MUL: epi_bin_step<TTLH_OP_MUL, REV, NG>(ins, acc, pr, s); break;
    case TTLH_OP_DIV: epi_bin_step<TTLH_OP_DIV, REV, NG>(ins, acc, pr, s); break;
    case TTLH_OP_MAX: epi_bin_step<TTLH_OP_MAX, REV, NG>(ins, acc, pr, s); break;
    default: epi_bin_step<TTLH_OP_MIN, REV, NG>(ins, acc, pr, s); break;
  }
}

// One program step over a group.  Every branch is on the (uniform) step and
// is taken once per group; each (op, source) pair has its own straight-line
// arm that updates the accumulators in place, so no arm copies values into
// a shared temporary.
template <int NG>
__device__ __forceinline__ void epi_step(const Ins ins, float (&acc)[kEpiG][8],
                                         const u32x4 (&pr)[kEpiG], const EpiGroup& s) {
  if (ins.kind == K_UNARY) {
    switch (ins.op) {
      case TTLH_OP_EXP: epi_un<TTLH_OP_EXP>(acc); break;
      case TTLH_OP_SQRT: epi_un<TTLH_OP_SQRT>(acc); break;
      case TTLH_OP_RSQRT: epi_un<TTLH_OP_RSQRT>(acc); break;
      case TTLH_OP_ABS: epi_un<TTLH_OP_ABS>(acc); break;
      case TTLH_OP_NEG: epi_un<TTLH_OP_NEG>(acc); break;
      case TTLH_OP_RELU: epi_un<TTLH_OP_RELU>(acc); break;
      default: epi_un<TTLH_OP_RECIP>(acc); break;
    }
  } else if (ins.kind == K_SET) {
    epi_bin_step<kEpiSet, false, NG>(ins, acc, pr, s);
  } else if (ins.kind == K_BIN) {
    epi_bin_op<false, NG>(ins, acc, pr, s);
  } else {  // K_BIN_REV
    epi_bin_op<true, NG>(ins, acc, pr, s);
  }
  if (ins.rnd == TTLH_BF16) {  // round_bf16x8's rounding, element pairs
#pragma unroll
    for (int u = 0; u < kEpiG; ++u) {
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        const uint32_t w = cvt_pk_bf16x2(acc[u][i], acc[u][i + 1]);
        acc[u][i] = __uint_as_float(w << 16);
        acc[u][i + 1] = __uint_as_float(w & 0xffff0000u);
      }
    }
  }
}

// The program and the store for one group whose operand loads were issued.
template <int NG>
__device__ __forceinline__ void epi_finish(const EltArgs& e, const MmArgs& p, const uint16_t* top,
                                           const uint16_t* bot, int r0, int c0, int lane, int g0,
                                           EpiGroup& s) {
  u32x4 pr[kEpiG];
#pragma unroll
  for (int u = 0; u < kEpiG; ++u) {
    const int qi = (g0 + u) * 64 + lane, row = qi >> 4, c8 = (qi & 15) * 8;
    pr[u] = epi_staged(top, bot, row, c8);
  }
  epi_normalise<NG>(e, s);
  float acc[kEpiG][8];
  // each step's scalar load is issued a step ahead: with one wave per SIMD
  // nothing else would cover its latency
  Ins cur = e.prog[0];
  for (int k = 0; k < e.n_instr; ++k) {
    const Ins nxt = e.prog[min(k + 1, e.n_instr - 1)];
    epi_step<NG>(cur, acc, pr, s);
    cur = nxt;
  }
#pragma unroll
  for (int u = 0; u < kEpiG; ++u) {
    const int qi = (g0 + u) * 64 + lane, row = qi >> 4, c8 = (qi & 15) * 8;
    if (r0 + row < p.M && c0 + c8 < p.N) {
      u32x4 w;
      w.x = cvt_pk_bf16(acc[u][0], acc[u][1]);
      w.y = cvt_pk_bf16(acc[u][2], acc[u][3]);
      w.z = cvt_pk_bf16(acc[u][4], acc[u][5]);
      w.w = cvt_pk_bf16(acc[u][6], acc[u][7]);
      const int64_t y = e.y0 + r0 + row, x = e.x0 + c0 + c8;
      __builtin_nontemporal_store(
          w, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(e.out) + y * e.out_ld + x));
    }
  }
}

// The program over the wave's quadrant, kEpiG chunks per lane at a time:
// the next group's operand loads are in flight while a group is computed
// and stored.  NG (the number of operands other than the product) is a
// template argument, so every load sequence is straight-line code and the
// waits for a group's loads count exactly the memory operations issued
// after them (a load in a branch makes the compiler wait for everything,
// the previous group's stores included).
template <int NG>
__device__ __forceinline__ void epi_groups(const EltArgs& e, const MmArgs& p, const uint16_t* top,
                                           const uint16_t* bot, int r0, int c0, int lane,
                                           EpiGroup& s0) {
  EpiGroup s1;
  for (int g0 = 0; g0 < 32; g0 += 2 * kEpiG) {
    epi_issue<NG>(e, p, r0, c0, lane, g0 + kEpiG, s1);
    epi_finish<NG>(e, p, top, bot, r0, c0, lane, g0, s0);
    if (g0 + 2 * kEpiG < 32) epi_issue<NG>(e, p, r0, c0, lane, g0 + 2 * kEpiG, s0);
    epi_finish<NG>(e, p, top, bot, r0, c0, lane, g0 + kEpiG, s1);
  }
}

template <int NG>
__global__ __launch_bounds__(kThreads, 1) void mm_dma_epi_kernel(const EpiArgs args) {
  const MmArgs& p = args.p;
  int bm, bn;
  block_coords2(p, bm, bn);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 128;
  const int wn = (wave & 1) * 128;
  f32x16 acc[4][4];
  dma_gemm_main(p, bm, bn, wm, wn, lane, acc);
  const int r0 = bm * LM + wm, c0 = bn * LN + wn;
  EpiGroup s0;  // the first group's operand loads overlap the staging
  epi_issue<NG>(args.e, p, r0, c0, lane, 0, s0);
  uint16_t *top, *bot;
  quadrant_to_lds(acc, wave, lane, top, bot);
  epi_groups<NG>(args.e, p, top, bot, r0, c0, lane, s0);
}

template <bool OUT_BF16, bool ACC>
bool launch_mm_dma_as(const MmArgs& a, hipStream_t s, int* status) {
  hipLaunchKernelGGL((mm_dma_kernel<OUT_BF16, ACC>), dim3(a.grid_m * a.grid_n), dim3(kThreads), 0,
                     s, a);
  *status = check_launch("mm_dma_kernel");
  return true;
}

// ---------------------------------------------------------------------------
// bf16 x bfloat8_b with the weights dequantised in LDS ahead of the MFMAs.
// Tiling, A pipeline, fragment reads and MFMA sequence are mm_dma_kernel's
// (256x256 block, four waves of 128x128, 32-k stages, A in a ring of four
// LDS buffers by global_load_lds).  B arrives packed:
//  - the eight bfloat8_b tiles of a stage (tile row s of Bq, n tiles
//    8 bn .. 8 bn + 7) are one contiguous 8704-byte range in HBM; it reaches
//    a ring of LDS slots by global_load_lds: two 16-byte loads and one
//    4-byte load per thread (waves 2 and 3 repeat the 4-byte part of waves 0
//    and 1, so every wave issues the same number of loads);
//  - a decode pass turns a slot into its stage's bf16 B buffer (two buffers,
//    32 k rows x 256 n, row-major).  A thread decodes one face row (the 16
//    elements sharing an exponent) per substep: one 16-byte LDS read of the
//    element bytes and one of the exponent byte, per element
//    v_cvt_f32_ubyte + v_ldexp_f32 (exact) with the top half of the fp32
//    pattern and the sign bit packed by v_perm_b32 / v_and_or_b32, then two
//    16-byte LDS writes.  The work sits between the MFMAs like the fragment
//    reads and the loads;
//  - stage s + 1 is decoded over the window between the barriers of stages
//    s - 1 and s (first half of its face rows in the second substep of
//    s - 1, second half in the first substep of s): B buffer (s + 1) & 1 is
//    read by nobody then, and stage s + 1's fragments are read only after
//    stage s's barrier;
//  - 16-byte chunk c of B row r sits at c ^ 5 (r & 3), which keeps the
//    transpose reads (4 rows x 4 chunks per 32 lanes), the decode's writes
//    and its element reads (16 lanes = 4 tiles x 4 face rows) conflict-free;
//  - the packed ring has five slots; load group G(s) = {A(s + 4), Bq(s + 6)}
//    is issued in stage s's second substep (Bq(s + 6) into the slot Bq(s + 1)
//    was decoded from); before stage s's barrier a wave waits for G(s - 3)
//    (A(s + 1), Bq(s + 3)), so at most two groups (14 loads) stay in flight,
//    and a stage's packed bytes are visible two barriers before its decode
//    window closes, early enough to read each substep's bytes one substep
//    ahead.  Groups and decodes past
//    the last stage load / decode the last stage again (L2 hits, results
//    never read), so every stage runs the same code.
constexpr int kDqSlot = 8 * TTLH_BFP8_TILE_BYTES;  // 8704 bytes: one stage's packed tiles

constexpr int kDqSlots = 5;                          // ring of packed stages
__shared__ __attribute__((aligned(16))) uint8_t dqQ[kDqSlots * kDqSlot];
__shared__ __attribute__((aligned(16))) uint16_t dqB0[DK * LN], dqB1[DK * LN];

template <int Q>
__device__ __forceinline__ uint16_t* dq_bbuf() {
  if constexpr (Q == 0) return dqB0;
  else return dqB1;
}

struct DqGeo {
  uint32_t q_off;         // byte offset in Bq of 16-byte load 0 of stage 0 (+4096: load 1)
  uint32_t q_off2;        // ... of the 4-byte load
  uint32_t a_off[4];      // byte offsets in A of this thread's four A loads, at k = 0
  int64_t q_stage;        // bytes between stages (one tile row of Bq)
  int d_elem;             // decode: element bytes of this thread's face row (first half)
  int d_exp;              // ... its exponent byte
  int d_out;              // byte offset of its first output chunk in the B buffer
  int d_out1;             // ... of the second
};

// B operand offsets for the c ^ 5 (r & 3) chunk swizzle (the transpose-read
// lane pattern is mm_dma_kernel's: row kb + (lane & 15) / 4, chunk
// wn / 8 + 4 j + e)
__device__ __forceinline__ void dq_fb(DmaGeo& g, int wn, int lane) {
  const int brow = (lane & 15) >> 2;
  const int e = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    g.fb[j] = brow * 512 + (wn / 8 + ((4 * j + e) ^ (5 * brow))) * 16 + 8 * (lane & 1);
}

__device__ __forceinline__ DqGeo make_dq_geo(const MmArgs& p, int bn, int lane) {
  DqGeo d;
  const int t = threadIdx.x, w = t >> 6;
  const uint32_t base = static_cast<uint32_t>(bn) * 8 * TTLH_BFP8_TILE_BYTES;
  d.q_off = base + 16 * t;
  d.q_off2 = base + 8192 + 4 * ((w & 1) * 64 + lane);
  d.q_stage = static_cast<int64_t>(p.bq_tiles_n) * TTLH_BFP8_TILE_BYTES;
  // face row of the first half: tile nt = (lane >> 2) & 3, face f = lane >> 4,
  // row r = 4 w + (lane & 3); the second half is tile nt + 4
  const int nt = (lane >> 2) & 3, f = lane >> 4, r = 4 * w + (lane & 3);
  d.d_elem = nt * TTLH_BFP8_TILE_BYTES + 64 + 256 * f + 16 * r;
  d.d_exp = nt * TTLH_BFP8_TILE_BYTES + 16 * f + r;
  const int k = 16 * (f >> 1) + r, sw = 5 * (r & 3), c0 = 4 * nt + 2 * (f & 1);
  d.d_out = k * 512 + (c0 ^ sw) * 16;
  d.d_out1 = k * 512 + ((c0 + 1) ^ sw) * 16;
  return d;
}

// Direct-to-LDS loads written as inline asm, uniform 64-bit base in SGPRs
// plus a 32-bit lane offset (the launcher keeps A and Bq below 2 GiB).  A
// compiler-visible LDS DMA makes the compiler treat LDS reads as completing
// out of order and wait for all of them (lgkmcnt(0)) before the decode's
// first use of its own read, stalling on the fragment reads issued after
// it; this kernel waits for its DMA explicitly (vmcnt before each barrier).
// The uniform operands pass through readfirstlane; M0 = the wave's LDS
// destination, one wait state before the load.
__device__ __forceinline__ uint64_t dq_sbase(const void* base) {
  const uint64_t g = reinterpret_cast<uint64_t>(base);
  return (uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(g >> 32)))) << 32) |
         uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(g))));
}
__device__ __forceinline__ void dq_dma16(uint64_t sbase, uint32_t off, const void* lds) {
  const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)lds));
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2"
      :
      : "s"(__builtin_amdgcn_readfirstlane(m0)), "v"(off), "s"(sbase)
      : "memory", "m0");
}
__device__ __forceinline__ void dq_dma4(uint64_t sbase, uint32_t off, const void* lds) {
  const uint32_t m0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)lds));
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, %2"
      :
      : "s"(__builtin_amdgcn_readfirstlane(m0)), "v"(off), "s"(sbase)
      : "memory", "m0");
}

// stage x (clamped to the last) of Bq into the slot at byte `slot` of the
// ring: load i of 3
__device__ __forceinline__ void dq_qload(const MmArgs& p, const DqGeo& d, int x, int slot, int i) {
  const int wbase = threadIdx.x & ~63;
  const uint64_t sb = dq_sbase(p.Bq + static_cast<int64_t>(x) * d.q_stage);
  uint8_t* s = dqQ + slot;
  if (i < 2)
    dq_dma16(sb, d.q_off + 4096 * i, s + 16 * (i * kThreads + wbase));
  else
    dq_dma4(sb, d.q_off2, s + 8192 + 4 * (wbase & 64));
}

// one face row being decoded: element bytes, exponent, bf16 pairs
struct DqDec {
  u32x4 w;
  uint32_t e;
  int sh;
  uint32_t m[4];
  uint32_t o[8];
};

__device__ __forceinline__ void dq_read(int slot, const DqGeo& d, int half, DqDec& s) {
  const uint8_t* b = dqQ + slot;
  s.w = *reinterpret_cast<const u32x4*>(b + d.d_elem + half * 4 * TTLH_BFP8_TILE_BYTES);
  s.e = b[d.d_exp + half * 4 * TTLH_BFP8_TILE_BYTES];
}

// bf16 pair p (elements 2p, 2p + 1): value (-1)^s m 2^(e - 133), exact.
// Two pieces, so the work can be spread between MFMAs: the conversions
// (piece 0: v_cvt_f32_ubyte + v_ldexp_f32 of both elements, the magnitude
// mask on a dword's first pair, the shift on the first pair) and the packing
// (piece 1: the top halves and the sign bits).
__device__ __forceinline__ void dq_pair_cvt(DqDec& s, int p, float& f0, float& f1) {
  const int i = p >> 1, h = p & 1;
  if (p == 0) s.sh = static_cast<int>(s.e) - 133;
  if (h == 0) s.m[i] = s.w[i] & 0x7f7f7f7fu;
  // v_cvt_f32_ubyte{0..3} of the masked dword, one instruction per element
  // (written out: from the C++ shift-and-mask form the compiler extracts each
  // 7-bit field first, an extra instruction per element)
  float c0, c1;
  if (h == 0) {
    asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(c0) : "v"(s.m[i]));
    asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(c1) : "v"(s.m[i]));
  } else {
    asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(c0) : "v"(s.m[i]));
    asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(c1) : "v"(s.m[i]));
  }
  f0 = __builtin_amdgcn_ldexpf(c0, s.sh);
  f1 = __builtin_amdgcn_ldexpf(c1, s.sh);
}
__device__ __forceinline__ void dq_pair_pack(DqDec& s, int p, float f0, float f1) {
  const int i = p >> 1, h = p & 1;
  const uint32_t hi = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  const uint32_t sg = __builtin_amdgcn_perm(s.w[i], s.w[i], h ? 0x030C020Cu : 0x010C000Cu);
  s.o[p] = (sg & 0x80008000u) | hi;
}
__device__ __forceinline__ void dq_pair(DqDec& s, int p) {
  float f0, f1;
  dq_pair_cvt(s, p, f0, f1);
  dq_pair_pack(s, p, f0, f1);
}

__device__ __forceinline__ void dq_write(uint16_t* bbuf, const DqGeo& d, int half, int h,
                                         const DqDec& s) {
  char* b = reinterpret_cast<char*>(bbuf) + (h ? d.d_out1 : d.d_out) + half * 256;
  *reinterpret_cast<u32x4*>(b) = u32x4{s.o[4 * h], s.o[4 * h + 1], s.o[4 * h + 2], s.o[4 * h + 3]};
}

// whole decode of one half of a slot (prologue)
__device__ __forceinline__ void dq_decode_half(int slot, uint16_t* bbuf, const DqGeo& d, int half) {
  DqDec s;
  dq_read(slot, d, half, s);
#pragma unroll
  for (int p = 0; p < 8; ++p) dq_pair(s, p);
  dq_write(bbuf, d, half, 0, s);
  dq_write(bbuf, d, half, 1, s);
}

// Decode work placed after MFMA x of a substep, for a face row whose element
// and exponent bytes are already in registers (read at the end of the
// previous substep): piece 2p / 2p + 1 = conversions / packing of pair p (at
// most six VALU instructions per MFMA), the first 16-byte write after pair 3
// is packed, the second after pair 7.
__device__ __forceinline__ void dq_piece_ready(uint16_t* bbuf, const DqGeo& d, int half,
                                               DqDec& s, float (&f)[2], int x) {
  const int p = x >> 1;
  if ((x & 1) == 0) {
    if (x == 8) dq_write(bbuf, d, half, 0, s);
    dq_pair_cvt(s, p, f[0], f[1]);
  } else {
    dq_pair_pack(s, p, f[0], f[1]);
    if (x == 15) dq_write(bbuf, d, half, 1, s);
  }
}

template <bool OUT_BF16, bool ACC>
__global__ __launch_bounds__(kThreads, 1) void mm_dq_kernel(const MmArgs p) {
  int bm, bn;
  block_coords2(p, bm, bn);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 128;
  const int wn = (wave & 1) * 128;
  DmaGeo g = make_dma_geo(p, bm, bn, wm, wn, lane);  // A loads and A fragment offsets
  dq_fb(g, wn, lane);                                // B fragment offsets (5 (r & 3) swizzle)
  DqGeo d = make_dq_geo(p, bn, lane);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    d.a_off[i] = static_cast<uint32_t>(reinterpret_cast<const char*>(g.a_src[i]) -
                                       reinterpret_cast<const char*>(p.A));

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int nk = p.K / DK;  // a multiple of 4 (launcher)
  auto a_load = [&](auto qq, int x, int i) {  // stage x (clamped) of A into buffer Q: load i of 4
    constexpr int Q = decltype(qq)::value;
    const int wbase = threadIdx.x & ~63;
    dq_dma16(dq_sbase(p.A + min(x, nk - 1) * DK), d.a_off[i],
             dma_abuf<Q>() + (i * kThreads + wbase) * 8);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;

  // prologue: Bq(0), Bq(1), then groups G(-4) .. G(-2) = {A(0), Bq(2)},
  // {A(1), Bq(3)}, {A(2), Bq(4)}; slot of stage x = x % 5
  auto slot_of = [](int x) { return (x % kDqSlots) * kDqSlot; };
  for (int i = 0; i < 3; ++i) dq_qload(p, d, 0, slot_of(0), i);
  for (int i = 0; i < 3; ++i) dq_qload(p, d, min(1, nk - 1), slot_of(1), i);
  for (int i = 0; i < 4; ++i) a_load(I0(), 0, i);
  for (int i = 0; i < 3; ++i) dq_qload(p, d, min(2, nk - 1), slot_of(2), i);
  for (int i = 0; i < 4; ++i) a_load(I1(), 1, i);
  for (int i = 0; i < 3; ++i) dq_qload(p, d, min(3, nk - 1), slot_of(3), i);
  for (int i = 0; i < 4; ++i) a_load(I2(), 2, i);
  for (int i = 0; i < 3; ++i) dq_qload(p, d, min(4, nk - 1), slot_of(4), i);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(14));  // Bq(0), Bq(1), G(-4) landed
  stage_barrier();
  dq_decode_half(slot_of(0), dq_bbuf<0>(), d, 0);  // stage 0 whole, stage 1 first half
  dq_decode_half(slot_of(0), dq_bbuf<0>(), d, 1);
  dq_decode_half(slot_of(1), dq_bbuf<1>(), d, 0);
  DqDec dnext;  // bytes of the face row the next substep decodes
  dq_read(slot_of(1), d, 1, dnext);
  __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0): decode reads / writes done
  stage_barrier();
  // G(-1) = {A(3), Bq(5)}: slot 0 is free now
  for (int i = 0; i < 4; ++i) a_load(I3(), 3, i);
  for (int i = 0; i < 3; ++i) dq_qload(p, d, min(5, nk - 1), slot_of(5), i);
  DFrags f0, f1;
  dma_read_frags(dma_abuf<0>(), dq_bbuf<0>(), g, 0, lane, f0);

  // Stage s.  The bytes a substep decodes were read at the end of the
  // previous substep: the second half of stage s + 1's face rows (its slot
  // visible since stage s - 2's barrier) and the first half of stage s + 2's
  // (visible since stage s - 1's barrier: Bq(s + 2) is in G(s - 4), which
  // that barrier's wait covers).  Those two reads may stay in flight across
  // the barrier (lgkmcnt(2)); their slot is reloaded only after the next
  // barrier, by which every wave has consumed them.
  auto stage = [&](auto qq, int s) {
    constexpr int q = decltype(qq)::value;  // A buffer of stage s
    uint16_t* Ab = dma_abuf<q>();
    uint16_t* Bb = dq_bbuf<q & 1>();
    uint16_t* An = dma_abuf<(q + 1) & 3>();
    uint16_t* Bn = dq_bbuf<(q + 1) & 1>();
    const int slot2 = slot_of(s + 2);  // Bq(s + 2)
    // substep 0: MFMAs on f0; this stage's substep-1 fragments; second half
    // of stage s + 1's decode into B buffer (q + 1) & 1; at the end, the
    // bytes of stage s + 2's first half
    {
      DFragParts parts;
      float fv[2];
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        dma_mfma_one(f0, acc, x);
        if (x < 12) dma_read_piece(Ab, Bb, g, 1, lane, parts, x);
        dq_piece_ready(Bn, d, 1, dnext, fv, x);
        __builtin_amdgcn_sched_barrier(0);
      }
      dq_read(slot2, d, 0, dnext);
      __builtin_amdgcn_sched_barrier(0);
      parts.to_frags(f1);
    }
    __builtin_amdgcn_s_waitcnt(0xC27F);         // lgkmcnt(2): all but the two byte reads done
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(14));  // G(s - 3) landed: A(s + 1), Bq(s + 3)
    stage_barrier();
    // substep 1: MFMAs on f1; stage s + 1's substep-0 fragments; G(s) =
    // {A(s + 4) -> A buffer q, Bq(s + 6) -> the slot of Bq(s + 1)}; first
    // half of stage s + 2's decode into B buffer q & 1; at the end, the bytes
    // of stage s + 2's second half
    {
      DFragParts nparts;
      float fv[2];
      const int slot6 = slot_of(s + 6);
#pragma unroll
      for (int x = 0; x < 16; ++x) {
        dma_mfma_one(f1, acc, x);
        if (x < 12) dma_read_piece(An, Bn, g, 0, lane, nparts, x);
        if ((x & 1) && x < 8) a_load(qq, s + 4, x >> 1);
        if ((x & 1) && x >= 9) dq_qload(p, d, min(s + 6, nk - 1), slot6, (x - 9) >> 1);
        dq_piece_ready(Bb, d, 0, dnext, fv, x);
        __builtin_amdgcn_sched_barrier(0);
      }
      dq_read(slot2, d, 1, dnext);
      __builtin_amdgcn_sched_barrier(0);
      nparts.to_frags(f0);
    }
  };

  for (int s = 0; s < nk; s += 4) {
    stage(I0(), s);
    stage(I1(), s + 1);
    stage(I2(), s + 2);
    stage(I3(), s + 3);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // the last (unused) groups

  const int r0 = bm * LM + wm, c0 = bn * LN + wn;
  static_for<16>([&](auto ij) {
    constexpr int i = decltype(ij)::value / 4, j = decltype(ij)::value % 4;
    if (r0 + i * 32 < p.M)
      store_acc_tile_pairs<OUT_BF16, ACC>(p, acc[i][j], r0 + i * 32, c0 + j * 32, lane);
  });
}

// Launches the 256x256 kernel when the problem has enough 256x256 blocks to
// fill the chip; returns false otherwise.
template <bool BQ>
bool launch_mm256(MmArgs a, hipStream_t s, int* status) {
  const int gm = (a.M + LM - 1) / LM, gn = (a.N + LN - 1) / LN;
  if (static_cast<int64_t>(gm) * gn < 192) return false;
  if (static_cast<int64_t>(a.M) * a.ldc >= (int64_t(1) << 31)) return false;  // 32-bit C offsets
  a.grid_m = gm;
  a.grid_n = gn;
  if constexpr (BQ) {
    // weights dequantised in LDS: whole 256-column blocks of whole stage
    // quads, tiles 16-byte aligned
    if (a.N % LN == 0 && a.K % (4 * DK) == 0 && (reinterpret_cast<uintptr_t>(a.Bq) & 15) == 0 &&
        static_cast<int64_t>(a.M) * a.lda * 2 < (int64_t(1) << 31) &&
        static_cast<int64_t>(a.K / 32) * (a.N / 32) * TTLH_BFP8_TILE_BYTES < (int64_t(1) << 31)) {
      hipLaunchKernelGGL((mm_dq_kernel<true, false>), dim3(a.grid_m * a.grid_n), dim3(kThreads), 0,
                         s, a);
      *status = check_launch("mm_dq_kernel");
      return true;
    }
    return launch_mm256_as<true, true, false>(a, s, status);
  } else {
    if (a.c_dtype == TTLH_BF16)
      return a.accumulate ? launch_mm_dma_as<true, true>(a, s, status)
                          : launch_mm_dma_as<true, false>(a, s, status);
    return a.accumulate ? launch_mm_dma_as<false, true>(a, s, status)
                        : launch_mm_dma_as<false, false>(a, s, status);
  }
}

// ---------------------------------------------------------------------------
// fp32: 64x64 blocks, 4 waves (2x2) of 32x32 v_mfma_f32_32x32x2f32 tiles,
// BK = 32 through LDS (A row-major, B row-major; the f32 MFMA operands are
// single elements, read with ds_read_b32).
struct MmArgsF {
  const float* A;
  const float* B;
  void* C;
  int64_t lda, ldb, ldc;
  int32_t M, N, K;
  int32_t c_dtype, accumulate;
};

constexpr int FBM = 64, FBN = 64, FBK = 32;

__global__ __launch_bounds__(256) void mm_f32_kernel(const MmArgsF p) {
  __shared__ float As[FBM][FBK + 1];
  __shared__ float Bs[FBK][FBN + 1];
  const int bm = blockIdx.y, bn = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  for (int k0 = 0; k0 < p.K; k0 += FBK) {
#pragma unroll
    for (int i = 0; i < (FBM * FBK) / 256; ++i) {
      const int c = t + i * 256, r = c / FBK, k = c % FBK;
      const int gr = bm * FBM + r, gk = k0 + k;
      As[r][k] = (gr < p.M && gk < p.K) ? p.A[static_cast<int64_t>(gr) * p.lda + gk] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < (FBK * FBN) / 256; ++i) {
      const int c = t + i * 256, k = c / FBN, n = c % FBN;
      const int gk = k0 + k, gn = bn * FBN + n;
      Bs[k][n] = (gk < p.K && gn < p.N) ? p.B[static_cast<int64_t>(gk) * p.ldb + gn] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < FBK; kk += 2) {
      const float a = As[wm + (lane & 31)][kk + (lane >> 5)];
      const float b = Bs[kk + (lane >> 5)][wn + (lane & 31)];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
    }
    __syncthreads();
  }
  const int gc = bn * FBN + wn + (lane & 31);
  if (gc >= p.N) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int gr = bm * FBM + wm + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    if (gr >= p.M) continue;
    const int64_t off = static_cast<int64_t>(gr) * p.ldc + gc;
    float v = acc[r];
    if (p.c_dtype == TTLH_BF16) {
      uint16_t* c = static_cast<uint16_t*>(p.C) + off;
      if (p.accumulate) v += bf16_to_f32(*c);
      *c = f32_to_bf16(v);
    } else {
      float* c = static_cast<float*>(p.C) + off;
      if (p.accumulate) v += *c;
      *c = v;
    }
  }
}

}  // namespace
}  // namespace ttlh

using namespace ttlh;

extern "C" int ttlh_matmul(const void* A, int a_dtype, int64_t lda, const void* B, int b_dtype,
                           int64_t ldb, void* C, int c_dtype, int64_t ldc, int64_t M, int64_t N,
                           int64_t K, int accumulate, void* stream) {
  clear_error();
  TTLH_REQUIRE(A && B && C, TTLH_EINVAL, "ttlh_matmul: null pointer");
  TTLH_REQUIRE(M > 0 && N > 0 && K > 0 && M % 32 == 0 && N % 32 == 0 && K % 32 == 0, TTLH_EINVAL,
               "ttlh_matmul: M, N, K must be positive multiples of 32 (got %lld, %lld, %lld)",
               (long long)M, (long long)N, (long long)K);
  TTLH_REQUIRE(M < (1 << 30) && N < (1 << 30) && K < (1 << 30), TTLH_EUNSUPPORTED,
               "ttlh_matmul: dimension too large");
  TTLH_REQUIRE(lda >= K && ldb >= N && ldc >= N, TTLH_EINVAL, "ttlh_matmul: bad leading dims");
  TTLH_REQUIRE(c_dtype == TTLH_BF16 || c_dtype == TTLH_F32, TTLH_EINVAL,
               "ttlh_matmul: bad output dtype");
  TTLH_REQUIRE(a_dtype == b_dtype && (a_dtype == TTLH_BF16 || a_dtype == TTLH_F32),
               TTLH_EUNSUPPORTED, "ttlh_matmul: A and B must both be bf16 or both f32");
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (a_dtype == TTLH_BF16) {
    TTLH_REQUIRE((reinterpret_cast<uintptr_t>(A) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(B) & 15) == 0 && lda % 8 == 0 && ldb % 8 == 0,
                 TTLH_EUNSUPPORTED, "ttlh_matmul: bf16 operands need 16-byte aligned rows");
    MmArgs a = {};
    a.A = static_cast<const uint16_t*>(A);
    a.B = static_cast<const uint16_t*>(B);
    a.C = C;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.M = static_cast<int32_t>(M);
    a.N = static_cast<int32_t>(N);
    a.K = static_cast<int32_t>(K);
    a.c_dtype = c_dtype;
    a.accumulate = accumulate ? 1 : 0;
    int status = TTLH_OK;
    if (launch_mm256<false>(a, s, &status)) return status;
    a.grid_m = static_cast<int32_t>((M + BM - 1) / BM);
    a.grid_n = static_cast<int32_t>((N + BN - 1) / BN);
    hipLaunchKernelGGL(mm_bf16_kernel<false>, dim3(a.grid_m * a.grid_n), dim3(kThreads), 0, s, a);
    return check_launch("mm_bf16_kernel");
  }
  MmArgsF a;
  a.A = static_cast<const float*>(A);
  a.B = static_cast<const float*>(B);
  a.C = C;
  a.lda = lda;
  a.ldb = ldb;
  a.ldc = ldc;
  a.M = static_cast<int32_t>(M);
  a.N = static_cast<int32_t>(N);
  a.K = static_cast<int32_t>(K);
  a.c_dtype = c_dtype;
  a.accumulate = accumulate ? 1 : 0;
  dim3 grid(static_cast<unsigned>((N + FBN - 1) / FBN), static_cast<unsigned>((M + FBM - 1) / FBM));
  hipLaunchKernelGGL(mm_f32_kernel, grid, dim3(256), 0, s, a);
  return check_launch("mm_f32_kernel");
}

extern "C" int ttlh_matmul_eltwise(const void* A, int64_t lda, const void* B, int64_t ldb,
                                   int64_t M, int64_t N, int64_t K, const ttlh_instr* prog,
                                   const ttlh_operand* in, int n_instr, int prod_step, void* out,
                                   int out_dtype, int64_t out_ld, int64_t y0, int64_t x0,
                                   void* stream) {
  clear_error();
  TTLH_REQUIRE(A && B && out && prog && in, TTLH_EINVAL, "ttlh_matmul_eltwise: null pointer");
  TTLH_REQUIRE(M > 0 && N > 0 && K > 0 && M % 32 == 0 && N % 32 == 0 && K % 32 == 0, TTLH_EINVAL,
               "ttlh_matmul_eltwise: M, N, K must be positive multiples of 32 (got %lld, %lld, %lld)",
               (long long)M, (long long)N, (long long)K);
  TTLH_REQUIRE(M < (1 << 30) && N < (1 << 30) && K < (1 << 30), TTLH_EUNSUPPORTED,
               "ttlh_matmul_eltwise: dimension too large");
  TTLH_REQUIRE(lda >= K && ldb >= N && lda % 8 == 0 && ldb % 8 == 0 &&
                   (reinterpret_cast<uintptr_t>(A) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(B) & 15) == 0,
               TTLH_EINVAL, "ttlh_matmul_eltwise: A and B need 16-byte aligned rows");
  TTLH_REQUIRE(out_dtype == TTLH_BF16 || out_dtype == TTLH_F32, TTLH_EINVAL,
               "ttlh_matmul_eltwise: bad output dtype");
  TTLH_REQUIRE(out_dtype == TTLH_BF16, TTLH_EUNSUPPORTED,
               "ttlh_matmul_eltwise: the fused epilogue writes bf16 outputs only");
  TTLH_REQUIRE(y0 >= 0 && x0 >= 0 && x0 % 8 == 0 && out_ld >= x0 + N && out_ld % 8 == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0,
               TTLH_EINVAL, "ttlh_matmul_eltwise: bad output region or alignment");
  TTLH_REQUIRE(n_instr > 0 && n_instr <= TTLH_MAX_INSTR && prod_step >= 0 && prod_step < n_instr,
               TTLH_EINVAL, "ttlh_matmul_eltwise: bad product step %d", prod_step);
  const int pf = prog[prod_step].form;
  TTLH_REQUIRE(in[prod_step].ptr == nullptr &&
                   (pf == TTLH_FORM_LOAD || pf == TTLH_FORM_PUSH || pf == TTLH_FORM_BIN ||
                    pf == TTLH_FORM_BIN_REV),
               TTLH_EINVAL,
               "ttlh_matmul_eltwise: the product step must read an operand whose pointer is NULL");
  const int gm = static_cast<int>((M + LM - 1) / LM), gn = static_cast<int>((N + LN - 1) / LN);
  TTLH_REQUIRE(int64_t(gm) * gn >= 192 && (y0 + M) * out_ld < (int64_t(1) << 31), TTLH_EUNSUPPORTED,
               "ttlh_matmul_eltwise: the fused epilogue runs on the large-problem GEMM only "
               "(>= 192 blocks of 256x256, 32-bit output offsets)");
  // the product slot gets a stand-in operand for validation (the output at
  // the element itself), then a null pointer for the kernel
  ttlh_operand ops[TTLH_MAX_INSTR];
  for (int k = 0; k < n_instr; ++k) ops[k] = in[k];
  ops[prod_step] = ttlh_operand{out, out_dtype, 0, out_ld, 1, -1, -1, 0, 0};
  EltArgs e = {};
  ProgInfo pi;
  int st = decode_program("ttlh_matmul_eltwise", prog, ops, n_instr, y0, x0, M, N, e, pi);
  if (st != TTLH_OK) return st;
  TTLH_REQUIRE(pi.vec && pi.off32, TTLH_EUNSUPPORTED,
               "ttlh_matmul_eltwise: every operand must allow 8-wide chunks with 32-bit offsets");
  TTLH_REQUIRE(pi.n_ops <= 4 && pi.max_depth == 1 && pi.all_bf16, TTLH_EUNSUPPORTED,
               "ttlh_matmul_eltwise: the fused epilogue takes stack-free programs of at most 4 "
               "bf16 operand reads (the product included)");
  for (int k = 0; k < n_instr; ++k)
    TTLH_REQUIRE(is_inline_op(prog[k].form, prog[k].op), TTLH_EUNSUPPORTED,
                 "ttlh_matmul_eltwise: op %d is not available in the fused epilogue (+ - * / max "
                 "min exp sqrt rsqrt abs neg relu recip are)", prog[k].op);
  // the kernel's operand numbering: the other operands compacted to
  // 0 .. NG-1 in consumption order, the product as kEpiProd
  const EltArgs d = e;
  int ng = 0;
  for (int k = 0; k < n_instr; ++k) {
    if (e.prog[k].src != SRC_OPERAND) continue;
    if (k == prod_step) {
      e.prog[k].arg = kEpiProd;
    } else {
      e.ops[ng] = d.ops[d.prog[k].arg];
      e.prog[k].arg = static_cast<uint8_t>(ng++);
    }
  }
  e.n_ops = ng;
  e.out = out;
  e.out_ld = out_ld;
  e.out_dtype = out_dtype;
  MmArgs a = {};
  a.A = static_cast<const uint16_t*>(A);
  a.B = static_cast<const uint16_t*>(B);
  a.C = out;
  a.lda = lda;
  a.ldb = ldb;
  a.ldc = out_ld;
  a.M = static_cast<int32_t>(M);
  a.N = static_cast<int32_t>(N);
  a.K = static_cast<int32_t>(K);
  a.c_dtype = out_dtype;
  a.grid_m = gm;
  a.grid_n = gn;
  EpiArgs ea;
  ea.e = e;
  ea.p = a;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (ng) {
    case 0: hipLaunchKernelGGL(mm_dma_epi_kernel<0>, dim3(gm * gn), dim3(kThreads), 0, s, ea); break;
    case 1: hipLaunchKernelGGL(mm_dma_epi_kernel<1>, dim3(gm * gn), dim3(kThreads), 0, s, ea); break;
    case 2: hipLaunchKernelGGL(mm_dma_epi_kernel<2>, dim3(gm * gn), dim3(kThreads), 0, s, ea); break;
    default: hipLaunchKernelGGL(mm_dma_epi_kernel<3>, dim3(gm * gn), dim3(kThreads), 0, s, ea); break;
  }
  return check_launch("mm_dma_epi_kernel");
}

extern "C" int ttlh_matmul_bfp8w(const void* A, int64_t lda, const void* Bq, void* C, int64_t ldc,
                                 int64_t M, int64_t N, int64_t K, void* stream) {
  clear_error();
  TTLH_REQUIRE(A && Bq && C, TTLH_EINVAL, "ttlh_matmul_bfp8w: null pointer");
  TTLH_REQUIRE(M > 0 && N > 0 && K > 0 && M % 32 == 0 && N % 32 == 0 && K % 32 == 0, TTLH_EINVAL,
               "ttlh_matmul_bfp8w: M, N, K must be positive multiples of 32");
  TTLH_REQUIRE(M < (1 << 30) && N < (1 << 30) && K < (1 << 30), TTLH_EUNSUPPORTED,
               "ttlh_matmul_bfp8w: dimension too large");
  TTLH_REQUIRE(lda >= K && ldc >= N && lda % 8 == 0, TTLH_EINVAL,
               "ttlh_matmul_bfp8w: bad leading dims");
  TTLH_REQUIRE((reinterpret_cast<uintptr_t>(A) & 15) == 0 && (reinterpret_cast<uintptr_t>(Bq) & 7) == 0,
               TTLH_EINVAL, "ttlh_matmul_bfp8w: A must be 16-byte and Bq 8-byte aligned");
  MmArgs a = {};
  a.A = static_cast<const uint16_t*>(A);
  a.Bq = static_cast<const uint8_t*>(Bq);
  a.bq_tiles_n = static_cast<int32_t>(N / 32);
  a.C = C;
  a.lda = lda;
  a.ldb = N;
  a.ldc = ldc;
  a.M = static_cast<int32_t>(M);
  a.N = static_cast<int32_t>(N);
  a.K = static_cast<int32_t>(K);
  a.c_dtype = TTLH_BF16;
  a.accumulate = 0;
  int status = TTLH_OK;
  if (launch_mm256<true>(a, static_cast<hipStream_t>(stream), &status)) return status;
  a.grid_m = static_cast<int32_t>((M + BM - 1) / BM);
  a.grid_n = static_cast<int32_t>((N + BN - 1) / BN);
  hipLaunchKernelGGL(mm_bf16_kernel<true>, dim3(a.grid_m * a.grid_n), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("mm_bf16_kernel<bfp8>");
}

extern "C" int64_t ttlh_matmul_bfp8w_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  (void)M;
  return K > 0 && N > 0 ? K * N * 2 : 0;
}

extern "C" int ttlh_matmul_bfp8w_ws(const void* A, int64_t lda, const void* Bq, void* C,
                                    int64_t ldc, int64_t M, int64_t N, int64_t K,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  TTLH_REQUIRE(workspace, TTLH_EINVAL, "ttlh_matmul_bfp8w_ws: null workspace");
  TTLH_REQUIRE(K > 0 && N > 0 && workspace_bytes >= K * N * 2, TTLH_EINVAL,
               "ttlh_matmul_bfp8w_ws: workspace of %lld bytes is smaller than K*N*2 = %lld",
               (long long)workspace_bytes, (long long)(K > 0 && N > 0 ? K * N * 2 : 0));
  TTLH_REQUIRE(A && Bq && C, TTLH_EINVAL, "ttlh_matmul_bfp8w_ws: null pointer");
  TTLH_REQUIRE(M > 0 && M % 32 == 0 && N % 32 == 0 && K % 32 == 0, TTLH_EINVAL,
               "ttlh_matmul_bfp8w_ws: M, N, K must be positive multiples of 32");
  TTLH_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(Bq) & 15) == 0,
               TTLH_EINVAL, "ttlh_matmul_bfp8w_ws: Bq and the workspace must be 16-byte aligned");
  // pass 1: Bq tiles -> row-major bf16 [K, N] in the workspace (HBM bound);
  // pass 2: the bf16 GEMM.  The error text of a failing pass names it.
  int st = ttlh_bfp8_unpack(Bq, workspace, K, N, stream);
  if (st != TTLH_OK) return st;
  return ttlh_matmul(A, TTLH_BF16, lda, workspace, TTLH_BF16, N, C, TTLH_BF16, ldc, M, N, K, 0,
                     stream);
}
