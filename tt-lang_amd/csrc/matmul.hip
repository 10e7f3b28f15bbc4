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

#include "ttlh_bfp8.h"
#include "ttlh_common.h"

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
  a.grid_m = static_cast<int32_t>((M + BM - 1) / BM);
  a.grid_n = static_cast<int32_t>((N + BN - 1) / BN);
  hipLaunchKernelGGL(mm_bf16_kernel<true>, dim3(a.grid_m * a.grid_n), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("mm_bf16_kernel<bfp8>");
}
