// Fused scaled-dot-product attention forward for gfx950:
//   O[b, h] = softmax(Q[b, h] K[b, h]^T * scale) V[b, h],  bf16 in / out,
//   fp32 scores and online softmax.
//
// The reference has no attention kernel; this composes the spec's tile ops
// (@, exp, reduce_max, reduce_sum, recip, broadcast:
// docs/sphinx/specs/TTLangSpecification.md:693-761) into one flash-style pass.
//
// MI355X design.  One workgroup = one (batch, head) and 128 query rows; four
// waves own 32 query rows each.  K/V stream through a double-buffered LDS
// stage 64 rows at a time (K row-major, V transposed on its way in).  Per KV
// block each wave computes
//     S^T = K Q^T   (16 x v_mfma_f32_32x32x16_bf16, Q^T operands kept in VGPRs)
//     O^T += V^T P^T (16 more MFMAs)
// Computing the transposes puts one query row in each lane's accumulator
// column for both products, so the softmax statistics (running max m and sum
// l) and the O rescale are per-lane scalars; the two lane halves that share a
// query combine with one xor-32 swizzle.  P goes from the S accumulators to
// the second MFMA without touching LDS: the accumulator layout hands each
// lane kv rows {16c + 4h + 8u + i}, so the V^T operand reads the same kv
// order (two 8-byte LDS reads), the contraction being invariant under a
// common permutation of kv.  exp is v_exp_f32 on pre-scaled log2-domain
// scores; P is rounded to bf16 for the MFMA; O is divided by l at the end.
// Workgroup ids are regrouped so the query blocks of one (batch, head) land
// on the same XCD and share K/V in its L2.

#include <cmath>

#include "ttlh_common.h"

namespace ttlh {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef const __attribute__((address_space(1))) u32x4 gu32x4;

constexpr int BQ = 128;   // query rows per workgroup
constexpr int BKV = 64;   // kv rows per stage
constexpr int kThreads = 256;

struct SdpaArgs {
  const uint16_t* Q;
  const uint16_t* K;
  const uint16_t* V;
  uint16_t* O;
  int32_t S;
  int32_t nqb;        // query blocks per (b, h)
  int32_t nbh;        // B * H
  float scale_log2;   // scale * log2(e)
};

__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(lo))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(hi))) << 16);
}

template <int D>
struct KvStage {
  u32x4 k[D / 32];  // K: 64 x D, D/32 chunks of 8 per thread
  u32x4 v[D / 32];  // V: 4 (kv) x 8 (d) block per thread for D = 128 (2 x 8 for D = 64)
};

template <int D>
__device__ __forceinline__ void load_kv(const SdpaArgs& p, int64_t base, int kv0, KvStage<D>& st) {
  const int t = threadIdx.x;
  constexpr int kChunksPerRow = D / 8;
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    const int c = t + i * kThreads;
    const int r = c / kChunksPerRow, dc = (c % kChunksPerRow) * 8;
    st.k[i] = *reinterpret_cast<gu32x4*>(
        reinterpret_cast<uintptr_t>(p.K + base + static_cast<int64_t>(kv0 + r) * D + dc));
  }
  // V: thread -> (kv group, d octet).  Consecutive lanes take consecutive kv
  // groups of one octet, so the transposed LDS stores of 16 lanes are one
  // contiguous 128-byte run (all 32 banks).
  constexpr int kOct = D / 8;
  constexpr int kRowsPerThread = BKV * kOct / kThreads;  // 4 for D = 128, 2 for D = 64
  constexpr int kGroups = BKV / kRowsPerThread;           // 16 for D = 128, 32 for D = 64
  const int quad = t % kGroups, oct = t / kGroups;
#pragma unroll
  for (int i = 0; i < kRowsPerThread; ++i) {
    const int r = quad * kRowsPerThread + i;
    st.v[i] = *reinterpret_cast<gu32x4*>(
        reinterpret_cast<uintptr_t>(p.V + base + static_cast<int64_t>(kv0 + r) * D + oct * 8));
  }
}

template <int D>
__device__ __forceinline__ void store_kv(const KvStage<D>& st, uint16_t* Ks, uint16_t* Vts) {
  constexpr int KP = D + 8, VP = BKV + 4;
  const int t = threadIdx.x;
  constexpr int kChunksPerRow = D / 8;
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    const int c = t + i * kThreads;
    const int r = c / kChunksPerRow, dc = (c % kChunksPerRow) * 8;
    *reinterpret_cast<u32x4*>(Ks + r * KP + dc) = st.k[i];
  }
  constexpr int kOct = D / 8;
  constexpr int kRowsPerThread = BKV * kOct / kThreads;
  constexpr int kGroups = BKV / kRowsPerThread;
  const int quad = t % kGroups, oct = t / kGroups;
  // transpose: rows kv = quad*R + i, cols d = oct*8 + j  ->  Vt[d][kv]
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int w = j >> 1;
    uint32_t e[kRowsPerThread];
#pragma unroll
    for (int i = 0; i < kRowsPerThread; ++i)
      e[i] = (j & 1) ? (st.v[i][w] >> 16) : (st.v[i][w] & 0xffffu);
    uint16_t* dst = Vts + (oct * 8 + j) * VP + quad * kRowsPerThread;
    if constexpr (kRowsPerThread == 4) {
      *reinterpret_cast<u32x2*>(dst) = u32x2{e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
    } else {
      *reinterpret_cast<uint32_t*>(dst) = e[0] | (e[1] << 16);
    }
  }
}

// the block's queries: q blocks of one (b, h) are kept on one XCD
__device__ __forceinline__ void block_coords(const SdpaArgs& p, int& bh, int& qb) {
  const int nblk = p.nbh * p.nqb;
  int id = blockIdx.x;
  constexpr int kXcd = 8;
  if (nblk % kXcd == 0) {
    const int per = nblk / kXcd;
    id = (id % kXcd) * per + id / kXcd;
  }
  bh = id / p.nqb;
  qb = id - bh * p.nqb;
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(kThreads, 2) void sdpa_fwd_kernel(const SdpaArgs p) {
  constexpr int KP = D + 8, VP = BKV + 4;
  constexpr int ND = D / 32;   // d tiles of O^T
  constexpr int NDC = D / 16;  // 16-wide d chunks of the S^T contraction
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BKV * KP];
  __shared__ __attribute__((aligned(16))) uint16_t Vts[2][D * VP];

  int bh, qb;
  block_coords(p, bh, qb);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t base = static_cast<int64_t>(bh) * p.S * D;
  const int q = qb * BQ + wave * 32 + l32;  // this lane's query row

  // Q^T operands (B of S^T = K Q^T): col = query, k = d
  bf16x8 qop[NDC];
#pragma unroll
  for (int dc = 0; dc < NDC; ++dc)
    qop[dc] = *reinterpret_cast<const bf16x8*>(p.Q + base + static_cast<int64_t>(q) * D +
                                               dc * 16 + 8 * h);

  f32x16 o[ND];
#pragma unroll
  for (int j = 0; j < ND; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[j][r] = 0.0f;
  float m = -INFINITY, l = 0.0f;

  const int nkv = CAUSAL ? (qb * BQ + BQ) / BKV : p.S / BKV;
  KvStage<D> st;
  load_kv<D>(p, base, 0, st);
  store_kv<D>(st, Ks[0], Vts[0]);
  __syncthreads();

  for (int kb = 0; kb < nkv; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < nkv) load_kv<D>(p, base, (kb + 1) * BKV, st);
    const uint16_t* K_ = Ks[cur];
    const uint16_t* Vt = Vts[cur];

    // S^T tiles: kv rows 32t.., query cols
    f32x16 s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[t][r] = 0.0f;
#pragma unroll
      for (int dc = 0; dc < NDC; ++dc) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(K_ + (32 * t + l32) * KP + dc * 16 + 8 * h);
        s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qop[dc], s[t], 0, 0, 0);
      }
    }
    // scale into the log2 domain, causal mask, block row max
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = s[t][r] * p.scale_log2;
        if constexpr (CAUSAL) {
          const int kv = kb * BKV + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
          if (kv > q) v = -INFINITY;
        }
        s[t][r] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx);
    const float alpha = __builtin_amdgcn_exp2f(m - m_new);  // 0 on the first block
    float rs = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = __builtin_amdgcn_exp2f(s[t][r] - m_new);
        s[t][r] = e;
        rs += e;
      }
    rs += __shfl_xor(rs, 32);
    l = l * alpha + rs;
    m = m_new;
#pragma unroll
    for (int j = 0; j < ND; ++j) o[j] *= alpha;

    // P^T operands: chunk c (16 kv) = tile c/2, accumulators 8(c%2) .. +8
    bf16x8 pb[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int t = c >> 1, r0 = 8 * (c & 1);
      u32x4 w;
      w.x = pk_bf16(s[t][r0 + 0], s[t][r0 + 1]);
      w.y = pk_bf16(s[t][r0 + 2], s[t][r0 + 3]);
      w.z = pk_bf16(s[t][r0 + 4], s[t][r0 + 5]);
      w.w = pk_bf16(s[t][r0 + 6], s[t][r0 + 7]);
      pb[c] = __builtin_bit_cast(bf16x8, w);
    }
    // O^T += V^T P^T; V^T operand rows d, kv order {16c + 4h + 8u + i}
#pragma unroll
    for (int j = 0; j < ND; ++j) {
      const uint16_t* vrow = Vt + (32 * j + l32) * VP;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow + 16 * c + 4 * h);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 16 * c + 4 * h + 8);
        const u32x4 w = {lo.x, lo.y, hi.x, hi.y};
        o[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w), pb[c], o[j],
                                                       0, 0, 0);
      }
    }
    if (kb + 1 < nkv) store_kv<D>(st, Ks[cur ^ 1], Vts[cur ^ 1]);
    __syncthreads();
  }

  // O[q][d], d = 32j + 8u + 4h + i: four contiguous bf16 per (j, u)
  const float inv = 1.0f / l;
  uint16_t* orow = p.O + base + static_cast<int64_t>(q) * D;
#pragma unroll
  for (int j = 0; j < ND; ++j)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int d = 32 * j + 8 * u + 4 * h;
      const u32x2 w = {pk_bf16(o[j][4 * u] * inv, o[j][4 * u + 1] * inv),
                       pk_bf16(o[j][4 * u + 2] * inv, o[j][4 * u + 3] * inv)};
      *reinterpret_cast<u32x2*>(orow + d) = w;
    }
}

template <int D, bool CAUSAL>
int launch(const SdpaArgs& a, hipStream_t s) {
  hipLaunchKernelGGL((sdpa_fwd_kernel<D, CAUSAL>), dim3(a.nbh * a.nqb), dim3(kThreads), 0, s, a);
  return check_launch("sdpa_fwd_kernel");
}

}  // namespace
}  // namespace ttlh

using namespace ttlh;

extern "C" int ttlh_sdpa_fwd(const void* Q, const void* K, const void* V, void* O, int64_t B,
                             int64_t H, int64_t S, int64_t D, float scale, int causal,
                             void* stream) {
  clear_error();
  TTLH_REQUIRE(Q && K && V && O, TTLH_EINVAL, "ttlh_sdpa_fwd: null pointer");
  TTLH_REQUIRE(B > 0 && H > 0 && S > 0, TTLH_EINVAL, "ttlh_sdpa_fwd: empty problem");
  TTLH_REQUIRE(D == 64 || D == 128, TTLH_EUNSUPPORTED, "ttlh_sdpa_fwd: head_dim must be 64 or 128");
  TTLH_REQUIRE(S % BQ == 0, TTLH_EUNSUPPORTED, "ttlh_sdpa_fwd: seq_len must be a multiple of %d",
               BQ);
  TTLH_REQUIRE(B * H * (S / BQ) < (int64_t(1) << 31), TTLH_EUNSUPPORTED,
               "ttlh_sdpa_fwd: too many query blocks");
  TTLH_REQUIRE(S * D < (int64_t(1) << 31), TTLH_EUNSUPPORTED, "ttlh_sdpa_fwd: seq_len too long");
  for (const void* ptr : {Q, K, V, static_cast<const void*>(O)})
    TTLH_REQUIRE((reinterpret_cast<uintptr_t>(ptr) & 15) == 0, TTLH_EINVAL,
                 "ttlh_sdpa_fwd: tensors must be 16-byte aligned");
  TTLH_REQUIRE(std::isfinite(scale), TTLH_EINVAL, "ttlh_sdpa_fwd: scale must be finite");
  SdpaArgs a;
  a.Q = static_cast<const uint16_t*>(Q);
  a.K = static_cast<const uint16_t*>(K);
  a.V = static_cast<const uint16_t*>(V);
  a.O = static_cast<uint16_t*>(O);
  a.S = static_cast<int32_t>(S);
  a.nqb = static_cast<int32_t>(S / BQ);
  a.nbh = static_cast<int32_t>(B * H);
  a.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (D == 128) return causal ? launch<128, true>(a, s) : launch<128, false>(a, s);
  return causal ? launch<64, true>(a, s) : launch<64, false>(a, s);
}
