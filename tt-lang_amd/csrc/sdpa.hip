// Fused scaled-dot-product attention forward for gfx950:
//   O[b, h] = softmax(Q[b, h] K[b, h]^T * scale) V[b, h],  bf16 in / out,
//   fp32 scores and online softmax.
//
// The reference has no attention kernel; this composes the spec's tile ops
// (@, exp, reduce_max, reduce_sum, recip, broadcast:
// docs/sphinx/specs/TTLangSpecification.md:693-761) into one flash-style pass.
//
// Per wave, 32 query rows and per KV block (64 rows):
//     S^T = K Q^T   (16 x v_mfma_f32_32x32x16_bf16, Q^T operands kept in VGPRs)
//     O^T += V^T P^T (16 more MFMAs)
// Computing the transposes puts one query row in each lane's accumulator
// column for both products, so the softmax statistics (running max m and sum
// l) and the O rescale are per-lane scalars; the two lane halves that share a
// query combine with one exchange.  P goes from the S accumulators to the
// second MFMA without touching LDS: the accumulator layout hands each lane kv
// rows {16c + 4h + 8u + i}, so the V^T operand is read in the same kv order
// (the contraction is invariant under a common permutation of kv), with two
// ds_read_b64_tr_b16 transpose loads from row-major V: within a group of 16
// lanes, output lane i, element k is element i % 4 of the 8 bytes that lane
// 4k + i / 4 addresses, so lanes addressing 4 kv rows x 16 d columns receive
// 4 consecutive kv of one d column each.
//
// Three kernels share that per-wave math:
//  * sdpa_w8_kernel (D = 128, non-causal, S a multiple of 256): 8 waves of
//    32 queries, two per SIMD, each interleaving the MFMAs of a KV block with
//    the softmax of the previous one, the second wave's VALU issuing under
//    the first one's MFMAs; Q pre-scaled and the S accumulation started from
//    -m, so the softmax is one exp2 per score; a persistent grid of one
//    workgroup per CU (details at its definition);
//  * sdpa_pp_kernel (other cases with S a multiple of 256): 8 waves, 256
//    queries per workgroup, the two groups of four waves in ping-pong, one
//    issuing the MFMAs of a block while the other runs the softmax of the
//    previous one;
//  * sdpa_fwd_kernel (S a multiple of 128): 4 waves, 128 queries, each wave
//    running both parts in turn, two workgroups per CU.
//
// K and V are staged in LDS as loaded (row-major, 16-byte stores).  gfx950's
// LDS serves 256 bytes (64 banks) per cycle: a ds_read_b128 is conflict-free
// when each 16 lanes hit 16 distinct 16-byte bank groups, a ds_read_b64 when
// each 32 lanes do.  Row pitches of D + 8 (K: 16 rows, one chunk each) and
// D + 32 elements (V: 4 rows x 4 chunks per 32 lanes of a transpose read)
// meet that.  The next block's K and V are fetched into registers while the
// current block computes.
// Softmax runs in the log2 domain: exp2(fma(s, scale log2 e, -m)) in the
// other two kernels, with the block max taken on the raw scores (sign of the
// scale handled by taking the min instead); the causal mask touches only the blocks
// that straddle the diagonal.  P is rounded to bf16 for the MFMA; O is
// divided by l at the end.  Workgroup ids are regrouped so the query blocks
// of one (batch, head) land on the same XCD and share K/V in its L2.

#include <cmath>
#include <type_traits>

#include "ttlh_common.h"

namespace ttlh {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef const __attribute__((address_space(1))) u32x4 gu32x4;
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int BQ = 128;   // query rows per workgroup
constexpr int BKV = 64;   // kv rows per block
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

__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) { return cvt_pk_bf16x2(lo, hi); }

// x combined with the value of lane l ^ 32, without LDS: v_permlane32_swap
// exchanges the upper half of its first operand with the lower half of its
// second, so with both operands = x the two results hold, per lane, x and
// x of lane l ^ 32 (in some order)
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_min(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fminf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_add(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// s_waitcnt immediate (gfx9 encoding): at most n global loads outstanding
constexpr int vmcnt_imm_sdpa(int n) { return 0x0F70 | (n & 0xF) | ((n >> 4) << 14); }

template <int D>
constexpr int kKPitch = D + 8;   // K rows in LDS (elements)
template <int D>
constexpr int kVPitch = D + 32;  // V rows in LDS (elements)

// K or V rows kv0 .. kv0 + 63 as 16-byte chunks, D / 32 per thread; with
// RAGGED, rows from `end` on (past the sequence) read as zeros
template <int D, bool RAGGED = false>
__device__ __forceinline__ void load_rows(const uint16_t* X, int64_t base, int kv0, u32x4 (&r)[D / 32],
                                          int end = 0) {
  const int t = threadIdx.x;
  constexpr int kChunksPerRow = D / 8;
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    const int c = t + i * kThreads;
    const int row = c / kChunksPerRow, dc = (c % kChunksPerRow) * 8;
    if (RAGGED && kv0 + row >= end) {
      r[i] = u32x4{0u, 0u, 0u, 0u};
      continue;
    }
    r[i] = *reinterpret_cast<gu32x4*>(
        reinterpret_cast<uintptr_t>(X + base + static_cast<int64_t>(kv0 + row) * D + dc));
  }
}

template <int D, int PITCH>
__device__ __forceinline__ void store_rows(const u32x4 (&r)[D / 32], uint16_t* dst) {
  const int t = threadIdx.x;
  constexpr int kChunksPerRow = D / 8;
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    const int c = t + i * kThreads;
    const int row = c / kChunksPerRow, dc = (c % kChunksPerRow) * 8;
    *reinterpret_cast<u32x4*>(dst + row * PITCH + dc) = r[i];
  }
}

// 4 consecutive kv rows (from kv0) of column d0 + (lane & 15) of V, as 4
// bf16 (see the transpose-load rule above)
template <int D>
__device__ __forceinline__ i16x4 read_v4(const uint16_t* Vs, int kv0, int d0, int lane) {
  const uint16_t* a = Vs + (kv0 + ((lane & 15) >> 2)) * kVPitch<D> + d0 + 4 * (lane & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)a);
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

template <int D, bool CAUSAL, bool RAGGED = false>
struct Sdpa {
  static constexpr int ND = D / 32;   // d tiles of O^T
  static constexpr int NDC = D / 16;  // 16-wide d chunks of the S^T contraction

  const SdpaArgs& p;
  uint16_t (*Ks)[BKV * kKPitch<D>];
  uint16_t (*Vs)[BKV * kVPitch<D>];
  int64_t base;
  int qb, wave, lane, l32, h, q, nkv;
  float sc;
  bf16x8 qop[NDC];
  f32x16 o[ND];
  float m, l;
  u32x4 stk[D / 32], stv[D / 32];  // K and V rows of the next block

  // S^T = K Q^T for the K block at K_ (raw scores)
  __device__ __forceinline__ void scores(const uint16_t* K_, f32x16 (&sv)[2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sv[t][r] = 0.0f;
#pragma unroll
      for (int dc = 0; dc < NDC; ++dc) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(K_ + (32 * t + l32) * kKPitch<D> +
                                                          dc * 16 + 8 * h);
        sv[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qop[dc], sv[t], 0, 0, 0);
      }
    }
  }

  __device__ __forceinline__ float expo(float v) const {
    return __builtin_amdgcn_exp2f(__builtin_fmaf(v, sc, -m));
  }

  // One KV block kb: the next block's K and V are fetched into registers
  // while this one computes S, the softmax and O += V(kb)^T P^T from LDS
  // buffer kb & 1, then stored into the other buffer (last read before the
  // previous barrier).
  __device__ __forceinline__ void step(int kb) {
    const uint16_t* Kc = Ks[kb & 1];
    const uint16_t* Vc = Vs[kb & 1];
    if (kb + 1 < nkv) {
      load_rows<D, RAGGED>(p.K, base, (kb + 1) * BKV, stk, p.S);
      load_rows<D, RAGGED>(p.V, base, (kb + 1) * BKV, stv, p.S);
    }
    f32x16 cur[2];
    scores(Kc, cur);

    // causal: only blocks that reach past this wave's first query need a
    // mask; ragged: the block that runs past the sequence end masks the kv
    // beyond it (masked scores drop out of the block extreme and get exp 0)
    const bool diag = (CAUSAL && kb * BKV + BKV - 1 > qb * BQ + wave * 32) ||
                      (RAGGED && kb * BKV + BKV > p.S);
    auto masked = [&](int kv) { return (CAUSAL && kv > q) || (RAGGED && kv >= p.S); };
    if (diag) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kv = kb * BKV + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
          if (masked(kv)) cur[t][r] = sc >= 0.0f ? -INFINITY : INFINITY;
        }
    }
    // block extreme of the raw scores: max if the scale is positive, else min
    float ex = cur[0][0];
    if (sc >= 0.0f) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) ex = fmaxf(ex, cur[t][r]);
      ex = fmaxf(ex, __shfl_xor(ex, 32));
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) ex = fminf(ex, cur[t][r]);
      ex = fminf(ex, __shfl_xor(ex, 32));
    }
    const float m_new = fmaxf(m, ex * sc);
    // rescale O only when some lane's running max moved
    if (__any(m_new != m)) {
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);  // 0 on the first block
      l *= alpha;
#pragma unroll
      for (int j = 0; j < ND; ++j) o[j] *= alpha;
      m = m_new;
    }
    float rs = 0.0f;
    if (diag) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kv = kb * BKV + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
          const float e = masked(kv) ? 0.0f : expo(cur[t][r]);
          cur[t][r] = e;
          rs += e;
        }
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = expo(cur[t][r]);
          cur[t][r] = e;
          rs += e;
        }
    }
    rs += __shfl_xor(rs, 32);
    l += rs;

    // P^T operands: chunk c (16 kv) = tile c/2, accumulators 8(c%2) .. +8
    bf16x8 pb[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int t = c >> 1, r0 = 8 * (c & 1);
      u32x4 w;
      w.x = pk_bf16(cur[t][r0 + 0], cur[t][r0 + 1]);
      w.y = pk_bf16(cur[t][r0 + 2], cur[t][r0 + 3]);
      w.z = pk_bf16(cur[t][r0 + 4], cur[t][r0 + 5]);
      w.w = pk_bf16(cur[t][r0 + 6], cur[t][r0 + 7]);
      pb[c] = __builtin_bit_cast(bf16x8, w);
    }
    // O^T += V^T P^T; the V^T operand of lane (d = 32j + l32, h) holds kv
    // {16c + 4h + i, 16c + 4h + 8 + i}
#pragma unroll
    for (int j = 0; j < ND; ++j) {
      const int d0 = 32 * j + 16 * ((lane >> 4) & 1);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const i16x4 lo = read_v4<D>(Vc, 16 * c + 4 * h, d0, lane);
        const i16x4 hi = read_v4<D>(Vc, 16 * c + 4 * h + 8, d0, lane);
        const i16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w), pb[c], o[j],
                                                       0, 0, 0);
      }
    }
    if (kb + 1 < nkv) {
      store_rows<D, kKPitch<D>>(stk, Ks[(kb + 1) & 1]);
      store_rows<D, kVPitch<D>>(stv, Vs[(kb + 1) & 1]);
    }
    __syncthreads();
  }
};

// RAGGED: S a multiple of 32 only.  The last query block holds waves past
// the sequence (S % 32 == 0 keeps each wave wholly in or out): they read a
// clamped Q row, take part in the K / V staging and barriers, store nothing.
// The last KV block reads rows past S as zeros and masks their scores.
template <int D, bool CAUSAL, bool RAGGED = false>
__global__ __launch_bounds__(kThreads, 2) void sdpa_fwd_kernel(const SdpaArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BKV * kKPitch<D>];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][BKV * kVPitch<D>];
  Sdpa<D, CAUSAL, RAGGED> w{p, Ks, Vs};
  int bh;
  block_coords(p, bh, w.qb);
  w.lane = threadIdx.x & 63;
  w.wave = threadIdx.x >> 6;
  w.l32 = w.lane & 31;
  w.h = w.lane >> 5;
  w.base = static_cast<int64_t>(bh) * p.S * D;
  w.q = w.qb * BQ + w.wave * 32 + w.l32;  // this lane's query row
  w.sc = p.scale_log2;
  w.m = -INFINITY;  // running max of s * scale * log2 e
  w.l = 0.0f;
  if constexpr (RAGGED) {
    const int nall = (p.S + BKV - 1) / BKV;
    w.nkv = CAUSAL ? min(nall, (w.qb * BQ + BQ) / BKV) : nall;
  } else {
    w.nkv = CAUSAL ? (w.qb * BQ + BQ) / BKV : p.S / BKV;
  }
  const int qload = RAGGED ? min(w.q, p.S - 1) : w.q;  // a wave past S reads a valid row

  // prologue: K(0), V(0) into LDS; Q^T into VGPRs
  load_rows<D, RAGGED>(p.K, w.base, 0, w.stk, p.S);
  load_rows<D, RAGGED>(p.V, w.base, 0, w.stv, p.S);
#pragma unroll
  for (int dc = 0; dc < D / 16; ++dc)
    w.qop[dc] = *reinterpret_cast<const bf16x8*>(p.Q + w.base + static_cast<int64_t>(qload) * D +
                                                 dc * 16 + 8 * w.h);
#pragma unroll
  for (int j = 0; j < D / 32; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) w.o[j][r] = 0.0f;
  store_rows<D, kKPitch<D>>(w.stk, Ks[0]);
  store_rows<D, kVPitch<D>>(w.stv, Vs[0]);
  // Q^T must have landed before the loop: otherwise the compiler, merging
  // the first iteration's state (Q loads in flight) with later ones, makes
  // every S MFMA of every block wait on the next block's K/V prefetch
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();

  for (int kb = 0; kb < w.nkv; ++kb) w.step(kb);
  if (RAGGED && w.q >= p.S) return;  // wave-uniform (S % 32 == 0); no barrier follows

  // O[q][d], d = 32j + 8u + 4h + i: four contiguous bf16 per (j, u)
  const float inv = 1.0f / w.l;
  uint16_t* orow = p.O + w.base + static_cast<int64_t>(w.q) * D;
#pragma unroll
  for (int j = 0; j < D / 32; ++j)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int d = 32 * j + 8 * u + 4 * w.h;
      const u32x2 v = {pk_bf16(w.o[j][4 * u] * inv, w.o[j][4 * u + 1] * inv),
                       pk_bf16(w.o[j][4 * u + 2] * inv, w.o[j][4 * u + 3] * inv)};
      *reinterpret_cast<u32x2*>(orow + d) = v;
    }
}

// ---------------------------------------------------------------------------
// Ping-pong variant: 512 threads = two groups of four waves, 256 queries per
// workgroup (wave w owns rows 32 w .. 32 w + 31; group g = w / 4).  Each wave
// alternates two phases per KV block i:
//   X(i): O^T += V(i-1)^T P(i-1)^T and S^T = K(i) Q^T  (32 MFMAs, no softmax)
//   Y(i): softmax of S(i) -> P(i), running max / sum, O rescale (VALU only)
// and group 1 runs one phase behind group 0, so on every SIMD (which holds one
// wave of each group) one wave issues MFMAs while the other does the softmax:
// the matrix core and the VALU overlap across waves.  A workgroup barrier
// separates the phases.  LDS holds two stages; stage i = {K(i), V(i-1)} (the
// operands of X(i)) in buffer i & 1.  Every wave loads its share of stage
// i + 1 into registers one phase before writing it to LDS, right after the
// last reader of that buffer has passed a barrier.
constexpr int PP_BQ = 256;
constexpr int PP_THREADS = 512;

template <int N, typename F>
__device__ __forceinline__ void sd_static_for(F&& f) {
  if constexpr (N > 0) {
    sd_static_for<N - 1>(f);
    f(std::integral_constant<int, N - 1>());
  }
}


template <int D>
__device__ __forceinline__ void pp_load(const uint16_t* X, int64_t base, int kv0,
                                        u32x4 (&r)[D / 64]) {
  const int t = threadIdx.x;
  constexpr int kChunksPerRow = D / 8;
#pragma unroll
  for (int i = 0; i < D / 64; ++i) {
    const int c = t + i * PP_THREADS;
    const int row = c / kChunksPerRow, dc = (c % kChunksPerRow) * 8;
    r[i] = *reinterpret_cast<gu32x4*>(
        reinterpret_cast<uintptr_t>(X + base + static_cast<int64_t>(kv0 + row) * D + dc));
  }
}

template <int D, int PITCH>
__device__ __forceinline__ void pp_store(const u32x4 (&r)[D / 64], uint16_t* dst) {
  const int t = threadIdx.x;
  constexpr int kChunksPerRow = D / 8;
#pragma unroll
  for (int i = 0; i < D / 64; ++i) {
    const int c = t + i * PP_THREADS;
    const int row = c / kChunksPerRow, dc = (c % kChunksPerRow) * 8;
    *reinterpret_cast<u32x4*>(dst + row * PITCH + dc) = r[i];
  }
}

// phase boundary: this wave's LDS accesses are complete, then a workgroup
// barrier with no memory fence (global loads stay in flight); the empty asm
// statements keep the compiler from moving memory accesses across it and the
// scheduling barriers keep MFMAs and VALU work in their phase
__device__ __forceinline__ void pp_boundary() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

template <int D, bool CAUSAL>
struct SdpaPP {
  static constexpr int ND = D / 32;
  static constexpr int NDC = D / 16;

  const SdpaArgs& p;
  uint16_t (*Ks)[BKV * kKPitch<D>];
  uint16_t (*Vs)[BKV * kVPitch<D>];
  int64_t base;
  int qb, wave, lane, l32, h, q, n;
  float sc;
  bf16x8 qop[NDC];
  f32x16 o[ND];
  f32x16 cur[2];
  bf16x8 pb[4];
  float m, l;
  u32x4 stk[D / 64], stv[D / 64];

  // stage j = {K(j) if j < n, V(j - 1) if j >= 1} into registers / into LDS
  __device__ __forceinline__ void load_stage(int j) {
    if (j < n) pp_load<D>(p.K, base, j * BKV, stk);
    if (j >= 1 && j <= n) pp_load<D>(p.V, base, (j - 1) * BKV, stv);
  }
  __device__ __forceinline__ void write_stage(int j) {
    if (j < n) pp_store<D, kKPitch<D>>(stk, Ks[j & 1]);
    if (j >= 1 && j <= n) pp_store<D, kVPitch<D>>(stv, Vs[j & 1]);
  }

  // X(i): DO_O adds V(i-1)^T P(i-1)^T, DO_S computes S(i); operands from
  // LDS buffer i & 1.  The MFMAs (S and O alternating when both run) form a
  // software pipeline: the LDS fragments of MFMA m + kPipe are requested
  // right after MFMA m issues, so LDS latency hides behind kPipe MFMAs; the
  // scheduling barriers keep that order.
  static constexpr int kPipe = 6;

  template <bool DO_O, bool DO_S, int M>
  __device__ __forceinline__ void x_frag(const uint16_t* Kc, const uint16_t* Vc, bf16x8& f) {
    constexpr bool kIsO = DO_O && DO_S ? (M & 1) != 0 : DO_O;
    constexpr int k = DO_O && DO_S ? (M >> 1) : M;
    if constexpr (kIsO) {
      constexpr int j = k >> 2, c = k & 3;
      const int d0 = 32 * j + 16 * ((lane >> 4) & 1);
      const i16x4 lo = read_v4<D>(Vc, 16 * c + 4 * h, d0, lane);
      const i16x4 hi = read_v4<D>(Vc, 16 * c + 4 * h + 8, d0, lane);
      const i16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      f = __builtin_bit_cast(bf16x8, w);
    } else {
      constexpr int t = k / NDC, dc = k % NDC;
      f = *reinterpret_cast<const bf16x8*>(Kc + (32 * t + l32) * kKPitch<D> + dc * 16 + 8 * h);
    }
  }

  template <bool DO_O, bool DO_S, int M>
  __device__ __forceinline__ void x_mfma(const bf16x8& f) {
    constexpr bool kIsO = DO_O && DO_S ? (M & 1) != 0 : DO_O;
    constexpr int k = DO_O && DO_S ? (M >> 1) : M;
    if constexpr (kIsO) {
      constexpr int j = k >> 2, c = k & 3;
      o[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f, pb[c], o[j], 0, 0, 0);
    } else {
      constexpr int t = k / NDC, dc = k % NDC;
      cur[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f, qop[dc], cur[t], 0, 0, 0);
    }
  }

  template <bool DO_O, bool DO_S>
  __device__ __forceinline__ void x_phase(int i) {
    const uint16_t* Kc = Ks[i & 1];
    const uint16_t* Vc = Vs[i & 1];
    constexpr int T = (DO_S ? 2 * NDC : 0) + (DO_O ? 4 * ND : 0);
    if constexpr (DO_S) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) cur[t][r] = 0.0f;
    }
    bf16x8 fr[T];
    sd_static_for<(kPipe < T ? kPipe : T)>([&](auto mc) {
      x_frag<DO_O, DO_S, decltype(mc)::value>(Kc, Vc, fr[decltype(mc)::value]);
    });
    __builtin_amdgcn_sched_barrier(0);
    sd_static_for<T>([&](auto mc) {
      constexpr int m = decltype(mc)::value;
      x_mfma<DO_O, DO_S, m>(fr[m]);
      if constexpr (m + kPipe < T) x_frag<DO_O, DO_S, m + kPipe>(Kc, Vc, fr[m + kPipe]);
      __builtin_amdgcn_sched_barrier(0);
    });
  }

  __device__ __forceinline__ float expo(float v) const {
    return __builtin_amdgcn_exp2f(__builtin_fmaf(v, sc, -m));
  }

  // Y(i): online softmax of S(i) into P(i) (masking and extreme rules as in
  // Sdpa::step).  The running max m moves lazily: only when a lane's block
  // maximum exceeds it by more than kLazy (log2 units), so O and l are rarely
  // rescaled; until then P = exp2(s - m) <= 2^kLazy, which fp32 O / l and the
  // bf16 P operands hold without loss (the final O / l is unchanged by the
  // choice of m).
  static constexpr float kLazy = 8.0f;

  __device__ __forceinline__ void y_phase(int kb) {
    const bool diag = CAUSAL && kb * BKV + BKV - 1 > qb * PP_BQ + wave * 32;
    // element (t, r) holds kv = kb*BKV + 4h + (32t + 8(r/4) + r%4): masked
    // when that offset exceeds lim (compared against literal constants)
    const int lim = q - kb * BKV - 4 * h;
    if (diag) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (32 * t + 8 * (r >> 2) + (r & 3) > lim) cur[t][r] = sc >= 0.0f ? -INFINITY : INFINITY;
    }
    // block extreme as a 4-way tree (short dependency chains)
    float ex;
    if (sc >= 0.0f) {
      float p4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int t = u >> 1, r0 = 8 * (u & 1);
        p4[u] = fmaxf(fmaxf(fmaxf(cur[t][r0], cur[t][r0 + 1]), fmaxf(cur[t][r0 + 2], cur[t][r0 + 3])),
                      fmaxf(fmaxf(cur[t][r0 + 4], cur[t][r0 + 5]), fmaxf(cur[t][r0 + 6], cur[t][r0 + 7])));
      }
      ex = xor32_max(fmaxf(fmaxf(p4[0], p4[1]), fmaxf(p4[2], p4[3])));
    } else {
      float p4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int t = u >> 1, r0 = 8 * (u & 1);
        p4[u] = fminf(fminf(fminf(cur[t][r0], cur[t][r0 + 1]), fminf(cur[t][r0 + 2], cur[t][r0 + 3])),
                      fminf(fminf(cur[t][r0 + 4], cur[t][r0 + 5]), fminf(cur[t][r0 + 6], cur[t][r0 + 7])));
      }
      ex = xor32_min(fminf(fminf(p4[0], p4[1]), fminf(p4[2], p4[3])));
    }
    const float m_blk = ex * sc;
    const bool grow = m_blk > m + kLazy;
    if (__any(grow)) {
      const float m_new = grow ? m_blk : m;
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);  // 1 where m stays, 0 at first
      l *= alpha;
#pragma unroll
      for (int j = 0; j < ND; ++j) o[j] *= alpha;
      m = m_new;
    }
    if (diag) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          cur[t][r] = 32 * t + 8 * (r >> 2) + (r & 3) > lim ? 0.0f : expo(cur[t][r]);
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) cur[t][r] = expo(cur[t][r]);
    }
    // row sum as four independent partial sums (short dependency chains)
    float rs4[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int t = c >> 1, r0 = 8 * (c & 1);
      u32x4 w;
      w.x = pk_bf16(cur[t][r0 + 0], cur[t][r0 + 1]);
      w.y = pk_bf16(cur[t][r0 + 2], cur[t][r0 + 3]);
      w.z = pk_bf16(cur[t][r0 + 4], cur[t][r0 + 5]);
      w.w = pk_bf16(cur[t][r0 + 6], cur[t][r0 + 7]);
      pb[c] = __builtin_bit_cast(bf16x8, w);
      rs4[c] = ((cur[t][r0] + cur[t][r0 + 1]) + (cur[t][r0 + 2] + cur[t][r0 + 3])) +
               ((cur[t][r0 + 4] + cur[t][r0 + 5]) + (cur[t][r0 + 6] + cur[t][r0 + 7]));
    }
    l += xor32_add((rs4[0] + rs4[1]) + (rs4[2] + rs4[3]));
  }

  // group 0: X(i), write stage i+1 | load stage i+2, Y(i).  The first and
  // last X phases (S only, O only) are peeled so the steady loop has one body.
  __device__ __forceinline__ void run_group0() {
    x_phase<false, true>(0);
    write_stage(1);
    pp_boundary();
    load_stage(2);
    y_phase(0);
    pp_boundary();
    for (int i = 1; i < n; ++i) {
      x_phase<true, true>(i);
      write_stage(i + 1);
      pp_boundary();
      load_stage(i + 2);
      y_phase(i);
      pp_boundary();
    }
    x_phase<true, false>(n);
    pp_boundary();
  }
  // group 1, one phase behind: Y(i-1), write stage i+1 | load stage i+2, X(i)
  __device__ __forceinline__ void run_group1() {
    write_stage(1);
    pp_boundary();
    load_stage(2);
    x_phase<false, true>(0);
    pp_boundary();
    for (int i = 1; i < n; ++i) {
      y_phase(i - 1);
      write_stage(i + 1);
      pp_boundary();
      load_stage(i + 2);
      x_phase<true, true>(i);
      pp_boundary();
    }
    y_phase(n - 1);
    pp_boundary();
    x_phase<true, false>(n);
  }
};

// the workgroup's queries: query blocks of one (b, h) kept on one XCD
__device__ __forceinline__ void pp_block_coords(const SdpaArgs& p, int& bh, int& qb) {
  block_coords(p, bh, qb);
}

template <int D, bool CAUSAL>
__global__ __launch_bounds__(PP_THREADS, 1) void sdpa_pp_kernel(const SdpaArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BKV * kKPitch<D>];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2][BKV * kVPitch<D>];
  SdpaPP<D, CAUSAL> w{p, Ks, Vs};
  int bh;
  pp_block_coords(p, bh, w.qb);
  w.lane = threadIdx.x & 63;
  w.wave = threadIdx.x >> 6;
  w.l32 = w.lane & 31;
  w.h = w.lane >> 5;
  w.base = static_cast<int64_t>(bh) * p.S * D;
  w.q = w.qb * PP_BQ + w.wave * 32 + w.l32;
  w.sc = p.scale_log2;
  w.m = -INFINITY;
  w.l = 0.0f;
  w.n = CAUSAL ? (w.qb * PP_BQ + PP_BQ) / BKV : p.S / BKV;

  // prologue: Q^T into VGPRs, stage 0 (K(0)) into LDS, stage 1 into registers
#pragma unroll
  for (int dc = 0; dc < D / 16; ++dc)
    w.qop[dc] = *reinterpret_cast<const bf16x8*>(p.Q + w.base + static_cast<int64_t>(w.q) * D +
                                                 dc * 16 + 8 * w.h);
  w.load_stage(0);
  // Q^T and K(0) must have landed before any later load is issued: the
  // stage loads are conditional, so a partial wait after them would leave Q
  // "possibly in flight" on some path, and the compiler would then make every
  // S MFMA wait for the stage prefetch in flight at that point
  __builtin_amdgcn_s_waitcnt(vmcnt_imm_sdpa(0));
  w.write_stage(0);
  w.load_stage(1);
#pragma unroll
  for (int j = 0; j < D / 32; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) w.o[j][r] = 0.0f;
  pp_boundary();

  if (w.wave < 4) w.run_group0();
  else w.run_group1();

  const float inv = 1.0f / w.l;
  uint16_t* orow = p.O + w.base + static_cast<int64_t>(w.q) * D;
#pragma unroll
  for (int j = 0; j < D / 32; ++j)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int d = 32 * j + 8 * u + 4 * w.h;
      const u32x2 v = {pk_bf16(w.o[j][4 * u] * inv, w.o[j][4 * u + 1] * inv),
                       pk_bf16(w.o[j][4 * u + 2] * inv, w.o[j][4 * u + 3] * inv)};
      *reinterpret_cast<u32x2*>(orow + d) = v;
    }
}

// ---------------------------------------------------------------------------
// 32 queries per wave, eight waves (two per SIMD) per block of 256 queries
// (D = 128, non-causal: C5).  KV blocks of 32 rows; step i of a block is one
// straight-line piece of code:
//     MFMAs: S(i) = K(i) Q^T and O += V(i-2)^T P(i-2)^T (16)
//     VALU:  the softmax of S(i-1) -> P(i-1) and its row sum (the running
//            max moves only on a rare path, see below)
// in eight sections, one per K / V fragment: the section's two MFMAs, a
// share of the softmax VALU, and the LDS reads of the fragments two sections
// ahead.  Two waves per SIMD because a wave alone cannot hide its VALU work:
// on gfx950 an MFMA holds its own wave's issue for about half of its 32
// cycles, so VALU placed between one wave's MFMAs mostly adds to them, while
// a second wave's VALU issues under them (measured: MFMA + 16 FMAs takes 80
// cycles for one wave, 62 for two).  The cost is LDS traffic: each K / V
// fragment feeds one MFMA (128 KB per step per CU; gfx950's LDS serves 256
// bytes per clock to ds_read_b128 and ~186 to ds_read_b64_tr_b16, measured,
// so the reads take ~600 of the step's 1024 MFMA cycles).  The accumulators
// fit in the architectural VGPRs (239, no AGPRs), so the softmax reads S
// without copies.  The waves raise their priority (s_setprio 1) over the first six
// sections, where MFMAs and LDS reads are densest, so a SIMD's matrix core
// is fed first and the other wave's VALU fills the gaps.
// K and V reach LDS by direct-to-LDS DMA (global_load_lds_dwordx4, lane l's
// 16 bytes at the wave's base + 16 l) into rings of four K and four V
// buffers (64 KB): step t reads K(t) from K buffer t % 4 and V(t - 2) from V
// buffer (t - 2) % 4, and loads K(t + 3) and V(t + 1); one workgroup barrier
// per step, and each step's first two K / V fragments are read before the
// previous step's barrier (their blocks were published one barrier earlier).
// Rows are unpadded with XOR-swizzled 16-byte chunks: K chunk c of row r at
// c ^ (r & 15) (the S operand reads 16 rows of one chunk per 16 lanes), V at
// c ^ 4 (r & 3) (a transpose read covers 4 rows x 4 chunks per 32 lanes).
// The grid is persistent: one workgroup per CU walks a sequence of query
// blocks, and the step pipeline runs across block boundaries (t counts steps
// over the sequence; a block is n steps, a multiple of 4, so the ring phases
// repeat).  A block's steps 0 and 1 also carry the previous block's last
// softmax and O products, its first K / V blocks are the loads that follow
// the previous block's, its Q is staged into LDS four steps ahead (64 KB, per
// wave) and loaded into registers at the end of the previous block, and a
// finished block's O is stored after the step holding its last product: per
// block there is no pipeline fill or drain, no Q load latency and no
// workgroup launch (3% faster than one workgroup per block).
constexpr int W8_BQ = 256;
constexpr int W8_THREADS = 512;
constexpr int W8_D = 128;
constexpr int W8_KV = 32;

// one array per ring, so a buffer is a constant offset from the others (an
// immediate in the LDS instructions, not another address register)
__shared__ __attribute__((aligned(16))) uint16_t w8K[4][W8_KV * W8_D];
__shared__ __attribute__((aligned(16))) uint16_t w8V[4][W8_KV * W8_D];
// per wave, the next block's 32 Q rows (staged four steps ahead)
__shared__ __attribute__((aligned(16))) uint16_t w8Q[8][32 * W8_D];

template <int B>
__device__ __forceinline__ uint16_t* w8_kbuf() {
  return w8K[B];
}
template <int B>
__device__ __forceinline__ uint16_t* w8_vbuf() {
  return w8V[B];
}

typedef __attribute__((address_space(3))) void w8_lds_void;

struct SdpaW8 {
  static constexpr int D = W8_D, ND = D / 32, NDC = D / 16;

  const SdpaArgs& p;
  int wave, lane, l32, h, n;
  bf16x8 qop[NDC];          // Q^T operands, scaled by scale * log2(e)
  f32x16 o[ND];             // O^T accumulators
  f32x16 s;                 // S(i) - m accumulating
  f32x16 sv;                // S(i - 1) - m (renamed, not copied: both live in VGPRs)
  f32x16 negm;              // -m in every element: where each S accumulation starts
  u32x4 pw[2][2];           // [parity][kv chunk]: P(i - 1), P(i - 2) as bf16 pairs
  float m, l;               // running max (log2 units), this lane's share of the row sum
  int k_src, v_src;         // per-lane DMA source offsets (elements)
  int v_frag[ND];           // LDS offsets of the V transpose reads
  uint32_t lds_wave;        // the wave's byte offset in a K / V buffer (uniform)
  bf16x8 kpf[2], vpf[2];    // the next step's first K / V fragments, read before the barrier

  __device__ __forceinline__ void setup() {
    lds_wave = __builtin_amdgcn_readfirstlane(wave * 1024);
    const int pos = wave * 64 + lane;  // 16-byte chunk position in the buffer
    const int r = pos >> 4, c = pos & 15;
    k_src = r * D + ((c ^ (r & 15)) << 3);
    v_src = r * D + ((c ^ ((r & 3) << 2)) << 3);
    // V transpose reads: row kv0 + (lane & 15) / 4, logical column d0 + 4 (lane & 3),
    // d0 = 32 j + 16 ((lane >> 4) & 1), i.e. chunk 4 j + 2 ((lane >> 4) & 1) + (lane & 3) / 2
    const int vr = (lane & 15) >> 2;
#pragma unroll
    for (int j = 0; j < ND; ++j) {
      const int chunk = 4 * j + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
      v_frag[j] = vr * D + ((chunk ^ (vr << 2)) << 3) + 4 * (lane & 1);
    }
  }

  // 32 K or V rows from kv0 into an LDS buffer: one DMA instruction per thread,
  // issued as inline asm: with a compiler-visible LDS DMA outstanding, the
  // compiler's wait-count model treats LDS reads as completing out of order
  // and waits for every LDS read (lgkmcnt(0)) before each use, which defeats
  // the fragment prefetch.  The DMA counts only on vmcnt, waited explicitly
  // at the end of every step, before any wave reads the buffer (the loop has
  // no other vector-memory loads, so vmcnt counts exactly these).  M0 carries the wave's LDS base (one wait
  // state before use).  The address is the uniform row base in an SGPR pair
  // plus the lane's 32-bit byte offset: no 64-bit VGPR address, which would
  // need an even-aligned register pair the asm constraint cannot request.
  // Both uniform operands pass through readfirstlane, so they are SGPRs
  // whatever the register allocator made of them (free when they already
  // are); readfirstlane returns int, so each pointer half widens unsigned.
  __device__ __forceinline__ void dma(const uint16_t* X, int64_t base, int src, int kv0,
                                      const uint16_t* lds) {
    const uint64_t g = reinterpret_cast<uint64_t>(X + base + static_cast<int64_t>(kv0) * D);
    const uint64_t gs =
        (uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(g >> 32)))) << 32) |
        uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(g))));
    const uint32_t buf = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((w8_lds_void*)lds));
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2"
        :
        : "s"(__builtin_amdgcn_readfirstlane(buf + lds_wave)),
          "v"(static_cast<uint32_t>(src) * 2u), "s"(gs)
        : "memory", "m0");
  }

  // K fragment (d chunk dc): row l32, 8 elements at 16 dc + 8 h (chunk 2 dc + h)
  __device__ __forceinline__ bf16x8 kfrag(const uint16_t* Kc, int dc) const {
    const int chunk = (2 * dc + h) ^ (l32 & 15);
    return *reinterpret_cast<const bf16x8*>(Kc + l32 * D + chunk * 8);
  }
  // V^T fragment (d tile j, kv chunk c): rows {16c + 4h + i, 16c + 4h + 8 + i}
  __device__ __forceinline__ bf16x8 vfrag(const uint16_t* Vc, int j, int c) const {
    const uint16_t* a0 = Vc + (16 * c + 4 * h) * D + v_frag[j];
    const uint16_t* a1 = a0 + 8 * D;
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)a0);
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)a1);
    const i16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8, w);
  }

  // The softmax of S(i - 1) - m (sv) into pw[PAR]: one pair of scores per
  // section (two exponentials, one bf16 pair, their sum).  Q is pre-scaled
  // by scale * log2(e) and every S accumulation starts from -m (negm), so the
  // exponent argument comes out of the MFMAs.  The running max m does not
  // move on the common path: a lane's block sum above kSumLimit (some P above
  // 2^8) sends the wave to rescale(), which moves m by the block max where
  // that exceeds kLazy.  Otherwise every P = exp2(s - m) <= 2^12, which fp32
  // O and l absorb.  Row maxima use v_maximum3 (NaN-propagating).
  static constexpr float kLazy = 8.0f;
  static constexpr float kSumLimit = 4096.0f;
  float rsum_;

  __device__ __forceinline__ static float max16(const f32x16& c) {
    const float a = __builtin_elementwise_maximum(__builtin_elementwise_maximum(c[0], c[1]), c[2]);
    const float b = __builtin_elementwise_maximum(__builtin_elementwise_maximum(c[3], c[4]), c[5]);
    const float d = __builtin_elementwise_maximum(__builtin_elementwise_maximum(c[6], c[7]), c[8]);
    const float e = __builtin_elementwise_maximum(__builtin_elementwise_maximum(c[9], c[10]), c[11]);
    const float f = __builtin_elementwise_maximum(__builtin_elementwise_maximum(c[12], c[13]), c[14]);
    const float g = __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), d);
    const float hh = __builtin_elementwise_maximum(__builtin_elementwise_maximum(e, f), c[15]);
    return __builtin_elementwise_maximum(g, hh);
  }

  // exponentials of S values 2g, 2g + 1 into one P dword.  The empty asm
  // keeps the bf16 packing in this section: left alone the compiler sinks it
  // into the next step, in front of that step's first LDS reads.  (Summing
  // the bf16 pair with v_dot2c_f32_bf16 instead of two adds measured 4%
  // slower.)
  template <int PAR, int g>
  __device__ __forceinline__ void expo2() {
    const float e0 = __builtin_amdgcn_exp2f(sv[2 * g]);
    const float e1 = __builtin_amdgcn_exp2f(sv[2 * g + 1]);
    uint32_t c = pk_bf16(e0, e1);
    asm volatile("" : "+v"(c));
    pw[PAR][g >> 2][g & 3] = c;
    rsum_ = g == 0 ? e0 + e1 : rsum_ + (e0 + e1);
  }

  // The rare path for P(i - 1) (its scores in sp): move m by the block max d
  // where that exceeds kLazy, recompute P(i - 1), scale O (blocks <= i - 2)
  // and l by 2^-d, shift S(i) (accumulated from the old -m, now in sv) and
  // the start value of the next accumulation.  The updates of O, S and -m
  // are inline asm with tied operands: written as C++, they made the compiler
  // keep a second copy of those registers across the branch (256 VGPRs and
  // spills in the main loop, against 214).  The asm is invisible to the
  // compiler's hazard tracking, so the wait states are explicit: the MFMA
  // results it reads were written before the ~40 VALU instructions above it,
  // and the s_nop after it precedes any MFMA that reads what it wrote.
  template <int PAR, bool SHIFT_S>
  __device__ __forceinline__ void rescale(const f32x16& sp) {
    // SHIFT_S: S(i) was accumulated from the old -m (main steps); otherwise
    // S(i) is a new block's raw first block or absent, and -m is reset
    const float bm = xor32_max(max16(sp));
    const float d = bm > kLazy ? bm : 0.0f;
    const float alpha = __builtin_amdgcn_exp2f(-d);
    m += d;
    float rs = 0.0f;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
      const float e0 = __builtin_amdgcn_exp2f(sp[2 * g] - d);
      const float e1 = __builtin_amdgcn_exp2f(sp[2 * g + 1] - d);
      pw[PAR][g >> 2][g & 3] = pk_bf16(e0, e1);
      rs += e0 + e1;
    }
    rsum_ = rs;
    l *= alpha;
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7");
#pragma unroll
    for (int j = 0; j < ND; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) asm volatile("v_mul_f32 %0, %1, %0" : "+v"(o[j][r]) : "v"(alpha));
    if constexpr (SHIFT_S) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        asm volatile("v_sub_f32 %0, %0, %1" : "+v"(sv[r]) : "v"(d));
        asm volatile("v_mov_b32 %0, %1" : "+v"(negm[r]) : "v"(-m));
      }
    }
    asm volatile("s_nop 7");
  }

  // VALU slots of a section (for the interleave below)
  static constexpr int kSectionValu[8] = {5, 4, 4, 4, 4, 4, 4, 4};

  // ---- the workgroup's sequence of query blocks (persistent grid) ----
  int G, g, nblk, nqb;
  float l_prev;
  __device__ __forceinline__ int perm() const {
    return G % 8 == 0 ? (g % 8) * (G / 8) + g / 8 : g;
  }
  __device__ __forceinline__ void block(int jb, int64_t& base, int& qb) const {
    const int L = jb * G + perm();
    const int bh = L / nqb;
    qb = L - bh * nqb;
    base = static_cast<int64_t>(bh) * p.S * D;
  }

  // Q rows of a block into the wave's staging buffer (swizzled like K),
  // 8 DMA instructions per wave; read back by the same wave only
  __device__ __forceinline__ void stage_q(int64_t base, int qb) {
    if (qb < 0) return;  // no next block
    const int64_t row0 = static_cast<int64_t>(qb) * W8_BQ + 32 * wave;
#pragma unroll
    for (int ins = 0; ins < 8; ++ins) {
      const int r = 4 * ins + (lane >> 4), pc = lane & 15;
      const int src = r * D + ((pc ^ (r & 15)) << 3);
      const uint64_t gq = reinterpret_cast<uint64_t>(p.Q + base + row0 * D);
      const uint64_t gs =
          (uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(gq >> 32)))) << 32) |
          uint64_t(uint32_t(__builtin_amdgcn_readfirstlane(uint32_t(gq))));
      const uint32_t buf = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
          (w8_lds_void*)(w8Q[wave] + ins * 512)));
      asm volatile(
          "s_mov_b32 m0, %0\n\t"
          "s_nop 0\n\t"
          "global_load_lds_dwordx4 %1, %2"
          :
          : "s"(__builtin_amdgcn_readfirstlane(buf)), "v"(static_cast<uint32_t>(src) * 2u),
            "s"(gs)
          : "memory", "m0");
    }
  }
  __device__ __forceinline__ void scale_q(const bf16x8 (&x)[NDC]) {
#pragma unroll
    for (int dc = 0; dc < NDC; ++dc)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        qop[dc][e] = static_cast<__bf16>(static_cast<float>(x[dc][e]) * p.scale_log2);
  }

  // O / l of a finished block into its rows: O[q][d], d = 32j + 8u + 4h + i
  __device__ __forceinline__ void store_o(int64_t base, int qb, float lsum) {
    const float inv = 1.0f / xor32_add(lsum);
    const int64_t q = static_cast<int64_t>(qb) * W8_BQ + 32 * wave + l32;
    uint16_t* orow = p.O + base + q * D;
#pragma unroll
    for (int j = 0; j < ND; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int d = 32 * j + 8 * u + 4 * h;
        const u32x2 v = {pk_bf16(o[j][4 * u] * inv, o[j][4 * u + 1] * inv),
                         pk_bf16(o[j][4 * u + 2] * inv, o[j][4 * u + 3] * inv)};
        *reinterpret_cast<u32x2*>(orow + d) = v;
      }
  }

  // one step at global step t (PAR = t % 2, KB = t % 4): S(t) = K(t) Q^T into
  // s (renamed to sv at the end), the softmax of sv into pw[PAR ^ 1], and
  // O += V(t - 2) P(t - 2) with P(t - 2) in pw[PAR]; K(t) in K buffer KB,
  // V(t - 2) in V buffer (KB + 2) % 4.  Flags:
  //   NEXT_S / NEXT_O  the next step computes S / O (its first fragments are
  //                    read at the end of this step, before the barrier);
  //   OZERO            O starts from zero (a block's first O step);
  //   SZERO            S starts from zero (a block's first KV step);
  //   CHECK / SHIFT    the rare-path check; whether it also shifts S(t), -m;
  //   QPF              also stage the next block's Q (8 more loads);
  //   QSW              at the end, load the next block's Q into qop.
  //   kb, kk / vb, vk: base and KV step of the K / V block this step loads
  //                    (K of step t + 3, V of step t + 1, possibly of the
  //                    next block)
  template <int PAR, int KB, bool DO_S, bool DO_SM, bool DO_O, bool NEXT_S, bool NEXT_O,
            bool OZERO, bool SZERO, bool CHECK, bool SHIFT, bool QPF = false, bool QSW = false>
  __device__ __forceinline__ void step(int64_t kb, int kk, int64_t vb, int vk,
                                       int64_t nq_base = 0, int nq_qb = 0) {
    const uint16_t* Kc = w8_kbuf<KB>();
    const uint16_t* Vc = w8_vbuf<(KB + 2) % 4>();
    const f32x16 sp = sv;  // S(t - 1) - m, for the rare path
    bf16x8 kf[8], vf[8];
    auto issue = [&](auto xc) {
      constexpr int x = decltype(xc)::value;
      if constexpr (DO_S) kf[x] = kfrag(Kc, x);
      if constexpr (DO_O) vf[x] = vfrag(Vc, x >> 1, x & 1);
    };
    if constexpr (DO_S) { kf[0] = kpf[0]; kf[1] = kpf[1]; }
    if constexpr (DO_O) { vf[0] = vpf[0]; vf[1] = vpf[1]; }
    if constexpr (DO_S) {
      dma(p.K, kb, k_src, kk * W8_KV, w8_kbuf<(KB + 3) % 4>());
      dma(p.V, vb, v_src, vk * W8_KV, w8_vbuf<(KB + 1) % 4>());
    }
    if constexpr (QPF) stage_q(nq_base, nq_qb);
    __builtin_amdgcn_sched_barrier(0);
    sd_static_for<8>([&](auto xc) {
      constexpr int x = decltype(xc)::value;
      if constexpr (x == 0) __builtin_amdgcn_s_setprio(1);
      if constexpr (x == 6) __builtin_amdgcn_s_setprio(0);
      if constexpr (DO_S) {
        const f32x16 z = {};
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[x], qop[x],
                                                    x == 0 ? (SZERO ? z : negm) : s, 0, 0, 0);
      }
      if constexpr (DO_O) {
        const f32x16 z = {};
        o[x >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            vf[x], __builtin_bit_cast(bf16x8, pw[PAR][x & 1]),
            (OZERO && (x & 1) == 0) ? z : o[x >> 1], 0, 0, 0);
      }
      if constexpr (x + 2 < 8) issue(std::integral_constant<int, x + 2>());
      if constexpr (DO_SM) expo2<PAR ^ 1, x>();
      if constexpr (DO_S && x == 7) sv = s;  // the next step's softmax reads S(t)
      constexpr int nm = (DO_S ? 1 : 0) + (DO_O ? 1 : 0);
      constexpr int nv = DO_SM ? (kSectionValu[x] + nm - 1) / nm : 0;
      sd_static_for<nm>([&](auto) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        __builtin_amdgcn_sched_group_barrier(0x402, nv, 0); // its share of VALU
      });
      __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (DO_SM) {
      if constexpr (CHECK) {
        if (__builtin_expect(__any(rsum_ > kSumLimit), 0)) rescale<PAR ^ 1, SHIFT>(sp);
      }
      l += rsum_;
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (QSW) {
      bf16x8 x[NDC];
#pragma unroll
      for (int dc = 0; dc < NDC; ++dc) x[dc] = kfrag(w8Q[wave], dc);
      scale_q(x);
    }
    // the next step's first fragments: K(t + 1) and V(t - 1), published at
    // the previous barrier (their loads were issued two steps ago)
    if constexpr (NEXT_S) {
      kpf[0] = kfrag(w8_kbuf<(KB + 1) % 4>(), 0);
      kpf[1] = kfrag(w8_kbuf<(KB + 1) % 4>(), 1);
    }
    if constexpr (NEXT_O) {
      vpf[0] = vfrag(w8_vbuf<(KB + 3) % 4>(), 0, 0);
      vpf[1] = vfrag(w8_vbuf<(KB + 3) % 4>(), 0, 1);
    }
    __builtin_amdgcn_sched_barrier(0);
    // the previous step's loads landed (this step's may stay in flight), this
    // step's reads are done except the prefetch: publish / release
    // The count covers exactly the loads this step issued: a QPF step whose
    // block has no next block stages no Q (stage_q returns), and allowing 8
    // more would leave the previous step's K / V loads unwaited, which the
    // next step's fragment prefetch reads.
    constexpr int npf = (NEXT_S ? 2 : 0) + (NEXT_O ? 4 : 0);
    constexpr int nvm = DO_S ? 2 : 0;
    constexpr int nvq = nvm + (QPF ? 8 : 0);
    if (QPF && nq_qb >= 0)
      __builtin_amdgcn_s_waitcnt((nvq & 15) | ((nvq >> 4) << 14) | 0x0070 | (npf << 8));
    else
      __builtin_amdgcn_s_waitcnt((nvm & 15) | ((nvm >> 4) << 14) | 0x0070 | (npf << 8));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  }

  // a block's S(0) (raw) is in sv: m = its maximum, S(0) and -m rebased
  __device__ __forceinline__ void start_block() {
    m = xor32_max(max16(sv));
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sv[r] -= m;
      negm[r] = -m;
    }
  }
};

// Block jb of workgroup g is query block jb * G + perm(g): perm puts the
// workgroups of one XCD (g % 8 under round-robin dispatch) on consecutive
// blocks, so at any time an XCD works on the query blocks of one or two heads
// and its L2 serves their K / V to all of them.
__global__ __launch_bounds__(W8_THREADS, 1) void sdpa_w8_kernel(const SdpaArgs p) {
  SdpaW8 w{p};
  w.lane = threadIdx.x & 63;
  w.wave = threadIdx.x >> 6;
  w.l32 = w.lane & 31;
  w.h = w.lane >> 5;
  w.n = p.S / W8_KV;
  w.nqb = p.nqb;
  w.G = gridDim.x;
  w.g = blockIdx.x;
  const int total = p.nbh * p.nqb;
  w.nblk = (total - w.perm() + w.G - 1) / w.G;
  w.l = 0.0f;
  w.setup();
  const int n = w.n;  // >= 8, a multiple of 8
  int64_t cur_base;
  int cur_qb;
  w.block(0, cur_base, cur_qb);
  {
    bf16x8 x[SdpaW8::NDC];
    const int64_t q = static_cast<int64_t>(cur_qb) * W8_BQ + 32 * w.wave + w.l32;
#pragma unroll
    for (int dc = 0; dc < SdpaW8::NDC; ++dc)
      x[dc] = *reinterpret_cast<const bf16x8*>(p.Q + cur_base + q * W8_D + dc * 16 + 8 * w.h);
    w.scale_q(x);
  }
  // K(0), K(1), K(2) and V(0) of block 0 (with Q landed), then the pipeline
  w.dma(p.K, cur_base, w.k_src, 0, w8_kbuf<0>());
  w.dma(p.K, cur_base, w.k_src, W8_KV, w8_kbuf<1>());
  w.dma(p.K, cur_base, w.k_src, 2 * W8_KV, w8_kbuf<2>());
  w.dma(p.V, cur_base, w.v_src, 0, w8_vbuf<0>());
  __builtin_amdgcn_s_waitcnt(0x0070);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  w.kpf[0] = w.kfrag(w8_kbuf<0>(), 0);
  w.kpf[1] = w.kfrag(w8_kbuf<0>(), 1);
  //          PAR KB S  SM O  NS NO OZ SZ CK SH
  w.step<0, 0, 1, 0, 0, 1, 0, 0, 1, 0, 0>(cur_base, 3, cur_base, 1);
  w.start_block();
  w.step<1, 1, 1, 1, 0, 1, 1, 0, 0, 0, 0>(cur_base, 4, cur_base, 2);
  // one path per block: steps 2 .. n - 1 of block jb, then the next block's
  // steps 0 and 1, which also finish block jb (its last softmax and O
  // products) before its O is stored.  After the last block the "next"
  // block's steps run for nothing: their loads repeat the last block's last
  // K / V rows (still in L2), nothing reads them, and no Q is staged.
  for (int jb = 0;; ++jb) {
    const int64_t cb = cur_base;
    w.step<0, 2, 1, 1, 1, 1, 1, 1, 0, 1, 1>(cb, 5, cb, 3);
    w.step<1, 3, 1, 1, 1, 1, 1, 0, 0, 1, 1>(cb, 6, cb, 4);
    for (int i = 4; i + 4 < n; i += 4) {
      w.step<0, 0, 1, 1, 1, 1, 1, 0, 0, 1, 1>(cb, i + 3, cb, i + 1);
      w.step<1, 1, 1, 1, 1, 1, 1, 0, 0, 1, 1>(cb, i + 4, cb, i + 2);
      w.step<0, 2, 1, 1, 1, 1, 1, 0, 0, 1, 1>(cb, i + 5, cb, i + 3);
      w.step<1, 3, 1, 1, 1, 1, 1, 0, 0, 1, 1>(cb, i + 6, cb, i + 4);
    }
    const bool last = jb + 1 == w.nblk;
    int64_t nb = cb;
    int nq = -1;
    if (!last) w.block(jb + 1, nb, nq);
    const auto nk = [&](int k) { return last ? n - 1 : k; };  // KV step of the next block
    // steps n - 4 .. n - 1: the next block's first K / V blocks, its Q staged
    // and then loaded into qop
    w.step<0, 0, 1, 1, 1, 1, 1, 0, 0, 1, 1, true, false>(cb, n - 1, cb, n - 3, nb, nq);
    w.step<1, 1, 1, 1, 1, 1, 1, 0, 0, 1, 1>(nb, nk(0), cb, n - 2);
    w.step<0, 2, 1, 1, 1, 1, 1, 0, 0, 1, 1>(nb, nk(1), cb, n - 1);
    w.step<1, 3, 1, 1, 1, 1, 1, 0, 0, 1, 1, false, true>(nb, nk(2), nb, nk(0));
    // the next block's steps 0 and 1 with this block's last softmax / O
    w.step<0, 0, 1, 1, 1, 1, 1, 0, 1, 1, 0>(nb, nk(3), nb, nk(1));
    w.l_prev = w.l;
    w.l = 0.0f;
    w.start_block();
    w.step<1, 1, 1, 1, 1, 1, 1, 0, 0, 0, 0>(nb, nk(4), nb, nk(2));
    w.store_o(cb, cur_qb, w.l_prev);
    if (last) break;
    cur_base = nb;
    cur_qb = nq;
  }
  // the unused loads of the last block's "next" block land before the end
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
}

template <int D, bool CAUSAL>
int launch(const SdpaArgs& a, hipStream_t s) {
  if (D == W8_D && !CAUSAL && a.S % W8_BQ == 0) {
    SdpaArgs b = a;
    b.nqb = a.S / W8_BQ;
    // persistent: one workgroup per CU (at most), each walking its blocks
    int dev = 0, cus = 0;
    TTLH_HIP_CHECK(hipGetDevice(&dev));
    TTLH_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    TTLH_REQUIRE(cus > 0, TTLH_EHIP, "ttlh_sdpa_fwd: the device reports no CUs");
    const int64_t total = static_cast<int64_t>(b.nbh) * b.nqb;
    const int grid = static_cast<int>(total < cus ? total : cus);
    hipLaunchKernelGGL(sdpa_w8_kernel, dim3(grid), dim3(W8_THREADS), 0, s, b);
    return check_launch("sdpa_w8_kernel");
  }
  if (a.S % PP_BQ == 0) {
    SdpaArgs b = a;
    b.nqb = a.S / PP_BQ;
    hipLaunchKernelGGL((sdpa_pp_kernel<D, CAUSAL>), dim3(b.nbh * b.nqb), dim3(PP_THREADS), 0, s, b);
    return check_launch("sdpa_pp_kernel");
  }
  if (a.S % BQ != 0) {  // a ragged tail (S % 32 == 0)
    hipLaunchKernelGGL((sdpa_fwd_kernel<D, CAUSAL, true>), dim3(a.nbh * a.nqb), dim3(kThreads), 0,
                       s, a);
    return check_launch("sdpa_fwd_kernel");
  }
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
  TTLH_REQUIRE(S % 32 == 0, TTLH_EUNSUPPORTED, "ttlh_sdpa_fwd: seq_len must be a multiple of 32");
  TTLH_REQUIRE(B * H * ((S + BQ - 1) / BQ) < (int64_t(1) << 31), TTLH_EUNSUPPORTED,
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
  a.nqb = static_cast<int32_t>((S + BQ - 1) / BQ);
  a.nbh = static_cast<int32_t>(B * H);
  a.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (D == 128) return causal ? launch<128, true>(a, s) : launch<128, false>(a, s);
  return causal ? launch<64, true>(a, s) : launch<64, false>(a, s);
}
