// Fused elementwise / broadcast tile-program kernel for gfx950.
//
// What it replaces: the compute thread of a TTL elementwise kernel, whose
// tile ops run one 32x32 tile at a time in DST registers
// (include/ttlang/Dialect/TTL/TTLElementwiseOps.def:61-82), fed by reader /
// writer threads that move one tile per NoC request
// (lib/Dialect/TTL/Transforms/ConvertTTLToTTKernel.cpp:563-751); in the
// simulator, Block._binary_op / broadcast_tensors (python/sim/block.py:870-1010,
// python/sim/ttnnsim.py:67-109).
//
// MI355X design.  The whole output region is one grid-wide launch and the
// circular-buffer staging disappears: every lane owns 8 consecutive output
// elements, reads each operand's 8 elements with one 16-byte
// global_load_dwordx4 straight from HBM into VGPRs (all loads issued before
// any arithmetic), runs the tile program on them in fp32 (the DST-register
// analogue) and writes one non-temporal 16-byte store.  Broadcast operands
// (row vectors, column vectors, tiles re-used across the grid) are addressed
// through stride-0 / masked coordinates and hit in L2.
//
// The kernel is VALU-issue bound before it is HBM-bound unless every lane
// spends well under ~300 wave instructions per 8 elements (C2 runs 32 waves
// per SIMD and a wave64 VALU op occupies a SIMD for 4 cycles), so:
//  - the program is interpreted by a runtime step loop whose dispatch
//    fields sit in SGPRs (wave-uniform scalar branches, no VALU);
//  - operands are selected by a uniform switch on the consumption index, so
//    no register moves and no dynamic register indexing (which would spill
//    to scratch);
//  - addresses are 32-bit offsets when every tensor is < 2^31 elements and
//    the chunk -> (row, col) split is a multiply-high by a host-computed
//    magic number;
//  - bf16 rounding is one v_cvt_pk_bf16_f32 per element pair (hardware RNE);
//  - exp is v_exp_f32 with an FMA-split argument (about 1 fp32 ulp),
//    branch-free over the whole range;
//  - ops with long expansions (pow, fmod, log, tanh, division, ...) live in
//    separate "full" kernel variants so the common-op variants fit 8 waves
//    per SIMD (<= 64 VGPRs) without spilling.

#include <cstring>
#include <mutex>
#include <utility>

#include "ttlh_common.h"
#include "ttlh_eltprog.h"

namespace ttlh {
namespace {

// Occupancy target per variant: the stack-free bf16 fast path fits 6 waves
// per SIMD without spilling, the others 4-5.
// (the common-op bf16 variants fit 8 waves per SIMD, i.e. <= 64 VGPRs)
template <bool BF16, bool STACK, bool FULL>
constexpr int waves() {
  return FULL ? 4 : (BF16 ? (STACK ? 6 : 8) : 5);
}

// One lane computes 8 consecutive output elements (VEC = 8) or one (VEC = 1).
template <int VEC, bool PRELOAD, bool BF16, bool STACK, bool OFF32, bool FULL>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(waves<BF16, STACK, FULL>(), waves<BF16, STACK, FULL>())))
void eltwise_kernel(const EltArgs args) {
  const uint32_t chunk = blockIdx.x * 256u + threadIdx.x;
  if (chunk >= args.total) return;
  const uint32_t yr = divide(chunk, args.magic, args.shift);
  const uint32_t xr = chunk - yr * args.cpr;
  const int64_t y = args.y0 + yr;
  const int64_t x = args.x0 + static_cast<int64_t>(xr) * VEC;
  Raw q0{}, q1{}, q2{}, q3{};
  if constexpr (PRELOAD) {
    // addresses first (the descriptor reads batch into a few s_loads), then
    // the loads back to back; unused slots re-read operand 0 (a cache hit)
    const int n = args.n_ops;
    const uintptr_t p0 = operand_addr<OFF32>(args.ops[0], y, x);
    const uintptr_t p1 = n > 1 ? operand_addr<OFF32>(args.ops[1], y, x) : p0;
    const uintptr_t p2 = n > 2 ? operand_addr<OFF32>(args.ops[2], y, x) : p0;
    const uintptr_t p3 = n > 3 ? operand_addr<OFF32>(args.ops[3], y, x) : p0;
    q0 = load_raw<VEC, BF16>(args.ops[0], p0);
    q1 = load_raw<VEC, BF16>(args.ops[1], p1);
    q2 = load_raw<VEC, BF16>(args.ops[2], p2);
    q3 = load_raw<VEC, BF16>(args.ops[3], p3);
    asm volatile("" ::: "memory");  // all loads stay above the arithmetic
  }
  const f32x8 acc =
      run_program<VEC, PRELOAD, BF16, STACK, OFF32, FULL>(args, q0, q1, q2, q3, y, x);
  store_chunk<VEC>(args, y, x, acc);
}

template <int VEC, bool PRELOAD, bool BF16, bool STACK, bool OFF32, bool FULL>
int launch(const EltArgs& a, hipStream_t s) {
  const uint32_t blocks = (a.total + 255u) / 256u;
  hipLaunchKernelGGL((eltwise_kernel<VEC, PRELOAD, BF16, STACK, OFF32, FULL>), dim3(blocks),
                     dim3(256), 0, s, a);
  return check_launch("eltwise_kernel");
}

// ---------------------------------------------------------------------------
// Chain kernel: the fast path for linear programs, i.e. every step after the
// first LOAD combines acc with at most one operand or immediate (a + b,
// exp(a + b) * c, a * b + c, ...).  N steps are unrolled at compile time and
// step k statically owns operand slot k, so the operand a step reads is a
// fixed register: no per-step scalar loads, no operand switch, no stack.
// Slots of steps that read no operand are skipped by a uniform branch (one
// load path, so no register merge that would force an early s_waitcnt).
enum : uint8_t {
  C_ADD = 0, C_SUB, C_RSUB, C_MUL, C_EXP, C_NEG, C_ABS, C_RELU, C_RECIP, C_NONE
};
struct ChainArgs {
  EltOperand ops[TTLH_MAX_INSTR];  // slot k belongs to step k
  uint8_t code[TTLH_MAX_INSTR];    // C_* for steps 1..N-1
  uint8_t imm_src[TTLH_MAX_INSTR]; // 1: the step reads imm[k]; 2: it reads nothing
  uint8_t rnd[TTLH_MAX_INSTR];
  float imm[TTLH_MAX_INSTR];
  void* out;
  int64_t out_ld;
  int64_t y0, x0;
  uint32_t cpr, total, magic, shift;
  int32_t out_dtype;
};

__device__ __forceinline__ f32x8 chain_op(uint8_t code, f32x8 acc, f32x8 v) {
  switch (code) {
    case C_ADD: return acc + v;
    case C_SUB: return acc - v;
    case C_RSUB: return v - acc;
    case C_MUL: return acc * v;
    case C_EXP: return vexp_uniform(acc);
    case C_NEG: return -acc;
    case C_ABS: return map8(acc, [](float t) { return fabsf(t); });
    case C_RELU: return map8(acc, [](float t) { return relu1(t); });
    default: return 1.0f / acc;  // C_RECIP
  }
}

// Each lane runs U chunks, 256 chunks apart (a wave's loads stay 1 KiB
// contiguous per operand); every load of every chunk is issued before the
// first arithmetic.  Lanes past the end clamp their chunk index for the loads
// (an in-bounds re-read) and skip the store.
constexpr int kChainU = 1;

template <int N, bool BF16, bool ALLVEC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BF16 ? 8 : 6, BF16 ? 8 : 6)))
void chain_kernel(const ChainArgs args) {
  constexpr int U = kChainU;
  const uint32_t base = blockIdx.x * (256u * U) + threadIdx.x;
  int64_t y[U], x[U];
  Raw q[U][N];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t chunk = min(base + 256u * j, args.total - 1u);
    const uint32_t yr = divide(chunk, args.magic, args.shift);
    const uint32_t xr = chunk - yr * args.cpr;
    y[j] = args.y0 + yr;
    x[j] = args.x0 + static_cast<int64_t>(xr) * 8;
#pragma unroll
    for (int k = 0; k < N; ++k)
      if (k == 0 || args.imm_src[k] == 0)
        q[j][k] = load_raw<8, BF16>(args.ops[k], operand_addr<true>(args.ops[k], y[j], x[j]));
  }
  asm volatile("" ::: "memory");  // all loads stay above the arithmetic
#pragma unroll
  for (int j = 0; j < U; ++j) {
    f32x8 acc = to_f32<8, BF16, ALLVEC>(args.ops[0], q[j][0]);
#pragma unroll
    for (int k = 1; k < N; ++k) {
      f32x8 v = acc;
      if (args.imm_src[k] == 0) v = to_f32<8, BF16, ALLVEC>(args.ops[k], q[j][k]);
      else if (args.imm_src[k] == 1) v = splat(args.imm[k]);
      acc = chain_op(args.code[k], acc, v);
      // a bf16 rounding right before a bf16 store is the store's own RNE
      const bool last_into_bf16 = k == N - 1 && args.out_dtype == TTLH_BF16;
      if (args.rnd[k] == TTLH_BF16 && !last_into_bf16) acc = round_bf16x8(acc);
    }
    if (base + 256u * j < args.total) store_chunk<8>(args, y[j], x[j], acc);
  }
}

template <int N, bool BF16>
int launch_chain(const ChainArgs& a, hipStream_t s) {
  const uint32_t per_block = 256u * kChainU;
  const uint32_t blocks = (a.total + per_block - 1u) / per_block;
  bool allvec = true;
  for (int k = 0; k < N; ++k)
    if (k == 0 || a.imm_src[k] == 0) allvec &= a.ops[k].vec != 0;
  if (allvec)
    hipLaunchKernelGGL((chain_kernel<N, BF16, true>), dim3(blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((chain_kernel<N, BF16, false>), dim3(blocks), dim3(256), 0, s, a);
  return check_launch("chain_kernel");
}

constexpr int kMaxChain = 6;

// Builds ChainArgs when `prog` is a linear chain of common ops; returns false
// otherwise (the generic interpreter then runs it).
bool make_chain(const ttlh_instr* prog, int n, const EltArgs& e, ChainArgs* c) {
  if (n > kMaxChain || prog[0].form != TTLH_FORM_LOAD) return false;
  *c = ChainArgs{};
  int next = 0;
  c->ops[0] = e.ops[next++];
  for (int k = 1; k < n; ++k) {
    const ttlh_instr& p = prog[k];
    c->rnd[k] = p.rnd;
    c->imm[k] = p.imm;
    c->ops[k] = c->ops[0];  // (not loaded: steps without an operand skip their slot)
    const bool rev = p.form == TTLH_FORM_BIN_REV || p.form == TTLH_FORM_BIN_IMM_REV;
    switch (p.form) {
      case TTLH_FORM_UNARY:
        switch (p.op) {
          case TTLH_OP_EXP: c->code[k] = C_EXP; break;
          case TTLH_OP_NEG: c->code[k] = C_NEG; break;
          case TTLH_OP_ABS: c->code[k] = C_ABS; break;
          case TTLH_OP_RELU: c->code[k] = C_RELU; break;
          case TTLH_OP_RECIP: c->code[k] = C_RECIP; break;
          default: return false;
        }
        c->imm_src[k] = 2;
        break;
      case TTLH_FORM_BIN:
      case TTLH_FORM_BIN_REV:
      case TTLH_FORM_BIN_IMM:
      case TTLH_FORM_BIN_IMM_REV:
        switch (p.op) {
          case TTLH_OP_ADD: c->code[k] = C_ADD; break;
          case TTLH_OP_MUL: c->code[k] = C_MUL; break;
          case TTLH_OP_SUB: c->code[k] = rev ? C_RSUB : C_SUB; break;
          default: return false;
        }
        if (p.form == TTLH_FORM_BIN || p.form == TTLH_FORM_BIN_REV) c->ops[k] = e.ops[next++];
        else c->imm_src[k] = 1;
        break;
      default: return false;
    }
  }
  c->out = e.out;
  c->out_ld = e.out_ld;
  c->y0 = e.y0;
  c->x0 = e.x0;
  c->cpr = e.cpr;
  c->total = e.total;
  c->magic = e.magic;
  c->shift = e.shift;
  c->out_dtype = e.out_dtype;
  return true;
}

template <bool BF16>
int dispatch_chain(const ChainArgs& c, int n, hipStream_t s) {
  switch (n) {
    case 1: return launch_chain<1, BF16>(c, s);
    case 2: return launch_chain<2, BF16>(c, s);
    case 3: return launch_chain<3, BF16>(c, s);
    case 4: return launch_chain<4, BF16>(c, s);
    case 5: return launch_chain<5, BF16>(c, s);
    default: return launch_chain<6, BF16>(c, s);
  }
}

// ---------------------------------------------------------------------------
// Stream kernel: the chain kernel specialised for the common case — every
// operand bf16 and 8-wide (unit column stride, 16-byte aligned rows), at most
// 4 steps, 32-bit offsets, row indices and row strides below 2^24.  Which
// steps read an operand is a compile-time mask, so the loads form one
// straight block issued back to back; the grid is 2-D (lanes of a workgroup
// cover 1 << lsh chunks of a row, 256 >> lsh rows), so no division; the
// element offset of an operand is one 24-bit multiply-add.
struct StreamOp {
  const uint16_t* ptr;
  uint32_t rs, rmask, roff, cmask, coff, pad;
};
struct StreamArgs {
  StreamOp ops[4];
  uint8_t code[4];
  uint8_t rnd[4];
  float imm[4];
  void* out;
  uint32_t out_ld, y0, x0, h, cpr, lsh;
  int32_t out_dtype;
};

__device__ __forceinline__ f32x8 unpack_bf16x8(const u32x4 q) {
  return f32x8{__uint_as_float(q.x << 16), __uint_as_float(q.x & 0xffff0000u),
               __uint_as_float(q.y << 16), __uint_as_float(q.y & 0xffff0000u),
               __uint_as_float(q.z << 16), __uint_as_float(q.z & 0xffff0000u),
               __uint_as_float(q.w << 16), __uint_as_float(q.w & 0xffff0000u)};
}

template <int N, unsigned MASK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8, 8)))
void stream_kernel(const StreamArgs a) {
  const uint32_t t = threadIdx.x;
  uint32_t yr = blockIdx.y * (256u >> a.lsh) + (t >> a.lsh);
  uint32_t cr = (blockIdx.x << a.lsh) + (t & ((1u << a.lsh) - 1u));
  const bool live = yr < a.h && cr < a.cpr;
  yr = min(yr, a.h - 1u);  // dead lanes re-read an in-bounds chunk and store nothing
  cr = min(cr, a.cpr - 1u);
  const uint32_t y = a.y0 + yr;
  const uint32_t x = a.x0 + cr * 8u;
  u32x4 q[N];
#pragma unroll
  for (int k = 0; k < N; ++k)
    if ((MASK >> k) & 1u) {
      const StreamOp& o = a.ops[k];
      const uint32_t e = __umul24((y & o.rmask) + o.roff, o.rs) + (x & o.cmask) + o.coff;
      q[k] = *reinterpret_cast<gu32x4*>(reinterpret_cast<uintptr_t>(o.ptr + e));
    }
  // keep every load above this point: without it the compiler sinks a load
  // to its first use, past the arithmetic of the earlier steps, and the wave
  // then waits for memory twice
  asm volatile("" ::: "memory");
  f32x8 acc = unpack_bf16x8(q[0]);
#pragma unroll
  for (int k = 1; k < N; ++k) {
    const f32x8 v = ((MASK >> k) & 1u) ? unpack_bf16x8(q[k]) : splat(a.imm[k]);
    acc = chain_op(a.code[k], acc, v);
    const bool last_into_bf16 = k == N - 1 && a.out_dtype == TTLH_BF16;
    if (a.rnd[k] == TTLH_BF16 && !last_into_bf16) acc = round_bf16x8(acc);
  }
  if (!live) return;
  const uint32_t off = y * a.out_ld + x;
  if (a.out_dtype == TTLH_BF16) {
    u32x4 r;
    r.x = cvt_pk_bf16(acc[0], acc[1]);
    r.y = cvt_pk_bf16(acc[2], acc[3]);
    r.z = cvt_pk_bf16(acc[4], acc[5]);
    r.w = cvt_pk_bf16(acc[6], acc[7]);
    __builtin_nontemporal_store(r, reinterpret_cast<u32x4*>(static_cast<uint16_t*>(a.out) + off));
  } else {
    float* p = static_cast<float*>(a.out) + off;
    __builtin_nontemporal_store(f32x4{acc[0], acc[1], acc[2], acc[3]}, reinterpret_cast<f32x4*>(p));
    __builtin_nontemporal_store(f32x4{acc[4], acc[5], acc[6], acc[7]},
                                reinterpret_cast<f32x4*>(p + 4));
  }
}

// ---------------------------------------------------------------------------
// Flat kernel: the stream kernel's case when the output region is whole rows
// of the output and every operand is either a tensor of the output's row
// pitch read at the same element (chunk i of the region is chunk i of the
// operand) or one row of 8 * cpr elements re-read by every output row (a row
// vector, cpr a power of two).  Chunk i of the region is then base + 8 i in
// every array, so a lane's address is one 64-bit add off a 1-D index and
// there is no row / column split at all: on a 25 MB stream this saves about
// 0.35 us per launch over the 2-D stream kernel.
//
// The arguments the first loads need come first and as scalars: eltwise.hip
// is compiled with kernarg preloading of four arguments, so the first three
// operand bases and the chunk count are in SGPRs when the wave starts and
// the address arithmetic does not wait for a scalar load of the argument
// block (C1 add 4.58 -> 4.41 us, C2 15.66 -> 15.59 us; preloading all
// thirteen scalar dwords measured 4.39 / 15.68: each preloaded SGPR costs
// every wave's launch).  The rest, including the op codes needed only once
// the data is in, is fetched by s_load while the first loads are in flight.
struct FlatOps {
  uint8_t code[4];
  uint8_t rnd[4];
  float imm[4];
};

// A lane runs U chunks 256 apart: all loads first, then each step's op code
// is dispatched once for the lane's U accumulators, which halves the per-wave
// cost of the runtime op dispatch and of the argument loads (C2 15.9 -> 15.7
// us).  U = 1 for a plain copy (faster with one chunk per lane) and for four
// loaded operands (two chunks of each would not fit 64 VGPRs).
template <int N, unsigned MASK>
constexpr int flat_u() { return N > 1 && __builtin_popcount(MASK) < 4 ? 2 : 1; }

template <int U>
__device__ __forceinline__ void chain_op_u(uint8_t code, f32x8 (&acc)[U], const f32x8 (&v)[U]) {
  switch (code) {
#define TTLH_CHAIN_ALL(EXPR) _Pragma("unroll") for (int j = 0; j < U; ++j) acc[j] = EXPR; return;
    case C_ADD: TTLH_CHAIN_ALL(acc[j] + v[j])
    case C_SUB: TTLH_CHAIN_ALL(acc[j] - v[j])
    case C_RSUB: TTLH_CHAIN_ALL(v[j] - acc[j])
    case C_MUL: TTLH_CHAIN_ALL(acc[j] * v[j])
    case C_EXP: TTLH_CHAIN_ALL(vexp_uniform(acc[j]))
    default: TTLH_CHAIN_ALL(chain_op(code, acc[j], v[j]))
#undef TTLH_CHAIN_ALL
  }
}

// p0..p3: chunk 0 of the program's loaded operands in step order (the
// operand of step k is p[popcount(MASK & ((1 << k) - 1))], unused slots
// null); n: chunks in the region; bit c of bcast: p[c] is a row vector, read
// at chunk i & rowmask (rowmask = chunks per row - 1) instead of chunk i.
template <int N, unsigned MASK, bool OUT_BF16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8, 8)))
void flat_kernel(const u32x4* p0, const u32x4* p1, const u32x4* p2, uint32_t n, uint32_t bcast,
                 uint32_t rowmask, const u32x4* p3, void* out, const FlatOps a) {
  constexpr int U = flat_u<N, MASK>();
  const u32x4* const ptr[4] = {p0, p1, p2, p3};
  uint32_t i[U], q[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    i[j] = blockIdx.x * (256u * U) + 256u * j + threadIdx.x;
    q[j] = min(i[j], n - 1u);  // dead lanes re-read the last chunk and store nothing
  }
  u32x4 v[U][N];
#pragma unroll
  for (int k = 0; k < N; ++k)
    if ((MASK >> k) & 1u) {
      const int c = __builtin_popcount(MASK & ((1u << k) - 1u));
      const uint32_t im = ((bcast >> c) & 1u) ? rowmask : ~0u;
#pragma unroll
      for (int j = 0; j < U; ++j) v[j][k] = ptr[c][q[j] & im];
    }
  asm volatile("" ::: "memory");  // every load above the arithmetic (see stream_kernel)
  f32x8 acc[U];
#pragma unroll
  for (int j = 0; j < U; ++j) acc[j] = unpack_bf16x8(v[j][0]);
#pragma unroll
  for (int k = 1; k < N; ++k) {
    f32x8 x[U];
#pragma unroll
    for (int j = 0; j < U; ++j)
      x[j] = ((MASK >> k) & 1u) ? unpack_bf16x8(v[j][k]) : splat(a.imm[k]);
    chain_op_u<U>(a.code[k], acc, x);
    const bool last_into_bf16 = k == N - 1 && OUT_BF16;
    if (a.rnd[k] == TTLH_BF16 && !last_into_bf16)
#pragma unroll
      for (int j = 0; j < U; ++j) acc[j] = round_bf16x8(acc[j]);
  }
#pragma unroll
  for (int j = 0; j < U; ++j) {
    if (i[j] >= n) break;
    if constexpr (OUT_BF16) {
      u32x4 r;
      r.x = cvt_pk_bf16(acc[j][0], acc[j][1]);
      r.y = cvt_pk_bf16(acc[j][2], acc[j][3]);
      r.z = cvt_pk_bf16(acc[j][4], acc[j][5]);
      r.w = cvt_pk_bf16(acc[j][6], acc[j][7]);
      __builtin_nontemporal_store(r, static_cast<u32x4*>(out) + i[j]);
    } else {
      f32x4* p = static_cast<f32x4*>(out) + 2u * i[j];
      __builtin_nontemporal_store(f32x4{acc[j][0], acc[j][1], acc[j][2], acc[j][3]}, p);
      __builtin_nontemporal_store(f32x4{acc[j][4], acc[j][5], acc[j][6], acc[j][7]}, p + 1);
    }
  }
}

// Launches the flat kernel when `c` qualifies (see above); returns false to
// let the caller try the stream kernel.
bool try_flat(const ChainArgs& c, int n, hipStream_t s, int* status) {
  if (n > 4 || c.x0 != 0 || int64_t(c.cpr) * 8 != c.out_ld) return false;
  const bool pow2 = (c.cpr & (c.cpr - 1u)) == 0;
  const u32x4* ptr[4] = {};
  FlatOps a{};
  unsigned mask = 0, bcast = 0;
  for (int k = 0; k < n; ++k) {
    const bool reads = k == 0 || c.imm_src[k] == 0;
    if (reads) {
      const EltOperand& o = c.ops[k];
      if (o.dtype != TTLH_BF16 || !o.vec || o.cs != 1 || o.cmask != -1) return false;
      const uint16_t* p = static_cast<const uint16_t*>(o.ptr);
      const int ci = __builtin_popcount(mask);
      if (o.rmask == -1 && o.rs == c.out_ld) {  // same element as the output
        ptr[ci] = reinterpret_cast<const u32x4*>(p + (c.y0 + o.roff) * o.rs + o.coff);
      } else if ((o.rmask == 0 || o.rs == 0) && pow2) {  // one row, re-read by every row
        const int64_t row = o.rs == 0 ? 0 : o.roff;
        ptr[ci] = reinterpret_cast<const u32x4*>(p + row * o.rs + o.coff);
        bcast |= 1u << ci;
      } else {
        return false;
      }
      mask |= 1u << k;
    }
    a.code[k] = c.code[k];
    a.rnd[k] = c.rnd[k];
    a.imm[k] = c.imm[k];
  }
  const int esz = c.out_dtype == TTLH_BF16 ? 2 : 4;
  void* const out = static_cast<char*>(c.out) + c.y0 * c.out_ld * esz;
  const uint32_t rowmask = c.cpr - 1u;
#define TTLH_FLAT_CASE(NN, MM)                                                         \
  case (NN << 4) | MM: {                                                                \
    const dim3 grid((c.total + 256u * flat_u<NN, MM>() - 1u) / (256u * flat_u<NN, MM>())); \
    if (c.out_dtype == TTLH_BF16)                                                       \
      hipLaunchKernelGGL((flat_kernel<NN, MM, true>), grid, dim3(256), 0, s, ptr[0], ptr[1], \
                         ptr[2], c.total, bcast, rowmask, ptr[3], out, a);               \
    else                                                                                \
      hipLaunchKernelGGL((flat_kernel<NN, MM, false>), grid, dim3(256), 0, s, ptr[0], ptr[1], \
                         ptr[2], c.total, bcast, rowmask, ptr[3], out, a);               \
    break;                                                                              \
  }
  switch ((n << 4) | mask) {
    TTLH_FLAT_CASE(1, 1)
    TTLH_FLAT_CASE(2, 1) TTLH_FLAT_CASE(2, 3)
    TTLH_FLAT_CASE(3, 1) TTLH_FLAT_CASE(3, 3) TTLH_FLAT_CASE(3, 5) TTLH_FLAT_CASE(3, 7)
    TTLH_FLAT_CASE(4, 1) TTLH_FLAT_CASE(4, 3) TTLH_FLAT_CASE(4, 5) TTLH_FLAT_CASE(4, 7)
    TTLH_FLAT_CASE(4, 9) TTLH_FLAT_CASE(4, 11) TTLH_FLAT_CASE(4, 13) TTLH_FLAT_CASE(4, 15)
    default: return false;
  }
#undef TTLH_FLAT_CASE
  *status = check_launch("flat_kernel");
  return true;
}

// Launches the stream kernel when `c` qualifies (see above); returns false
// to let the caller fall back to the chain kernel.
// (Only called where every operand and output offset over the region fits
// 31 bits, which the kernel's 32-bit element offsets need.)
bool try_stream(const ChainArgs& c, int n, hipStream_t s, int* status) {
  if (n > 4 || c.out_ld >= (int64_t(1) << 31)) return false;
  StreamArgs a{};
  unsigned mask = 0;
  for (int k = 0; k < n; ++k) {
    const bool reads = k == 0 || c.imm_src[k] == 0;
    if (reads) {
      const EltOperand& o = c.ops[k];
      if (o.dtype != TTLH_BF16 || !o.vec || o.rs >= (int64_t(1) << 24)) return false;
      const int64_t ymax = mask_max(o.rmask, c.y0 + int64_t(c.total / c.cpr) - 1) + o.roff;
      if (ymax >= (int64_t(1) << 24)) return false;
      mask |= 1u << k;
      a.ops[k] = StreamOp{static_cast<const uint16_t*>(o.ptr), static_cast<uint32_t>(o.rs),
                          static_cast<uint32_t>(o.rmask), static_cast<uint32_t>(o.roff),
                          static_cast<uint32_t>(o.cmask), static_cast<uint32_t>(o.coff), 0};
    }
    a.code[k] = c.code[k];
    a.rnd[k] = c.rnd[k];
    a.imm[k] = c.imm[k];
  }
  const uint32_t h = c.total / c.cpr;
  uint32_t lsh = 0;
  while (lsh < 8 && (1u << lsh) < c.cpr) ++lsh;
  // narrower row blocks (down to 32 chunks, 512 contiguous bytes) where the
  // last block of each row would otherwise hold many dead lanes: 384 chunks
  // per row take three blocks of 128, not two of 256 with 128 dead (C2's
  // program at 4096 x 3072: 15.8 -> 14.7 us)
  while (lsh > 5) {
    const uint32_t bw = 1u << lsh, nb = (c.cpr + bw - 1u) / bw;
    if (nb * bw - c.cpr <= c.cpr / 8u) break;
    --lsh;
  }
  const uint32_t gx = (c.cpr + (1u << lsh) - 1u) >> lsh;
  const uint32_t rpb = 256u >> lsh;
  const uint32_t gy = (h + rpb - 1u) / rpb;
  if (gy > 65535u) return false;
  a.out = c.out;
  a.out_ld = static_cast<uint32_t>(c.out_ld);
  a.y0 = static_cast<uint32_t>(c.y0);
  a.x0 = static_cast<uint32_t>(c.x0);
  a.h = h;
  a.cpr = c.cpr;
  a.lsh = lsh;
  a.out_dtype = c.out_dtype;
  const dim3 grid(gx, gy), block(256);
#define TTLH_STREAM_CASE(NN, MM)                                                   \
  case (NN << 4) | MM:                                                              \
    hipLaunchKernelGGL((stream_kernel<NN, MM>), grid, block, 0, s, a);             \
    break;
  switch ((n << 4) | mask) {
    TTLH_STREAM_CASE(1, 1)
    TTLH_STREAM_CASE(2, 1) TTLH_STREAM_CASE(2, 3)
    TTLH_STREAM_CASE(3, 1) TTLH_STREAM_CASE(3, 3) TTLH_STREAM_CASE(3, 5) TTLH_STREAM_CASE(3, 7)
    TTLH_STREAM_CASE(4, 1) TTLH_STREAM_CASE(4, 3) TTLH_STREAM_CASE(4, 5) TTLH_STREAM_CASE(4, 7)
    TTLH_STREAM_CASE(4, 9) TTLH_STREAM_CASE(4, 11) TTLH_STREAM_CASE(4, 13) TTLH_STREAM_CASE(4, 15)
    default: return false;
  }
#undef TTLH_STREAM_CASE
  *status = check_launch("stream_kernel");
  return true;
}

// ---------------------------------------------------------------------------
// Scaled reductions (ttlh_reduce).  The tile program runs through the generic
// interpreter (all ops, mixed dtypes, 64-bit addressing); each element is
// multiplied by the scale and combined in fp32.
//  * rows (reduce over columns): one wave per iteration row, lane l takes the
//    8-element chunks l, l + 64, ... of the row, then an xor-shuffle tree;
//  * columns (reduce over rows): lane l of every wave takes the same 8
//    columns, wave w rows w, w + 4, ... of the block's row split; the four
//    waves combine through LDS; with several splits the fp32 partials go to
//    the workspace and a second pass combines them in split order;
//  * both: the row kernel writes one fp32 value per row to the workspace and
//    one workgroup combines them.
struct RedArgs {
  EltArgs e;             // program and operands; e.y0 / e.x0 = iteration origin
  int64_t h, w;          // iteration region
  const void* scaler;
  int32_t scaler_dtype;
  float scale_imm;
  void* out;
  int64_t out_ld;
  int32_t out_dtype, out_pad;
  float* ws;
  int64_t rows_per_split;
  int32_t kind, splits;
};

__device__ __forceinline__ float red_identity(int kind) {
  return kind == TTLH_REDUCE_MAX ? -__builtin_inff() : 0.0f;
}

__device__ __forceinline__ float red_combine(int kind, float a, float b) {
  if (kind == TTLH_REDUCE_MAX) return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
  return a + b;
}

// One value v, scaled by s, into a running reduction r: a sum adds v * s with
// one rounding (a fused multiply-add, written out so that every kernel
// rounds the same way whatever the compiler would contract), a maximum takes
// the rounded product.
__device__ __forceinline__ float red_acc(int kind, float r, float v, float s) {
  return kind == TTLH_REDUCE_MAX ? red_combine(kind, r, v * s) : __builtin_fmaf(v, s, r);
}

// The scaler value through a 32-bit load of its (4-byte aligned, so in-bounds)
// dword: a uniform 32-bit load compiles to s_load_dword, which the row loads
// do not wait behind; a 16-bit load is a vector load whose vmcnt(0) wait
// sat in front of every workgroup's first row load (9.7 -> 7 us on a
// 4096 x 4096 row sum).
__device__ __forceinline__ float red_scale(const RedArgs& a) {
  float s = a.scale_imm;
  if (a.scaler) {
    const uintptr_t u = reinterpret_cast<uintptr_t>(a.scaler);
    const uint32_t w =
        *reinterpret_cast<const __attribute__((address_space(1))) uint32_t*>(u & ~uintptr_t(3));
    s *= a.scaler_dtype == TTLH_BF16 ? __uint_as_float((u & 2) ? (w & 0xffff0000u) : (w << 16))
                                     : __uint_as_float(w);
  }
  return s;
}

__device__ __forceinline__ void red_store(const RedArgs& a, int64_t off, float v) {
  if (a.out_dtype == TTLH_BF16)
    static_cast<uint16_t*>(a.out)[off] = f32_to_bf16(v);
  else
    static_cast<float*>(a.out)[off] = v;
}

// result `idx` of a row reduce (DIM1) / column reduce (DIM0), with the zero
// padding of the result tile when out_pad is set
template <int DIMS>
__device__ __forceinline__ void red_write(const RedArgs& a, int64_t idx, float v) {
  if constexpr (DIMS == TTLH_REDUCE_DIM1) {
    const int64_t off = idx * a.out_ld;
    red_store(a, off, v);
    if (a.out_pad)
      for (int c = 1; c < 32; ++c) red_store(a, off + c, 0.0f);
  } else {
    red_store(a, idx, v);
    if (a.out_pad)
      for (int r = 1; r < 32; ++r) red_store(a, idx + r * a.out_ld, 0.0f);
  }
}

__device__ __forceinline__ float red_wave(int kind, float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = red_combine(kind, v, __shfl_xor(v, off, 64));
  return v;
}

// Kernel variants of the reductions (MODE):
//   0: the generic loop, loads inside the program (any operand count and
//      alignment, VEC 8 or 1, every op);
//   1: plain (the program is one LOAD step: the operand itself);
//   2: up to four operands, common ops (add sub mul exp neg abs relu recip).
// Modes 1 and 2 read 8-wide chunks in a four-deep software pipeline (chunk
// k + 4 is fetched as soon as chunk k is consumed, so four loads per lane
// stay in flight; nothing is fetched past the end: a wave does not wait on
// loads whose values it never reads).
// Programs with other ops take mode 0: four inlined copies of the every-op
// interpreter (pow, fmod, log, ...) would overflow the instruction cache.
struct RedChunk {
  Raw q0, q1, q2, q3;
};

template <int MODE>
__device__ __forceinline__ RedChunk red_fetch(const EltArgs& e, int64_t y, int64_t x) {
  RedChunk c;
  const uintptr_t p0 = operand_addr<false>(e.ops[0], y, x);
  c.q0 = load_raw<8, false>(e.ops[0], p0);
  if constexpr (MODE >= 2) {  // unused slots re-read operand 0 (a cache hit)
    const int n = e.n_ops;
    const uintptr_t p1 = n > 1 ? operand_addr<false>(e.ops[1], y, x) : p0;
    const uintptr_t p2 = n > 2 ? operand_addr<false>(e.ops[2], y, x) : p0;
    const uintptr_t p3 = n > 3 ? operand_addr<false>(e.ops[3], y, x) : p0;
    c.q1 = load_raw<8, false>(e.ops[1], p1);
    c.q2 = load_raw<8, false>(e.ops[2], p2);
    c.q3 = load_raw<8, false>(e.ops[3], p3);
  }
  return c;
}

template <int MODE>
__device__ __forceinline__ f32x8 red_eval(const EltArgs& e, const RedChunk& c, int64_t y,
                                          int64_t x) {
  if constexpr (MODE == 1) {
    const f32x8 v = to_f32<8, false>(e.ops[0], c.q0);
    return e.prog[0].rnd == TTLH_BF16 ? round_bf16x8(v) : v;
  } else {
    return run_program<8, true, false, true, false, false>(e, c.q0, c.q1, c.q2, c.q3, y, x);
  }
}

// pipeline depth: the plain mode keeps all eight chunks of a 4096-wide row
// in flight per lane, the interpreting mode four (register budget)
template <int MODE>
constexpr int red_depth() {
  return MODE == 1 ? 8 : 4;
}

// f(integral_constant<int, i>) for i = 0 .. N-1, unrolled at compile time
// (constant indices keep the chunk arrays in registers)
template <typename F, int... I>
__device__ __forceinline__ void red_unroll(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>()), ...);
}

template <int VEC, bool TO_WS, int MODE>
__global__ __launch_bounds__(256) void reduce_rows_kernel(const RedArgs a) {
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= a.h) return;  // wave-uniform
  const int64_t y = a.e.y0 + row;
  float r = red_identity(a.kind);
  if constexpr (MODE == 0) {
    const float s = red_scale(a);
    const Raw q{};
    for (int64_t xo = int64_t(lane) * VEC; xo < a.w; xo += 64 * VEC) {
      const f32x8 v =
          run_program<VEC, false, false, true, false, true>(a.e, q, q, q, q, y, a.e.x0 + xo);
#pragma unroll
      for (int k = 0; k < VEC; ++k) r = red_acc(a.kind, r, v[k], s);
    }
  } else {
    constexpr int D = red_depth<MODE>();
    constexpr int64_t S = 64 * 8;
    const int64_t xf = int64_t(lane) * 8;
    if (xf < a.w) {
      RedChunk c[D];  // chunk slots past the row's end are neither fetched nor read
      red_unroll([&](auto i) {
        if (xf + i * S < a.w) c[i] = red_fetch<MODE>(a.e, y, a.e.x0 + xf + i * S);
      }, std::make_integer_sequence<int, D>());
      const float s = red_scale(a);  // after the first row loads are in flight
      for (int64_t xb = xf; xb < a.w; xb += D * S) {
        red_unroll([&](auto i) {
          const int64_t xo = xb + i * S;
          if (xo < a.w) {
            const f32x8 v = red_eval<MODE>(a.e, c[i], y, a.e.x0 + xo);
#pragma unroll
            for (int k = 0; k < 8; ++k) r = red_acc(a.kind, r, v[k], s);
          }
          if (xo + D * S < a.w) c[i] = red_fetch<MODE>(a.e, y, a.e.x0 + xo + D * S);
        }, std::make_integer_sequence<int, D>());
      }
    }
  }
  r = red_wave(a.kind, r);
  if (lane == 0) {
    if constexpr (TO_WS) a.ws[row] = r;
    else red_write<TTLH_REDUCE_DIM1>(a, row, r);
  }
}

// Row reduce of wide rows (w >= 2048, MODE 1 / 2): one workgroup per row, so
// a row's reads spread over four waves (a quarter of the chunks each, two
// chunks per lane in flight) and 4x as many waves hide each other's latency;
// the four wave results combine through LDS in wave order.
template <bool TO_WS, int MODE>
__global__ __launch_bounds__(256) void reduce_rows_wide_kernel(const RedArgs a) {
  __shared__ float part[4];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t y = a.e.y0 + row;
  constexpr int64_t S = 256 * 8;
  const int64_t xf = int64_t(t) * 8;  // a.w >= 2048: every lane has a chunk
  RedChunk c[2];  // chunk slots past the row's end are neither fetched nor read
  red_unroll([&](auto i) {
    if (xf + i * S < a.w) c[i] = red_fetch<MODE>(a.e, y, a.e.x0 + xf + i * S);
  }, std::make_integer_sequence<int, 2>());
  const float s = red_scale(a);  // after the first row loads are in flight
  float r = red_identity(a.kind);
  for (int64_t xb = xf; xb < a.w; xb += 2 * S) {
    red_unroll([&](auto i) {
      const int64_t xo = xb + i * S;
      if (xo < a.w) {
        const f32x8 v = red_eval<MODE>(a.e, c[i], y, a.e.x0 + xo);
#pragma unroll
        for (int k = 0; k < 8; ++k) r = red_acc(a.kind, r, v[k], s);
      }
      if (xo + 2 * S < a.w) c[i] = red_fetch<MODE>(a.e, y, a.e.x0 + xo + 2 * S);
    }, std::make_integer_sequence<int, 2>());
  }
  r = red_wave(a.kind, r);
  if (lane == 0) part[wave] = r;
  __syncthreads();
  if (t != 0) return;
  r = red_combine(a.kind, red_combine(a.kind, part[0], part[1]),
                  red_combine(a.kind, part[2], part[3]));
  if constexpr (TO_WS) a.ws[row] = r;
  else red_write<TTLH_REDUCE_DIM1>(a, row, r);
}

// Row reduce of the commonest program, one plain bf16 operand over rows of
// at least 2048 elements (the wide kernel's layout: one workgroup per row,
// lane t reads 16-byte chunks t, t + 256, ..., two in flight), with the
// reduction kind a template parameter and nothing interpreted per element:
// bf16 values are exact in fp32 and the operand's bf16 rounding is the
// identity on them.  NT: streaming loads, chosen by the host when the
// operand is read exactly once (no row stride 0).  4096 x 4096 row sum: 6.5
// us against 8.4 us through the wide kernel.  Element x of row r is at
// base[r rs + x]: the operand has no row or column mask (the host sends
// masked operands to the wide kernel), and base / rs / w lead the argument
// list as scalars, preloaded into SGPRs like the flat kernel's.  PROD: the
// program is a * b of two such bf16 operands (b at base2[r rs2 + x]), the
// product rounded to bf16 as the simulator materialises it, then reduced:
// the fused row kernel's chain for that program, element for element and in
// its summation order, so the bits are the same (4096 x 4096 row dot
// products: 14.0 us against 16.2 us there).
template <int KIND>
__device__ __forceinline__ float red_combine_k(float a, float b) {
  if constexpr (KIND == TTLH_REDUCE_MAX) return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
  else return a + b;
}
template <int KIND>
__device__ __forceinline__ float red_acc_k(float r, float v, float s) {
  if constexpr (KIND == TTLH_REDUCE_MAX) return red_combine_k<KIND>(r, v * s);
  else return __builtin_fmaf(v, s, r);
}

template <bool NT>
__device__ __forceinline__ u32x4 ld16(uintptr_t u) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<gu32x4*>(u));
  else return *reinterpret_cast<gu32x4*>(u);
}

template <int KIND, bool TO_WS, bool NT, bool PROD = false>
__global__ __launch_bounds__(256) void reduce_rows_bf16_kernel(const uint16_t* base, int64_t rs,
                                                               int64_t w, const RedArgs a,
                                                               const uint16_t* base2 = nullptr,
                                                               int64_t rs2 = 0) {
  __shared__ float part[4];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uintptr_t rowp = reinterpret_cast<uintptr_t>(base + row * rs);
  const uintptr_t rowq = PROD ? reinterpret_cast<uintptr_t>(base2 + row * rs2) : 0;
  constexpr int64_t S = 256 * 8;
  const int64_t xf = int64_t(t) * 8;
  u32x4 c[2], d[2];  // chunk slots past the row's end are neither fetched nor read
#pragma unroll
  for (int i = 0; i < 2; ++i)
    if (xf + i * S < w) {
      c[i] = ld16<NT>(rowp + 2 * (xf + i * S));
      if constexpr (PROD) d[i] = ld16<NT>(rowq + 2 * (xf + i * S));
    }
  const float s = red_scale(a);  // after the first row loads are in flight
  float r = red_identity(KIND);
  bool nan = false;  // maximum: whether a value was a NaN, kept apart from fmaxf
  for (int64_t xb = xf; xb < w; xb += 2 * S) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t xo = xb + i * S;
      if (xo < w) {
        f32x8 v = unpack_bf16x8(c[i]);
        if constexpr (PROD) v = round_bf16x8(binary8<TTLH_OP_MUL>(v, unpack_bf16x8(d[i])));
        if constexpr (KIND == TTLH_REDUCE_MAX) {
          // red_acc_k's value: fmaxf over the products, NaN once any is
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const float b = v[k] * s;
            nan |= b != b;
            r = fmaxf(r, b);
          }
        } else {
#pragma unroll
          for (int k = 0; k < 8; ++k) r = red_acc_k<KIND>(r, v[k], s);
        }
      }
      if (xo + 2 * S < w) {
        c[i] = ld16<NT>(rowp + 2 * (xo + 2 * S));
        if constexpr (PROD) d[i] = ld16<NT>(rowq + 2 * (xo + 2 * S));
      }
    }
  }
  if (nan) r = __builtin_nanf("");
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) r = red_combine_k<KIND>(r, __shfl_xor(r, off, 64));
  if (lane == 0) part[wave] = r;
  __syncthreads();
  if (t != 0) return;
  r = red_combine_k<KIND>(red_combine_k<KIND>(part[0], part[1]),
                          red_combine_k<KIND>(part[2], part[3]));
  if constexpr (TO_WS) a.ws[row] = r;
  else red_write<TTLH_REDUCE_DIM1>(a, row, r);
}

// Column reduce; MODE as for the row reduce (the pipeline runs over the
// wave's rows: rows r, r + 4, ... in flight).
template <int VEC, int MODE>
__global__ __launch_bounds__(256) void reduce_cols_kernel(const RedArgs a) {
  __shared__ float part[3][64 * VEC];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t xo = (int64_t(blockIdx.x) * 64 + lane) * VEC;  // this lane's first column
  const int64_t rb = int64_t(blockIdx.y) * a.rows_per_split;
  const int64_t re = rb + a.rows_per_split < a.h ? rb + a.rows_per_split : a.h;
  const float s = red_scale(a);
  const bool active = xo < a.w;  // VEC = 8 needs w % 8 == 0: all 8 columns valid
  float acc[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) acc[k] = red_identity(a.kind);
  if (active) {
    if constexpr (MODE == 0) {
      const Raw q{};
      for (int64_t row = rb + wave; row < re; row += 4) {
        const f32x8 v = run_program<VEC, false, false, true, false, true>(
            a.e, q, q, q, q, a.e.y0 + row, a.e.x0 + xo);
#pragma unroll
        for (int k = 0; k < VEC; ++k) acc[k] = red_acc(a.kind, acc[k], v[k], s);
      }
    } else {
      constexpr int D = red_depth<MODE>();
      const int64_t rf = rb + wave;
      if (rf < re) {
        const int64_t x = a.e.x0 + xo;
        RedChunk c[D];  // slots past the last row are neither fetched nor read
        red_unroll([&](auto i) {
          if (rf + 4 * i < re) c[i] = red_fetch<MODE>(a.e, a.e.y0 + rf + 4 * i, x);
        }, std::make_integer_sequence<int, D>());
        for (int64_t rr = rf; rr < re; rr += 4 * D) {
          red_unroll([&](auto i) {
            const int64_t row = rr + 4 * i;
            if (row < re) {
              const f32x8 v = red_eval<MODE>(a.e, c[i], a.e.y0 + row, x);
#pragma unroll
              for (int k = 0; k < VEC; ++k) acc[k] = red_acc(a.kind, acc[k], v[k], s);
            }
            if (row + 4 * D < re) c[i] = red_fetch<MODE>(a.e, a.e.y0 + row + 4 * D, x);
          }, std::make_integer_sequence<int, D>());
        }
      }
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int k = 0; k < VEC; ++k) part[wave - 1][lane * VEC + k] = acc[k];
  }
  __syncthreads();
  if (wave != 0 || !active) return;
#pragma unroll
  for (int k = 0; k < VEC; ++k) {
#pragma unroll
    for (int w = 0; w < 3; ++w) acc[k] = red_combine(a.kind, acc[k], part[w][lane * VEC + k]);
    if (a.splits == 1) red_write<TTLH_REDUCE_DIM0>(a, xo + k, acc[k]);
    else a.ws[int64_t(blockIdx.y) * a.w + xo + k] = acc[k];
  }
}

// p[0], p[stride], ..., p[(n - 1) stride] combined in that order, eight
// loads in flight
__device__ __forceinline__ float red_strided(int kind, const float* p, int64_t n, int64_t stride) {
  float r = red_identity(kind);
  int64_t i = 0;
  for (; i + 8 <= n; i += 8) {
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = p[(i + k) * stride];
#pragma unroll
    for (int k = 0; k < 8; ++k) r = red_combine(kind, r, v[k]);
  }
  for (; i < n; ++i) r = red_combine(kind, r, p[i * stride]);
  return r;
}

// Column reduce, several splits: a workgroup takes 32 columns; its eight
// thread groups combine the splits g, g + 8, ... of their column, then group
// 0 combines the eight results (fixed order throughout).
__global__ __launch_bounds__(256) void reduce_cols_finish_kernel(const RedArgs a) {
  __shared__ float part[8][32];
  const int t = threadIdx.x, c = t & 31, g = t >> 5;
  const int64_t col = int64_t(blockIdx.x) * 32 + c;
  float r = red_identity(a.kind);
  if (col < a.w && g < a.splits)
    r = red_strided(a.kind, a.ws + int64_t(g) * a.w + col, (a.splits - g + 7) / 8, 8 * a.w);
  part[g][c] = r;
  __syncthreads();
  if (g != 0 || col >= a.w) return;
#pragma unroll
  for (int k = 1; k < 8; ++k) r = red_combine(a.kind, r, part[k][c]);
  red_write<TTLH_REDUCE_DIM0>(a, col, r);
}

// full reduce: one workgroup combines the h row values (thread t: rows t,
// t + 256, ... in order, then a fixed tree) and writes the result tile
__global__ __launch_bounds__(256) void reduce_all_finish_kernel(const RedArgs a) {
  __shared__ float part[256];
  const int t = threadIdx.x;
  part[t] = t < a.h ? red_strided(a.kind, a.ws + t, (a.h - t + 255) / 256, 256)
                    : red_identity(a.kind);
  __syncthreads();
  for (int n = 128; n >= 1; n >>= 1) {
    if (t < n) part[t] = red_combine(a.kind, part[t], part[t + n]);
    __syncthreads();
  }
  if (t == 0) red_store(a, 0, part[0]);
  if (a.out_pad) {
    for (int i = t; i < 32 * 32; i += 256)
      if (i != 0) red_store(a, int64_t(i >> 5) * a.out_ld + (i & 31), 0.0f);
  }
}

// ---------------------------------------------------------------------------
// Row reductions and the elementwise program that reads their results, in one
// launch (ttlh_reduce_rows_eltwise).  A workgroup (rows of w >= 2048) or a
// wave (w < 2048) takes one row: it loads the row's chunks of the resident
// operands (identity-mapped bf16 operands) into registers once, runs every
// reduction stage over them in the summation order of the row-reduction
// kernels above (lane l accumulates its chunks l, l + L, l + 2L, ... in
// order, L = the lanes of the row; then the wave's butterfly; then, for a
// workgroup, the wave partials as (p0 + p1) + (p2 + p3)), writes each result
// where ttlh_reduce writes it, and hands it, rounded to its dtype, to the
// later stages as the row's scalar; then runs the elementwise stage over the
// same chunks.  Results are those of the separate ttlh_reduce and
// ttlh_eltwise calls, bit for bit.

constexpr int kRfRed = 3;     // reduction stages, at most
constexpr int kRfRes = 3;     // resident operands, at most
constexpr int kRfMem = 4;     // operands loaded at every use, at most
constexpr int kRfChunks = 4;  // 8-element chunks of a row per lane, at most
constexpr int kRfRow = 4;     // operands constant along a row (read once per row), at most
constexpr int kRfNodes = 8;   // row values a stage derives from earlier results, at most
constexpr int kRfNode0 = kRfRed + kRfRow;   // a row's scalars: reduction results, row
constexpr int kRfScal = kRfNode0 + kRfNodes;  // operands, then derived values

// Each stage's program is compiled on the host into a chain over the row's
// elements, acc = op(acc, operand) or op(acc) step by step, whose operands
// are resident rows, other operands, immediates or row scalars: the
// reductions' results, operands constant along the row (a column broadcast,
// read once per row) and values derived from those alone (recip of a row
// sum, a mean plus epsilon under rsqrt), which are computed once per row.
enum : uint8_t {
  RC_ADD, RC_SUB, RC_RSUB, RC_MUL, RC_DIV, RC_RDIV, RC_MAX, RC_RMAX, RC_MIN,  // binary: op(acc, v)
  RC_RMIN,                                   // (R*: op(v, acc))
  RC_EXP, RC_SQRT, RC_RSQRT, RC_ABS, RC_NEG, RC_RELU, RC_RECIP, RC_COPY       // unary
};
// operand sources
enum : uint8_t { RS_RES = 0x00, RS_MEM = 0x10, RS_SC = 0x20, RS_IMM = 0x30 };

struct RfStep {    // one chain step; step 0 is RC_COPY of the chain's first value
  uint8_t code;    // RC_*
  uint8_t src;     // binary steps and step 0: the operand (RS_* + index)
  uint8_t rnd;     // TTLH_BF16: the result is rounded to bf16
  uint8_t orn;     // TTLH_BF16: the operand is rounded to bf16 before use
  float imm;       // RS_IMM operand
};

struct RfNode {    // row scalar kRfNode0 + i = code(a, b) (unary: code(a); R*: op(b, a)), rounded
  uint8_t code, a, b, rnd;  // a, b: RS_SC + slot or RS_IMM
  float imm_a, imm_b;
};

struct RfStage {
  RfStep step[TTLH_MAX_INSTR];
  RfNode node[kRfNodes];
  int32_t n_steps, n_nodes;
  int32_t from_kept;  // > 0: the chain's first from_kept steps are the kept stage's chain
  int32_t kind, out_dtype, out_pad, scaler_dtype;  // reduction stages only from here
  float scale_imm;
  const void* scaler;
  void* out;  // result of region row r at out[r * out_ld]
  int64_t out_ld;
};

struct RfArgs {
  RfStage st[kRfRed + 1];  // the reductions, then (at kRfRed) the elementwise stage
  EltOperand mem[kRfMem];
  EltOperand res[kRfRes];
  EltOperand row[kRfRow];  // row scalars kRfRed + i
  int32_t n_row;
  void* out;
  int64_t out_ld;
  int64_t y0, x0, h, w;
  int32_t out_dtype, n_red;
  int32_t kept;  // reduction whose chain values later stages start from (-1: none)
};

__device__ __forceinline__ f32x8 bf16x8_f32(const u32x4 q) {
  return f32x8{__uint_as_float(q.x << 16), __uint_as_float(q.x & 0xffff0000u),
               __uint_as_float(q.y << 16), __uint_as_float(q.y & 0xffff0000u),
               __uint_as_float(q.z << 16), __uint_as_float(q.z & 0xffff0000u),
               __uint_as_float(q.w << 16), __uint_as_float(q.w & 0xffff0000u)};
}

// the ops, with the definitions every other kernel uses (exp: exp1, with its
// range handling hoisted where a chunk allows, giving the same values)
__device__ __forceinline__ float rc_op1(uint8_t c, float a, float b) {
  switch (c) {
    case RC_ADD: return binary1<TTLH_OP_ADD>(a, b);
    case RC_SUB: return binary1<TTLH_OP_SUB>(a, b);
    case RC_RSUB: return binary1<TTLH_OP_SUB>(b, a);
    case RC_MUL: return binary1<TTLH_OP_MUL>(a, b);
    case RC_DIV: return binary1<TTLH_OP_DIV>(a, b);
    case RC_RDIV: return binary1<TTLH_OP_DIV>(b, a);
    case RC_MAX: return binary1<TTLH_OP_MAX>(a, b);
    case RC_RMAX: return binary1<TTLH_OP_MAX>(b, a);
    case RC_MIN: return binary1<TTLH_OP_MIN>(a, b);
    case RC_RMIN: return binary1<TTLH_OP_MIN>(b, a);
    case RC_EXP: return unary1<TTLH_OP_EXP>(a);
    case RC_SQRT: return unary1<TTLH_OP_SQRT>(a);
    case RC_RSQRT: return unary1<TTLH_OP_RSQRT>(a);
    case RC_ABS: return unary1<TTLH_OP_ABS>(a);
    case RC_NEG: return unary1<TTLH_OP_NEG>(a);
    case RC_RELU: return unary1<TTLH_OP_RELU>(a);
    case RC_RECIP: return unary1<TTLH_OP_RECIP>(a);
    default: return a;  // RC_COPY
  }
}

__device__ __forceinline__ float rf_round1(float x, uint8_t rnd) {
  return rnd == TTLH_BF16 ? round_bf16(x) : x;
}

// The stage's row scalars derived from earlier results, once per row.  A
// row's scalars live in LDS, one copy per wave (every wave of a row computes
// the same values; a wave's LDS accesses take effect in program order), since
// they are addressed by runtime indices.
__device__ __forceinline__ void rf_nodes(const RfStage& st, float* sc) {
#pragma unroll 1
  for (int i = 0; i < st.n_nodes; ++i) {
    const RfNode nd = st.node[i];
    const float x = nd.a == RS_IMM ? nd.imm_a : sc[nd.a - RS_SC];
    const float y = nd.b == RS_IMM ? nd.imm_b : sc[nd.b - RS_SC];
    sc[kRfNode0 + i] = rf_round1(rc_op1(nd.code, x, y), nd.rnd);
  }
}

template <int N, typename F>
__device__ __forceinline__ void rf_each(F&& f) {
  red_unroll(f, std::make_integer_sequence<int, N>());
}

__device__ __forceinline__ f32x8 rc_op8(uint8_t c, f32x8 a, f32x8 v) {
  switch (c) {  // uniform
    case RC_ADD: return binary8<TTLH_OP_ADD>(a, v);
    case RC_SUB: return binary8<TTLH_OP_SUB>(a, v);
    case RC_RSUB: return binary8<TTLH_OP_SUB>(v, a);
    case RC_MUL: return binary8<TTLH_OP_MUL>(a, v);
    case RC_DIV: return binary8<TTLH_OP_DIV>(a, v);
    case RC_RDIV: return binary8<TTLH_OP_DIV>(v, a);
    case RC_MAX: return binary8<TTLH_OP_MAX>(a, v);
    case RC_RMAX: return binary8<TTLH_OP_MAX>(v, a);
    case RC_MIN: return binary8<TTLH_OP_MIN>(a, v);
    case RC_RMIN: return binary8<TTLH_OP_MIN>(v, a);
    case RC_EXP: return vexp_uniform(a);
    case RC_SQRT: return unary8<TTLH_OP_SQRT>(a);
    case RC_RSQRT: return unary8<TTLH_OP_RSQRT>(a);
    case RC_ABS: return unary8<TTLH_OP_ABS>(a);
    case RC_NEG: return unary8<TTLH_OP_NEG>(a);
    case RC_RELU: return unary8<TTLH_OP_RELU>(a);
    case RC_RECIP: return unary8<TTLH_OP_RECIP>(a);
    default: return a;  // RC_COPY
  }
}

// One stage's chain on one chunk (x: the chunk's first column, in bounds;
// q0..q2: the chunk of the resident operands; kept: the kept stage's value
// on the chunk, the start of a chain with from_kept > 0).
__device__ __forceinline__ f32x8 rf_chain(const RfArgs& a, const RfStage& st, const u32x4 q0,
                                          const u32x4 q1, const u32x4 q2, const float* sc,
                                          const f32x8 kept, int64_t y, int64_t x) {
  auto fetch = [&](const RfStep& p) -> f32x8 {
    f32x8 v;
    if (p.src == RS_RES + 0) v = bf16x8_f32(q0);
    else if (p.src == RS_RES + 1) v = bf16x8_f32(q1);
    else if (p.src == RS_RES + 2) v = bf16x8_f32(q2);
    else if (p.src >= RS_IMM) v = splat(p.imm);
    else if (p.src >= RS_SC) v = splat(sc[p.src - RS_SC]);
    else {
      const EltOperand& op = a.mem[p.src - RS_MEM];
      v = to_f32<8, false>(op, load_raw<8, false>(op, operand_addr<false>(op, y, x)));
    }
    return p.orn == TTLH_BF16 ? round_bf16x8(v) : v;
  };
  f32x8 acc = kept;
  int k0 = st.from_kept;
  if (k0 == 0) {
    const RfStep first = st.step[0];
    acc = fetch(first);
    if (first.rnd == TTLH_BF16) acc = round_bf16x8(acc);
    k0 = 1;
  }
#pragma unroll 1
  for (int k = k0; k < st.n_steps; ++k) {
    const RfStep p = st.step[k];
    acc = rc_op8(p.code, acc, p.code <= RC_RMIN ? fetch(p) : acc);
    if (p.rnd == TTLH_BF16) acc = round_bf16x8(acc);
  }
  return acc;
}

// the reduction's scaler (red_scale's aligned 32-bit read)
__device__ __forceinline__ float rf_scale(const RfStage& st) {
  float s = st.scale_imm;
  if (st.scaler) {
    const uintptr_t u = reinterpret_cast<uintptr_t>(st.scaler);
    const uint32_t w =
        *reinterpret_cast<const __attribute__((address_space(1))) uint32_t*>(u & ~uintptr_t(3));
    s *= st.scaler_dtype == TTLH_BF16 ? __uint_as_float((u & 2) ? (w & 0xffff0000u) : (w << 16))
                                      : __uint_as_float(w);
  }
  return s;
}

// result of region row `row` where ttlh_reduce writes it: lane 0 the value,
// lanes 1-31 the rest of the zero-padded result tile row
__device__ __forceinline__ void rf_write(const RfStage& st, int64_t row, float v, int li) {
  const int64_t off = row * st.out_ld + li;
  if (li != 0 && !(st.out_pad && li < 32)) return;
  const float x = li == 0 ? v : 0.0f;
  if (st.out_dtype == TTLH_BF16) static_cast<uint16_t*>(st.out)[off] = f32_to_bf16(x);
  else static_cast<float*>(st.out)[off] = x;
}

// One chunk's values into the lane's running reduction, as red_acc does it
// element by element: a sum adds fma(v, s, r) (r + v when s = 1: the same
// value); a maximum takes fmaxf(r, v * s) and records separately whether a
// value was a NaN (red_combine's propagation: then the lane's result is NaN).
__device__ __forceinline__ void rf_accumulate(int kind, float s, const f32x8 v, float& r,
                                              bool& nan) {
  if (kind == TTLH_REDUCE_SUM) {
    if (s == 1.0f) {
#pragma unroll
      for (int k = 0; k < 8; ++k) r += v[k];
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) r = __builtin_fmaf(v[k], s, r);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float b = s == 1.0f ? v[k] : v[k] * s;
      nan |= b != b;
      r = fmaxf(r, b);
    }
  }
}

// LANES: lanes per row (256: a workgroup per row; 64: a wave per row, four
// rows per workgroup).  NRES: resident operands.  NCH: chunks per lane,
// ceil(w / (8 LANES)); a chunk past the row's end reads the row's last chunk
// instead (in bounds, never used), so every load is issued unconditionally
// and all of them are in flight together.  KEEP: a reduction's chain values
// are kept for the later stages whose chains start with it.  The chunk loops
// run at run time (one copy of each chain); a chunk's registers are selected
// through constant indices.
template <int LANES, int NRES, int NCH, bool KEEP>
__global__ __launch_bounds__(256) void reduce_rows_eltwise_kernel(const RfArgs a) {
  constexpr int R = NRES > 0 ? NRES : 1;
  __shared__ float part[kRfRed][4];
  __shared__ float scl[4][kRfScal];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t row = LANES == 256 ? int64_t(blockIdx.x) : int64_t(blockIdx.x) * 4 + wave;
  if (LANES == 64 && row >= a.h) return;  // wave-uniform (no workgroup barrier in this layout)
  const int64_t y = a.y0 + row;
  const int li = LANES == 256 ? t : lane;  // the lane's index in its row
  constexpr int64_t S = int64_t(LANES) * 8;  // elements from one of a lane's chunks to the next
  const int64_t xl = int64_t(li) * 8;
  u32x4 rq[R][NCH];
  rf_each<NRES>([&](auto r) {
    const uintptr_t base = operand_addr<false>(a.res[r], y, a.x0);
    rf_each<NCH>([&](auto c) {
      const int64_t xo = xl + c * S;
      rq[r][c] = ld16<true>(base + 2 * (xo < a.w ? xo : a.w - 8));
    });
  });
  f32x8 kept[KEEP ? NCH : 1];
  // chunk c's resident values and kept value (uniform c)
  auto chunk = [&](int c, u32x4& q0, u32x4& q1, u32x4& q2, f32x8& kv) {
    q0 = q1 = q2 = u32x4{0u, 0u, 0u, 0u};
    kv = splat(0.0f);
    rf_each<NCH>([&](auto cc) {
      if (c == cc) {
        if constexpr (NRES > 0) q0 = rq[0][cc];
        if constexpr (NRES > 1) q1 = rq[1][cc];
        if constexpr (NRES > 2) q2 = rq[2][cc];
        if constexpr (KEEP) kv = kept[cc];
      }
    });
  };
  float* const sc = scl[wave];
#pragma unroll 1
  for (int i = 0; i < a.n_row; ++i) {  // the row's values of the column-broadcast operands
    const EltOperand& op = a.row[i];
    sc[kRfRed + i] = to_f32<8, false>(op, load_raw<8, false>(op, operand_addr<false>(op, y, a.x0)))[0];
  }
#pragma unroll 1
  for (int j = 0; j < a.n_red; ++j) {
    const RfStage& st = a.st[j];
    rf_nodes(st, sc);
    const float s = rf_scale(st);
    float r = red_identity(st.kind);
    bool nan = false;
#pragma unroll 1
    for (int c = 0; c < NCH; ++c) {
      const int64_t xo = xl + c * S;
      u32x4 q0, q1, q2;
      f32x8 kv;
      chunk(c, q0, q1, q2, kv);
      const f32x8 v = rf_chain(a, st, q0, q1, q2, sc, kv, y, a.x0 + (xo < a.w ? xo : a.w - 8));
      if constexpr (KEEP) {
        if (j == a.kept)
          rf_each<NCH>([&](auto cc) {
            if (c == cc) kept[cc] = v;
          });
      }
      if (xo < a.w) rf_accumulate(st.kind, s, v, r, nan);
    }
    if (nan) r = __builtin_nanf("");
    r = red_wave(st.kind, r);
    if constexpr (LANES == 256) {
      if (lane == 0) part[j][wave] = r;
      __syncthreads();
      r = red_combine(st.kind, red_combine(st.kind, part[j][0], part[j][1]),
                      red_combine(st.kind, part[j][2], part[j][3]));
    }
    rf_write(st, row, r, li);
    sc[j] = st.out_dtype == TTLH_BF16 ? round_bf16(r) : r;
  }
  const RfStage& fe = a.st[kRfRed];
  if (fe.n_steps == 0) return;  // reductions alone (ttlh_reduce)
  rf_nodes(fe, sc);
#pragma unroll 1
  for (int c = 0; c < NCH; ++c) {
    const int64_t xo = xl + c * S;
    if (xo < a.w) {
      u32x4 q0, q1, q2;
      f32x8 kv;
      chunk(c, q0, q1, q2, kv);
      store_chunk<8>(a, y, a.x0 + xo, rf_chain(a, fe, q0, q1, q2, sc, kv, y, a.x0 + xo));
    }
  }
}

// The row softmax, the commonest program of this launch, as compiled chains
// recognised on the host (rf_softmax_form): reduction 0 = max over the row of
// x (one resident bf16 operand) times s0; reduction 1 = sum of e = exp(x - m)
// times s1 (m = reduction 0's result); out = e * recip(l) or e / l (l =
// reduction 1's result), every step's rounding as the chains carry it.  The
// same layout, order of summation and op definitions as the generic kernel,
// written out without the interpreter: its results are the generic kernel's,
// bit for bit.
struct RfSoftmax {
  uint8_t r_sub, r_exp, r_node, r_out;  // per-step rounding (TTLH_BF16 or not)
  uint8_t r_m, r_g;                     // rounding of the operands m and g
  uint8_t recip;                        // out = e * g, g = recip(l), else e / g, g = l
};

template <int LANES, int NCH>
__global__ __launch_bounds__(256) void softmax_rows_kernel(const RfArgs a, const RfSoftmax f) {
  __shared__ float part[2][4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t row = LANES == 256 ? int64_t(blockIdx.x) : int64_t(blockIdx.x) * 4 + wave;
  if (LANES == 64 && row >= a.h) return;  // wave-uniform (no workgroup barrier in this layout)
  const int64_t y = a.y0 + row;
  const int li = LANES == 256 ? t : lane;
  constexpr int64_t S = int64_t(LANES) * 8;
  const int64_t xl = int64_t(li) * 8;
  u32x4 q[NCH];
  const uintptr_t base = operand_addr<false>(a.res[0], y, a.x0);
  rf_each<NCH>([&](auto c) {
    const int64_t xo = xl + c * S;
    q[c] = ld16<true>(base + 2 * (xo < a.w ? xo : a.w - 8));
  });
  const float s0 = rf_scale(a.st[0]), s1 = rf_scale(a.st[1]);
  auto row_value = [&](int j, float r) {  // the butterfly, the wave partials, the result's dtype
    r = red_wave(a.st[j].kind, r);
    if constexpr (LANES == 256) {
      if (lane == 0) part[j][wave] = r;
      __syncthreads();
      r = red_combine(a.st[j].kind, red_combine(a.st[j].kind, part[j][0], part[j][1]),
                      red_combine(a.st[j].kind, part[j][2], part[j][3]));
    }
    rf_write(a.st[j], row, r, li);
    return a.st[j].out_dtype == TTLH_BF16 ? round_bf16(r) : r;
  };
  // reduction 0: the row maximum
  float r = -__builtin_inff();
  bool nan = false;
  rf_each<NCH>([&](auto c) {
    if (xl + c * S < a.w) {
      const f32x8 x = bf16x8_f32(q[c]);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float b = s0 == 1.0f ? x[k] : x[k] * s0;
        nan |= b != b;
        r = fmaxf(r, b);
      }
    }
  });
  if (nan) r = __builtin_nanf("");
  const float m = row_value(0, r);
  // reduction 1: the sum of e = exp(x - m), e kept
  f32x8 e[NCH];
  r = 0.0f;
  const float mm = f.r_m == TTLH_BF16 ? round_bf16(m) : m;
  rf_each<NCH>([&](auto c) {
    f32x8 d = bf16x8_f32(q[c]) - splat(mm);
    if (f.r_sub == TTLH_BF16) d = round_bf16x8(d);
    e[c] = vexp_uniform(d);
    if (f.r_exp == TTLH_BF16) e[c] = round_bf16x8(e[c]);
    if (xl + c * S < a.w) {
      if (s1 == 1.0f) {
#pragma unroll
        for (int k = 0; k < 8; ++k) r += e[c][k];
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) r = __builtin_fmaf(e[c][k], s1, r);
      }
    }
  });
  const float l = row_value(1, r);
  // the output
  float g = l;
  if (f.recip) {
    g = unary1<TTLH_OP_RECIP>(l);
    if (f.r_node == TTLH_BF16) g = round_bf16(g);
  }
  if (f.r_g == TTLH_BF16) g = round_bf16(g);
  rf_each<NCH>([&](auto c) {
    const int64_t xo = xl + c * S;
    if (xo < a.w) {
      f32x8 o = f.recip ? binary8<TTLH_OP_MUL>(e[c], splat(g)) : binary8<TTLH_OP_DIV>(e[c], splat(g));
      if (f.r_out == TTLH_BF16) o = round_bf16x8(o);
      store_chunk<8>(a, y, a.x0 + xo, o);
    }
  });
}

// A row normalisation by the sum of squares, e.g. RMS norm x * rsqrt(mean(x
// x) + eps) * g, as compiled chains recognised on the host (rf_norm_form):
// one reduction, the sum of x * x (x the one resident bf16 operand) times
// its scale; the program x * c (* g), c a row scalar (a reduction result or
// a node computed from it, such as rsqrt(r + eps)), g an operand read from
// memory.  The generic kernel's layout, summation order, node evaluation and
// per-step / per-operand roundings (read from the stages), without the
// interpreter: the same bits.
template <int LANES, int NCH>
__global__ __launch_bounds__(256) void norm_rows_kernel(const RfArgs a) {
  __shared__ float part[4];
  __shared__ float scl[4][kRfScal];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int64_t row = LANES == 256 ? int64_t(blockIdx.x) : int64_t(blockIdx.x) * 4 + wave;
  if (LANES == 64 && row >= a.h) return;  // wave-uniform (no workgroup barrier in this layout)
  const int64_t y = a.y0 + row;
  const int li = LANES == 256 ? t : lane;
  constexpr int64_t S = int64_t(LANES) * 8;
  const int64_t xl = int64_t(li) * 8;
  u32x4 q[NCH];
  const uintptr_t base = operand_addr<false>(a.res[0], y, a.x0);
  rf_each<NCH>([&](auto c) {
    const int64_t xo = xl + c * S;
    q[c] = ld16<true>(base + 2 * (xo < a.w ? xo : a.w - 8));
  });
  auto rnd8 = [](f32x8 v, uint8_t r) { return r == TTLH_BF16 ? round_bf16x8(v) : v; };
  float* const sc = scl[wave];
#pragma unroll 1
  for (int i = 0; i < a.n_row; ++i) {  // the row's values of the column-broadcast operands
    const EltOperand& op = a.row[i];
    sc[kRfRed + i] = to_f32<8, false>(op, load_raw<8, false>(op, operand_addr<false>(op, y, a.x0)))[0];
  }
  // the reduction: the sum of x * x, times its scale
  const RfStage& st = a.st[0];
  const RfStep p0 = st.step[0], p1 = st.step[1];
  const float s = rf_scale(st);
  float r = 0.0f;
  rf_each<NCH>([&](auto c) {
    if (xl + c * S < a.w) {
      const f32x8 x = bf16x8_f32(q[c]);
      const f32x8 v = rnd8(binary8<TTLH_OP_MUL>(rnd8(rnd8(x, p0.orn), p0.rnd), rnd8(x, p1.orn)),
                           p1.rnd);
      if (s == 1.0f) {
#pragma unroll
        for (int k = 0; k < 8; ++k) r += v[k];
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) r = __builtin_fmaf(v[k], s, r);
      }
    }
  });
  r = red_wave(TTLH_REDUCE_SUM, r);
  if constexpr (LANES == 256) {
    if (lane == 0) part[wave] = r;
    __syncthreads();
    r = (part[0] + part[1]) + (part[2] + part[3]);
  }
  rf_write(st, row, r, li);
  sc[0] = st.out_dtype == TTLH_BF16 ? round_bf16(r) : r;
  // the program: x * c (* g)
  const RfStage& fe = a.st[kRfRed];
  rf_nodes(fe, sc);
  const RfStep f0 = fe.step[0], f1 = fe.step[1], f2 = fe.step[2];
  const f32x8 cv = rnd8(splat(sc[f1.src - RS_SC]), f1.orn);
  const bool has_g = fe.n_steps == 3;
  const EltOperand& g = a.mem[has_g ? f2.src - RS_MEM : 0];
  rf_each<NCH>([&](auto c) {
    const int64_t xo = xl + c * S;
    if (xo < a.w) {
      f32x8 o = rnd8(rnd8(bf16x8_f32(q[c]), f0.orn), f0.rnd);
      o = rnd8(binary8<TTLH_OP_MUL>(o, cv), f1.rnd);
      if (has_g) {
        const f32x8 gv = rnd8(
            to_f32<8, false>(g, load_raw<8, false>(g, operand_addr<false>(g, y, a.x0 + xo))),
            f2.orn);
        o = rnd8(binary8<TTLH_OP_MUL>(o, gv), f2.rnd);
      }
      store_chunk<8>(a, y, a.x0 + xo, o);
    }
  });
}

}  // namespace
}  // namespace ttlh

using namespace ttlh;

namespace ttlh {
namespace {
int rows_fused_impl(const char* who, const ttlh_row_reduce* red, int n_red,
                    const ttlh_instr* prog, const ttlh_operand* in, int n_instr, void* out,
                    int out_dtype, int64_t out_ld, int64_t y0, int64_t x0, int64_t h, int64_t w,
                    void* stream);
}  // namespace
}  // namespace ttlh

extern "C" int ttlh_eltwise(const ttlh_instr* prog, const ttlh_operand* in, int n_instr, void* out,
                            int out_dtype, int64_t out_ld, int64_t y0, int64_t x0, int64_t h,
                            int64_t w, void* stream) {
  clear_error();
  TTLH_REQUIRE(out && (out_dtype == TTLH_BF16 || out_dtype == TTLH_F32), TTLH_EINVAL,
               "ttlh_eltwise: bad output pointer or dtype");
  TTLH_REQUIRE(h >= 0 && w >= 0 && y0 >= 0 && x0 >= 0 && out_ld >= x0 + w, TTLH_EINVAL,
               "ttlh_eltwise: bad output region");

  EltArgs a = {};
  ProgInfo pi;
  const int st = decode_program("ttlh_eltwise", prog, in, n_instr, y0, x0, h, w, a, pi);
  if (st != TTLH_OK) return st;
  const bool off32 = pi.off32 && (y0 + h) * out_ld < (int64_t(1) << 31);
  const bool vec = pi.vec && (out_ld % 8 == 0) && aligned16(out);
  if (h == 0 || w == 0) return TTLH_OK;
  a.out = out;
  a.out_ld = out_ld;
  a.out_dtype = out_dtype;
  const int64_t vw = vec ? 8 : 1;
  const int64_t cpr = w / vw;
  const int64_t total = h * cpr;
  TTLH_REQUIRE(total < (int64_t(1) << 31) - 256, TTLH_EUNSUPPORTED,
               "ttlh_eltwise: region of %lld chunks is too large", (long long)total);
  a.cpr = static_cast<uint32_t>(cpr);
  a.total = static_cast<uint32_t>(total);
  division_magic(a.cpr, &a.magic, &a.shift);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int n_ops = pi.n_ops;
  const bool preload = n_ops >= 1 && n_ops <= 4;  // preload reads operand 0 unconditionally
  // rare shapes: one generic variant each
  if (!off32) return vec ? launch<8, false, false, true, false, true>(a, s)
                         : launch<1, false, false, true, false, true>(a, s);
  if (!vec) return launch<1, false, false, true, true, true>(a, s);
  ChainArgs chain;
  if (make_chain(prog, n_instr, a, &chain)) {
    int status = TTLH_OK;
    if (pi.all_bf16 && try_flat(chain, n_instr, s, &status)) return status;
    if (pi.all_bf16 && try_stream(chain, n_instr, s, &status)) return status;
    return pi.all_bf16 ? dispatch_chain<true>(chain, n_instr, s)
                       : dispatch_chain<false>(chain, n_instr, s);
  }
  if (w >= 512) {
    // not linear (a stack, an op of a broadcast value): the row kernel takes
    // the programs it compiles into a chain over each row, operands constant
    // along a row becoming row scalars (exp(x - m) * recip(s) with m, s column
    // broadcasts); rows of 512+ elements keep its lanes busy
    const int rc = rows_fused_impl("ttlh_eltwise", nullptr, 0, prog, in, n_instr, out, out_dtype,
                                   out_ld, y0, x0, h, w, stream);
    if (rc != TTLH_EUNSUPPORTED) return rc;
    clear_error();
  }
  if (!preload) return launch<8, false, false, true, true, true>(a, s);
  if (pi.full) return launch<8, true, false, true, true, true>(a, s);
  // common ops, 8-wide, preloaded
  if (!pi.all_bf16) return launch<8, true, false, true, true, false>(a, s);
  return pi.max_depth > 1 ? launch<8, true, true, true, true, false>(a, s)
                          : launch<8, true, true, false, true, false>(a, s);
}

namespace ttlh {
namespace {

// row splits of a column reduce: about 1024 workgroups, at least 32 rows
// each (8 per wave)
int64_t red_rows_per_split(int64_t h, int64_t w) {
  const int64_t bx = (w + 511) / 512;
  int64_t sp = (1024 + bx - 1) / bx;
  const int64_t max_sp = h / 32 > 1 ? h / 32 : 1;
  if (sp > max_sp) sp = max_sp;
  if (sp > 65535) sp = 65535;
  if (sp < 1) sp = 1;
  return (h + sp - 1) / sp;
}

}  // namespace
}  // namespace ttlh

extern "C" int64_t ttlh_reduce_workspace_bytes(int dims, int64_t h, int64_t w) {
  if (h <= 0 || w <= 0 || dims == TTLH_REDUCE_DIM1) return 0;
  if (dims == TTLH_REDUCE_DIM0) {
    const int64_t rps = red_rows_per_split(h, w);
    const int64_t splits = (h + rps - 1) / rps;
    return splits > 1 ? splits * w * int64_t(sizeof(float)) : 0;
  }
  return h * int64_t(sizeof(float));
}

// The fixed device array behind ttlh_reduce_noalloc: fp32 partial results
// of column and full reductions (every launch writes the partials it later
// reads, so nothing in it has to start at zero).  Each GPU the library runs
// on holds its own copy until the process ends.
static __device__ __align__(256) float scratch[TTLH_REDUCE_SCRATCH_BYTES / sizeof(float)];

namespace ttlh {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the device `stream` runs on, looked up
// once per device (with that device current) and kept.  Host code uses this
// pointer, never the array's name, which on the host is only a stand-in.
int reduce_scratch(const char* who, hipStream_t stream, float** ptr) {
  int cur = 0;
  TTLH_REQUIRE(hipGetDevice(&cur) == hipSuccess, TTLH_EHIP, "%s: hipGetDevice failed", who);
  if (stream != nullptr) {
    int sdev = cur;
    TTLH_REQUIRE(hipStreamGetDevice(stream, &sdev) == hipSuccess, TTLH_EHIP,
                 "%s: hipStreamGetDevice failed", who);
    TTLH_REQUIRE(sdev == cur, TTLH_EINVAL,
                 "%s: the stream belongs to device %d but device %d is current", who, sdev, cur);
  }
  TTLH_REQUIRE(cur >= 0 && cur < kMaxDevices, TTLH_EUNSUPPORTED, "%s: device %d out of range",
               who, cur);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[cur] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    TTLH_REQUIRE(e == hipSuccess && p != nullptr, TTLH_EHIP,
                 "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, cur,
                 hipGetErrorString(e));
    g_scratch_ptr[cur] = static_cast<float*>(p);
  }
  *ptr = g_scratch_ptr[cur];
  return TTLH_OK;
}

int reduce_impl(const char* who, const ttlh_instr* prog, const ttlh_operand* in, int n_instr,
                int kind, int dims, const void* scaler, int scaler_dtype, float scale_imm,
                void* out, int out_dtype, int64_t out_ld, int out_pad, int64_t y0, int64_t x0,
                int64_t h, int64_t w, float* workspace, int64_t workspace_bytes, void* stream);

int rows_fused_impl(const char* who, const ttlh_row_reduce* red, int n_red,
                    const ttlh_instr* prog, const ttlh_operand* in, int n_instr, void* out,
                    int out_dtype, int64_t out_ld, int64_t y0, int64_t x0, int64_t h, int64_t w,
                    void* stream);

}  // namespace
}  // namespace ttlh

extern "C" int ttlh_reduce(const ttlh_instr* prog, const ttlh_operand* in, int n_instr, int kind,
                           int dims, const void* scaler, int scaler_dtype, float scale_imm,
                           void* out, int out_dtype, int64_t out_ld, int out_pad, int64_t y0,
                           int64_t x0, int64_t h, int64_t w, void* workspace,
                           int64_t workspace_bytes, void* stream) {
  clear_error();
  return reduce_impl("ttlh_reduce", prog, in, n_instr, kind, dims, scaler, scaler_dtype,
                     scale_imm, out, out_dtype, out_ld, out_pad, y0, x0, h, w,
                     static_cast<float*>(workspace), workspace_bytes, stream);
}

extern "C" int ttlh_reduce_noalloc(const ttlh_instr* prog, const ttlh_operand* in, int n_instr,
                                   int kind, int dims, const void* scaler, int scaler_dtype,
                                   float scale_imm, void* out, int out_dtype, int64_t out_ld,
                                   int out_pad, int64_t y0, int64_t x0, int64_t h, int64_t w,
                                   void* stream) {
  clear_error();
  const int64_t need = ttlh_reduce_workspace_bytes(dims, h, w);
  TTLH_REQUIRE(need <= TTLH_REDUCE_SCRATCH_BYTES, TTLH_EUNSUPPORTED,
               "ttlh_reduce_noalloc: a %lld x %lld reduction needs %lld bytes of partial results; "
               "the library's fixed scratch holds %lld (use ttlh_reduce with a workspace)",
               (long long)h, (long long)w, (long long)need, (long long)TTLH_REDUCE_SCRATCH_BYTES);
  float* ws = nullptr;
  if (need > 0) {
    const int st = reduce_scratch("ttlh_reduce_noalloc", static_cast<hipStream_t>(stream), &ws);
    if (st != TTLH_OK) return st;
  }
  return reduce_impl("ttlh_reduce_noalloc", prog, in, n_instr, kind, dims, scaler, scaler_dtype,
                     scale_imm, out, out_dtype, out_ld, out_pad, y0, x0, h, w, ws,
                     TTLH_REDUCE_SCRATCH_BYTES, stream);
}

namespace ttlh {
namespace {

int reduce_impl(const char* who, const ttlh_instr* prog, const ttlh_operand* in, int n_instr,
                int kind, int dims, const void* scaler, int scaler_dtype, float scale_imm,
                void* out, int out_dtype, int64_t out_ld, int out_pad, int64_t y0, int64_t x0,
                int64_t h, int64_t w, float* workspace, int64_t workspace_bytes, void* stream) {
  TTLH_REQUIRE(kind == TTLH_REDUCE_SUM || kind == TTLH_REDUCE_MAX, TTLH_EINVAL,
               "%s: kind must be TTLH_REDUCE_SUM or TTLH_REDUCE_MAX", who);
  TTLH_REQUIRE(dims >= 1 && dims <= 3, TTLH_EINVAL,
               "%s: dims must be TTLH_REDUCE_DIM0, TTLH_REDUCE_DIM1 or both", who);
  TTLH_REQUIRE(out && (out_dtype == TTLH_BF16 || out_dtype == TTLH_F32), TTLH_EINVAL,
               "%s: bad output pointer or dtype", who);
  TTLH_REQUIRE(!scaler || scaler_dtype == TTLH_BF16 || scaler_dtype == TTLH_F32, TTLH_EINVAL,
               "%s: bad scaler dtype", who);
  TTLH_REQUIRE(out_pad == 0 || out_pad == 1, TTLH_EINVAL, "%s: out_pad must be 0 or 1", who);
  TTLH_REQUIRE(h >= 1 && w >= 1 && y0 >= 0 && x0 >= 0, TTLH_EINVAL,
               "%s: empty or negative region", who);
  TTLH_REQUIRE(out_ld >= (out_pad ? 32 : 1), TTLH_EINVAL, "%s: out_ld too small", who);
  RedArgs a = {};
  ProgInfo pi;
  const int st = decode_program(who, prog, in, n_instr, y0, x0, h, w, a.e, pi);
  if (st != TTLH_OK) return st;
  const int64_t need = ttlh_reduce_workspace_bytes(dims, h, w);
  TTLH_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), TTLH_EINVAL,
               "%s: needs a workspace of %lld bytes (got %lld)", who, (long long)need,
               (long long)workspace_bytes);
  TTLH_REQUIRE((h + 3) / 4 < (int64_t(1) << 31) && w / 64 < (int64_t(1) << 31), TTLH_EUNSUPPORTED,
               "%s: region too large", who);
  a.h = h;
  a.w = w;
  a.scaler = scaler;
  a.scaler_dtype = scaler_dtype;
  a.scale_imm = scale_imm;
  a.out = out;
  a.out_ld = out_ld;
  a.out_dtype = out_dtype;
  a.out_pad = out_pad;
  a.ws = workspace;
  a.kind = kind;
  a.splits = 1;
  a.rows_per_split = h;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 block(256);
  // kernel variant (see the reduction kernels): the pipelined 8-wide modes
  // need aligned operands and at most four of them
  const bool plain = n_instr == 1 && prog[0].form == TTLH_FORM_LOAD;
  const int mode = !pi.vec || pi.n_ops < 1 || pi.n_ops > 4 ? 0 : (plain ? 1 : (pi.full ? 0 : 2));
  const int variant = mode == 0 ? (pi.vec ? 1 : 0) : mode + 1;
  // a * b of two plain bf16 operands (a row dot product) over wide rows:
  // the bf16 row kernel's PROD variant, the fused row kernel's values
  const auto plain_row = [&](const EltOperand& o) {
    return o.dtype == TTLH_BF16 && o.vec && o.rmask == -1 && o.cmask == -1 && o.cs == 1;
  };
  if (dims == TTLH_REDUCE_DIM1 && n_instr == 2 && prog[0].form == TTLH_FORM_LOAD &&
      prog[1].form == TTLH_FORM_BIN && prog[1].op == TTLH_OP_MUL && prog[1].rnd == TTLH_BF16 &&
      pi.vec && pi.n_ops == 2 && w >= 2048 && plain_row(a.e.ops[0]) && plain_row(a.e.ops[1])) {
    const EltOperand& o0 = a.e.ops[0];
    const EltOperand& o1 = a.e.ops[1];
    const uint16_t* b0 = static_cast<const uint16_t*>(o0.ptr) + (a.e.y0 + o0.roff) * o0.rs +
                         a.e.x0 + o0.coff;
    const uint16_t* b1 = static_cast<const uint16_t*>(o1.ptr) + (a.e.y0 + o1.roff) * o1.rs +
                         a.e.x0 + o1.coff;
    const bool nt = (o0.rs != 0 && o1.rs != 0) || h == 1;  // no element read twice
    const dim3 grid(static_cast<uint32_t>(h));
#define TTLH_ROWS_PROD(K)                                                                    \
  if (nt) hipLaunchKernelGGL((reduce_rows_bf16_kernel<K, false, true, true>), grid, block, 0, s, \
                             b0, int64_t(o0.rs), int64_t(w), a, b1, int64_t(o1.rs));         \
  else hipLaunchKernelGGL((reduce_rows_bf16_kernel<K, false, false, true>), grid, block, 0, s, \
                          b0, int64_t(o0.rs), int64_t(w), a, b1, int64_t(o1.rs));
    if (kind == TTLH_REDUCE_SUM) {
      TTLH_ROWS_PROD(TTLH_REDUCE_SUM)
    } else {
      TTLH_ROWS_PROD(TTLH_REDUCE_MAX)
    }
#undef TTLH_ROWS_PROD
    return check_launch("reduce_rows_bf16_kernel");
  }
  if (dims == TTLH_REDUCE_DIM1 && !plain) {
    // a program: the fused row kernel's chain, which its row reductions
    // share (so a row reduction gives the same values alone and fused);
    // programs it does not take run on the kernels below
    const ttlh_row_reduce r = {prog, in, n_instr, kind, scaler, scaler_dtype, scale_imm, out,
                               out_dtype, out_pad, out_ld};
    const int rc = rows_fused_impl(who, &r, 1, nullptr, nullptr, 0, nullptr, 0, 0, y0, x0, h, w,
                                   stream);
    if (rc != TTLH_EUNSUPPORTED) return rc;
    clear_error();
  }
  if (dims != TTLH_REDUCE_DIM0) {
    const bool wide = mode != 0 && w >= 2048;
    const dim3 grid(static_cast<uint32_t>(wide ? h : (h + 3) / 4));
    // the specialised kernel: a plain bf16 operand; streaming loads when no
    // element of it is read twice
    const EltOperand& o0 = a.e.ops[0];
    const bool plain_bf16 = wide && mode == 1 && o0.dtype == TTLH_BF16 && o0.rmask == -1 &&
                            o0.cmask == -1 && o0.cs == 1;
    const bool nt = o0.rs != 0 || h == 1;
    // element x of region row r: base[r rs + x] (no masks on this path)
    const uint16_t* const rbase =
        plain_bf16 ? static_cast<const uint16_t*>(o0.ptr) + (a.e.y0 + o0.roff) * o0.rs +
                         a.e.x0 + o0.coff
                   : nullptr;
#define TTLH_ROWS_BF16(K, WS)                                                                \
  if (nt) hipLaunchKernelGGL((reduce_rows_bf16_kernel<K, WS, true>), grid, block, 0, s, rbase, \
                             int64_t(o0.rs), int64_t(w), a);                                 \
  else hipLaunchKernelGGL((reduce_rows_bf16_kernel<K, WS, false>), grid, block, 0, s, rbase,  \
                          int64_t(o0.rs), int64_t(w), a);
#define TTLH_ROWS(WS)                                                                        \
  if (plain_bf16 && kind == TTLH_REDUCE_SUM) {                                               \
    TTLH_ROWS_BF16(TTLH_REDUCE_SUM, WS)                                                      \
  } else if (plain_bf16) {                                                                   \
    TTLH_ROWS_BF16(TTLH_REDUCE_MAX, WS)                                                      \
  } else if (wide && mode == 1)                                                              \
    hipLaunchKernelGGL((reduce_rows_wide_kernel<WS, 1>), grid, block, 0, s, a);             \
  else if (wide)                                                                             \
    hipLaunchKernelGGL((reduce_rows_wide_kernel<WS, 2>), grid, block, 0, s, a);             \
  else switch (variant) {                                                                    \
    case 0: hipLaunchKernelGGL((reduce_rows_kernel<1, WS, 0>), grid, block, 0, s, a); break; \
    case 1: hipLaunchKernelGGL((reduce_rows_kernel<8, WS, 0>), grid, block, 0, s, a); break; \
    case 2: hipLaunchKernelGGL((reduce_rows_kernel<8, WS, 1>), grid, block, 0, s, a); break; \
    default: hipLaunchKernelGGL((reduce_rows_kernel<8, WS, 2>), grid, block, 0, s, a); break; \
  }
    if (dims == TTLH_REDUCE_DIM1) {
      TTLH_ROWS(false)
      return check_launch("reduce_rows_kernel");
    }
    TTLH_ROWS(true)
#undef TTLH_ROWS
#undef TTLH_ROWS_BF16
    int rc = check_launch("reduce_rows_kernel");
    if (rc != TTLH_OK) return rc;
    hipLaunchKernelGGL(reduce_all_finish_kernel, dim3(1), block, 0, s, a);
    return check_launch("reduce_all_finish_kernel");
  }
  {
    a.rows_per_split = red_rows_per_split(h, w);
    a.splits = static_cast<int32_t>((h + a.rows_per_split - 1) / a.rows_per_split);
    const int vw = pi.vec ? 8 : 1;
    const dim3 grid(static_cast<uint32_t>((w + 64 * vw - 1) / (64 * vw)),
                    static_cast<uint32_t>(a.splits));
    switch (variant) {
      case 0: hipLaunchKernelGGL((reduce_cols_kernel<1, 0>), grid, block, 0, s, a); break;
      case 1: hipLaunchKernelGGL((reduce_cols_kernel<8, 0>), grid, block, 0, s, a); break;
      case 2: hipLaunchKernelGGL((reduce_cols_kernel<8, 1>), grid, block, 0, s, a); break;
      default: hipLaunchKernelGGL((reduce_cols_kernel<8, 2>), grid, block, 0, s, a); break;
    }
    int rc = check_launch("reduce_cols_kernel");
    if (rc != TTLH_OK || a.splits == 1) return rc;
    hipLaunchKernelGGL(reduce_cols_finish_kernel, dim3(static_cast<uint32_t>((w + 31) / 32)),
                       block, 0, s, a);
    return check_launch("reduce_cols_finish_kernel");
  }
}

}  // namespace
}  // namespace ttlh

namespace ttlh {
namespace {

// [lo, hi): the bytes operand o can touch over the region (a superset)
void operand_span(const EltOperand& o, int64_t y0, int64_t x0, int64_t h, int64_t w,
                  uintptr_t* lo, uintptr_t* hi) {
  auto first = [](int64_t m, int64_t c) {
    return m == -1 ? c : (m == ~int64_t(31) ? (c & ~int64_t(31)) : int64_t(0));
  };
  const int64_t esz = o.dtype == TTLH_BF16 ? 2 : 4;
  const int64_t e0 = (first(o.rmask, y0) + o.roff) * o.rs + (first(o.cmask, x0) + o.coff) * o.cs;
  const int64_t e1 = (mask_max(o.rmask, y0 + h - 1) + o.roff) * o.rs +
                     (mask_max(o.cmask, x0 + w - 1) + o.coff) * o.cs;
  const uintptr_t p = reinterpret_cast<uintptr_t>(o.ptr);
  *lo = p + static_cast<uintptr_t>(e0 * esz);
  *hi = p + static_cast<uintptr_t>((e1 + 1) * esz);
}

bool overlap(uintptr_t a0, uintptr_t a1, uintptr_t b0, uintptr_t b1) { return a0 < b1 && b0 < a1; }

// bytes of a row reduction's results, the tile padding included
void row_result_span(const ttlh_row_reduce& r, int64_t h, uintptr_t* lo, uintptr_t* hi) {
  const int64_t esz = r.out_dtype == TTLH_BF16 ? 2 : 4;
  *lo = reinterpret_cast<uintptr_t>(r.out);
  *hi = *lo + static_cast<uintptr_t>(((h - 1) * r.out_ld + (r.out_pad ? 32 : 1)) * esz);
}

// whether o reads, at every element (y, x) of the region, reduction r's
// result for row y (the element ttlh_reduce writes it to)
bool reads_row_result(const EltOperand& o, const ttlh_row_reduce& r, int64_t y0, int64_t x0,
                      int64_t h, int64_t w) {
  if (o.dtype != r.out_dtype) return false;
  const bool one_col = o.cs == 0 || o.cmask == 0 || w == 1;
  const bool rows = h == 1 || (o.rmask == -1 && o.rs == r.out_ld);
  if (!one_col || !rows) return false;
  const int64_t esz = o.dtype == TTLH_BF16 ? 2 : 4;
  const int64_t e = ((y0 & o.rmask) + o.roff) * o.rs + ((x0 & o.cmask) + o.coff) * o.cs;
  return reinterpret_cast<uintptr_t>(o.ptr) + static_cast<uintptr_t>(e * esz) ==
         reinterpret_cast<uintptr_t>(r.out);
}

bool same_map(const EltOperand& a, const EltOperand& b) {
  return a.ptr == b.ptr && a.dtype == b.dtype && a.rs == b.rs && a.cs == b.cs &&
         a.rmask == b.rmask && a.cmask == b.cmask && a.roff == b.roff && a.coff == b.coff;
}

// rev: the op applied as op(operand, acc)
uint8_t rc_code(int op, bool rev = false) {
  switch (op) {
    case TTLH_OP_ADD: return RC_ADD;
    case TTLH_OP_SUB: return rev ? RC_RSUB : RC_SUB;
    case TTLH_OP_MUL: return RC_MUL;
    case TTLH_OP_DIV: return rev ? RC_RDIV : RC_DIV;
    case TTLH_OP_MAX: return rev ? RC_RMAX : RC_MAX;
    case TTLH_OP_MIN: return rev ? RC_RMIN : RC_MIN;
    case TTLH_OP_EXP: return RC_EXP;
    case TTLH_OP_SQRT: return RC_SQRT;
    case TTLH_OP_RSQRT: return RC_RSQRT;
    case TTLH_OP_ABS: return RC_ABS;
    case TTLH_OP_NEG: return RC_NEG;
    case TTLH_OP_RELU: return RC_RELU;
    default: return RC_RECIP;  // TTLH_OP_RECIP (is_inline_op admits no other)
  }
}

// The decoded stage program `e` (nj steps; operand i's source src_of[i], an
// RS_* code) as a chain over the row (RfStep) and the row scalars it needs
// (RfNode): the expression tree the stack program evaluates, each node with
// its step's rounding, walked from the root down the one child that depends
// on the row's elements; the other child of every binary node must be a leaf,
// an immediate or a subtree of row scalars and immediates only (a row
// scalar).  Returns false when the program is no such chain.
bool rf_compile(const EltArgs& e, int nj, const uint8_t* src_of, RfStage& st) {
  struct Node {
    uint8_t type;  // 0 operand leaf, 1 immediate, 2 unary, 3 binary
    uint8_t op, rnd, src;
    int a, b;
    float imm;
    bool uni;      // a row scalar: leaves of row results and immediates only
  };
  Node t[2 * TTLH_MAX_INSTR];
  int nt = 0, stk[TTLH_MAX_STACK + 1], sp = 0;
  for (int k = 0; k < nj; ++k) {
    const Ins& ins = e.prog[k];
    int v = -1;
    if (ins.src == SRC_OPERAND) {
      const uint8_t src = src_of[ins.arg];
      t[nt] = Node{0, 0, TTLH_F32, src, -1, -1, 0.0f, src >= RS_SC && src < RS_IMM};
      v = nt++;
    } else if (ins.src == SRC_IMM) {
      t[nt] = Node{1, 0, TTLH_F32, RS_IMM, -1, -1, ins.imm, true};
      v = nt++;
    } else if (ins.src == SRC_POP) {
      v = stk[sp - 2];
      stk[sp - 2] = stk[sp - 1];
      --sp;
    }
    int r = v;
    switch (ins.kind) {
      case K_SET: stk[sp++] = v; break;  // LOAD / CONST: the stack was empty
      case K_PUSH: stk[sp++] = v; break;
      case K_UNARY:
        t[nt] = Node{2, ins.op, TTLH_F32, 0, stk[sp - 1], -1, 0.0f, t[stk[sp - 1]].uni};
        r = stk[sp - 1] = nt++;
        break;
      case K_BIN:
        t[nt] = Node{3, ins.op, TTLH_F32, 0, stk[sp - 1], v, 0.0f, t[stk[sp - 1]].uni && t[v].uni};
        r = stk[sp - 1] = nt++;
        break;
      default:  // K_BIN_REV (BIN_POP included: v is the value popped)
        t[nt] = Node{3, ins.op, TTLH_F32, 0, v, stk[sp - 1], 0.0f, t[stk[sp - 1]].uni && t[v].uni};
        r = stk[sp - 1] = nt++;
        break;
    }
    t[r].rnd = ins.rnd;
  }
  if (sp != 1) return false;
  auto imm_of = [&](const Node& x) {  // an immediate with its own rounding applied
    return x.rnd == TTLH_BF16 ? bf16_to_f32(f32_to_bf16(x.imm)) : x.imm;
  };
  // a row-scalar subtree as an operand of a node: (RS_SC + slot or RS_IMM, imm)
  int n_nodes = 0;
  bool ok = true;
  auto hoist = [&](auto&& self, int m, float& imm) -> uint8_t {
    const Node& x = t[m];
    imm = 0.0f;
    if (x.type == 1) {
      imm = imm_of(x);
      return RS_IMM;
    }
    uint8_t a = RS_IMM, b = RS_IMM;
    float ia = 0.0f, ib = 0.0f;
    uint8_t code = RC_COPY;
    if (x.type == 0) {
      if (x.rnd != TTLH_BF16) return x.src;
      a = x.src;
    } else {
      a = self(self, x.a, ia);
      if (x.type == 3) b = self(self, x.b, ib);
      code = rc_code(x.op);
    }
    if (n_nodes >= kRfNodes) {
      ok = false;
      return RS_IMM;
    }
    st.node[n_nodes] = RfNode{code, a, b, x.rnd, ia, ib};
    return static_cast<uint8_t>(RS_SC + kRfNode0 + n_nodes++);
  };
  RfStep rev_steps[TTLH_MAX_INSTR + 1];
  int ns = 0;
  int n = stk[0];
  for (;;) {
    const Node& x = t[n];
    RfStep p{};
    p.rnd = x.rnd;
    if (x.uni || x.type <= 1) {  // the chain's first value
      p.code = RC_COPY;
      if (x.type == 0) {
        p.src = x.src;
        p.orn = x.rnd;
      } else {
        p.src = hoist(hoist, n, p.imm);
        p.rnd = TTLH_F32;  // a node or an immediate carries its rounding
        p.orn = TTLH_F32;
      }
      rev_steps[ns++] = p;
      break;
    }
    if (x.type == 2) {
      p.code = rc_code(x.op);
      rev_steps[ns++] = p;
      n = x.a;
      continue;
    }
    const Node &A = t[x.a], &B = t[x.b];
    int spine, opnd;
    bool rev;
    if (!A.uni && !B.uni) {
      if (B.type == 0) spine = x.a, opnd = x.b, rev = false;
      else if (A.type == 0) spine = x.b, opnd = x.a, rev = true;
      else return false;  // two operands computed from the row: no chain
    } else if (B.uni) {
      spine = x.a, opnd = x.b, rev = false;
    } else {
      spine = x.b, opnd = x.a, rev = true;
    }
    p.code = rc_code(x.op, rev);
    const Node& o = t[opnd];
    if (o.type == 0) {
      p.src = o.src;
      p.orn = o.rnd;
    } else {
      // a node or an immediate carries its own rounding: the fetch adds none
      // (left at the zero default, TTLH_BF16, it would round an f32 node or
      // an immediate such as 0.1 to bf16, where ttlh_eltwise does not)
      p.src = hoist(hoist, opnd, p.imm);
      p.orn = TTLH_F32;
    }
    rev_steps[ns++] = p;
    n = spine;
    if (ns > TTLH_MAX_INSTR) return false;
  }
  if (!ok) return false;
  st.n_steps = ns;
  st.n_nodes = n_nodes;
  for (int k = 0; k < ns; ++k) st.step[k] = rev_steps[ns - 1 - k];
  return true;
}

// A reduction whose whole chain begins the chain of later stages (softmax:
// exp(x - max) summed, then exp(x - max) scaled): its per-chunk values are
// kept in registers and those stages start from them.  The shared steps may
// read resident rows, other operands, immediates and reduction results, not
// the stage-local derived scalars.  The reduction saving the most steps (of a
// chain of at least two) is kept (a.kept = -1: none).
void rf_choose_kept(RfArgs& a) {
  a.kept = -1;
  int best = 0;
  for (int j = 0; j < a.n_red; ++j) {
    const RfStage& sj = a.st[j];
    if (sj.n_steps < 2) continue;  // a plain load: keeping it saves no arithmetic
    bool local = false;
    for (int k = 0; k < sj.n_steps; ++k)
      local = local || (sj.step[k].src >= RS_SC + kRfNode0 && sj.step[k].src < RS_IMM &&
                        (k == 0 || sj.step[k].code <= RC_RMIN));
    if (local) continue;
    int saved = 0;
    for (int q = j + 1; q <= kRfRed; ++q) {
      if (q >= a.n_red && q != kRfRed) continue;
      const RfStage& sq = a.st[q];
      if (sq.n_steps >= sj.n_steps &&
          memcmp(sq.step, sj.step, sizeof(RfStep) * sj.n_steps) == 0)
        saved += sj.n_steps;
    }
    if (saved > best) best = saved, a.kept = j;
  }
  for (int q = 0; q <= kRfRed; ++q) a.st[q].from_kept = 0;
  if (a.kept < 0) return;
  const RfStage& sj = a.st[a.kept];
  for (int q = a.kept + 1; q <= kRfRed; ++q) {
    if (q >= a.n_red && q != kRfRed) continue;
    RfStage& sq = a.st[q];
    if (sq.n_steps >= sj.n_steps && memcmp(sq.step, sj.step, sizeof(RfStep) * sj.n_steps) == 0)
      sq.from_kept = sj.n_steps;
  }
}

// Whether the compiled stages are the row softmax softmax_rows_kernel runs
// (its comment has the form), and its rounding flags.
bool rf_softmax_form(const RfArgs& a, RfSoftmax* f) {
  if (a.n_red != 2 || a.kept != 1) return false;
  const RfStage &s0 = a.st[0], &s1 = a.st[1], &fe = a.st[kRfRed];
  // x, the one resident operand, is bf16: a bf16 rounding of it (a step's or
  // an operand's) is the identity, so those flags do not matter
  const uint8_t x = RS_RES + 0;
  if (s0.kind != TTLH_REDUCE_MAX || s0.n_steps != 1 || s0.n_nodes != 0 ||
      s0.step[0].code != RC_COPY || s0.step[0].src != x)
    return false;
  if (s1.kind != TTLH_REDUCE_SUM || s1.n_steps != 3 || s1.n_nodes != 0 || s1.from_kept != 0 ||
      s1.step[0].code != RC_COPY || s1.step[0].src != x || s1.step[1].code != RC_SUB ||
      s1.step[1].src != RS_SC + 0 || s1.step[2].code != RC_EXP)
    return false;
  if (fe.from_kept != 3 || fe.n_steps != 4) return false;
  const RfStep& o = fe.step[3];
  if (o.code == RC_MUL && o.src == RS_SC + kRfNode0 && fe.n_nodes == 1 &&
      fe.node[0].code == RC_RECIP && fe.node[0].a == RS_SC + 1) {
    f->recip = 1;
    f->r_node = fe.node[0].rnd;
  } else if (o.code == RC_DIV && o.src == RS_SC + 1 && fe.n_nodes == 0) {
    f->recip = 0;
    f->r_node = TTLH_F32;
  } else {
    return false;
  }
  f->r_sub = s1.step[1].rnd;
  f->r_exp = s1.step[2].rnd;
  f->r_out = o.rnd;
  f->r_m = s1.step[1].orn;
  f->r_g = o.orn;
  return true;
}

// Whether the compiled stages are the row normalisation norm_rows_kernel
// runs: one reduction, the sum of x * x; the program x * c or x * c * g with
// c a row scalar and g an operand read from memory (x the resident operand).
bool rf_norm_form(const RfArgs& a) {
  if (a.n_red != 1 || a.kept != -1) return false;
  const uint8_t x = RS_RES + 0;
  const RfStage &st = a.st[0], &fe = a.st[kRfRed];
  if (st.kind != TTLH_REDUCE_SUM || st.n_steps != 2 || st.n_nodes != 0 || st.from_kept != 0 ||
      st.step[0].code != RC_COPY || st.step[0].src != x || st.step[1].code != RC_MUL ||
      st.step[1].src != x)
    return false;
  if ((fe.n_steps != 2 && fe.n_steps != 3) || fe.from_kept != 0 || fe.step[0].code != RC_COPY ||
      fe.step[0].src != x || fe.step[1].code != RC_MUL || fe.step[1].src < RS_SC ||
      fe.step[1].src >= RS_IMM)
    return false;
  if (fe.n_steps == 3 && (fe.step[2].code != RC_MUL || fe.step[2].src < RS_MEM ||
                          fe.step[2].src >= RS_SC))
    return false;
  return true;
}

}  // namespace
}  // namespace ttlh

namespace ttlh {
namespace {

// one workgroup per row group (a row, or four rows of a wave each)
template <int L, int R, int C>
int rf_launch(const RfArgs& a, int64_t groups, hipStream_t s) {
  TTLH_REQUIRE(groups < (int64_t(1) << 31), TTLH_EUNSUPPORTED,
               "ttlh_reduce_rows_eltwise: region too large");
  if (a.kept >= 0)
    hipLaunchKernelGGL((reduce_rows_eltwise_kernel<L, R, C, true>),
                       dim3(static_cast<uint32_t>(groups)), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((reduce_rows_eltwise_kernel<L, R, C, false>),
                       dim3(static_cast<uint32_t>(groups)), dim3(256), 0, s, a);
  return check_launch("reduce_rows_eltwise_kernel");
}

}  // namespace
}  // namespace ttlh

extern "C" int ttlh_reduce_rows_eltwise(const ttlh_row_reduce* red, int n_red,
                                        const ttlh_instr* prog, const ttlh_operand* in,
                                        int n_instr, void* out, int out_dtype, int64_t out_ld,
                                        int64_t y0, int64_t x0, int64_t h, int64_t w,
                                        void* stream) {
  clear_error();
  const char* who = "ttlh_reduce_rows_eltwise";
  TTLH_REQUIRE(prog && in && n_instr > 0, TTLH_EINVAL, "%s: needs the elementwise program", who);
  TTLH_REQUIRE(red && n_red >= 1, TTLH_EINVAL, "%s: needs at least one reduction", who);
  return rows_fused_impl(who, red, n_red, prog, in, n_instr, out, out_dtype, out_ld, y0, x0, h, w,
                         stream);
}

namespace ttlh {
namespace {

// The fused row launch (n_instr == 0: the reductions alone, no elementwise
// stage and no output).  TTLH_EUNSUPPORTED: nothing launched.
int rows_fused_impl(const char* who, const ttlh_row_reduce* red, int n_red,
                    const ttlh_instr* prog, const ttlh_operand* in, int n_instr, void* out,
                    int out_dtype, int64_t out_ld, int64_t y0, int64_t x0, int64_t h, int64_t w,
                    void* stream) {
  const bool has_out = n_instr > 0;
  TTLH_REQUIRE(n_red >= 0 && (n_red == 0 || red) && (has_out || n_red >= 1), TTLH_EINVAL,
               "%s: needs a reduction or an elementwise program", who);
  TTLH_REQUIRE(!has_out || (out && (out_dtype == TTLH_BF16 || out_dtype == TTLH_F32)),
               TTLH_EINVAL, "%s: bad output pointer or dtype", who);
  TTLH_REQUIRE(h >= 1 && w >= 1 && y0 >= 0 && x0 >= 0 && (!has_out || out_ld >= x0 + w),
               TTLH_EINVAL, "%s: bad region", who);
  for (int j = 0; j < n_red; ++j) {
    const ttlh_row_reduce& r = red[j];
    TTLH_REQUIRE(r.kind == TTLH_REDUCE_SUM || r.kind == TTLH_REDUCE_MAX, TTLH_EINVAL,
                 "%s: reduction %d: kind must be TTLH_REDUCE_SUM or TTLH_REDUCE_MAX", who, j);
    TTLH_REQUIRE(r.out && (r.out_dtype == TTLH_BF16 || r.out_dtype == TTLH_F32), TTLH_EINVAL,
                 "%s: reduction %d: bad output pointer or dtype", who, j);
    TTLH_REQUIRE(!r.scaler || r.scaler_dtype == TTLH_BF16 || r.scaler_dtype == TTLH_F32,
                 TTLH_EINVAL, "%s: reduction %d: bad scaler dtype", who, j);
    TTLH_REQUIRE(r.out_pad == 0 || r.out_pad == 1, TTLH_EINVAL,
                 "%s: reduction %d: out_pad must be 0 or 1", who, j);
    TTLH_REQUIRE(r.out_ld >= (r.out_pad ? 32 : 1), TTLH_EINVAL, "%s: reduction %d: out_ld too small",
                 who, j);
  }
  TTLH_REQUIRE(n_red <= kRfRed, TTLH_EUNSUPPORTED, "%s: at most %d reductions (got %d)", who,
               kRfRed, n_red);
  TTLH_REQUIRE(w <= int64_t(kRfChunks) * 2048, TTLH_EUNSUPPORTED,
               "%s: rows of %lld elements (at most %d)", who, (long long)w, kRfChunks * 2048);
  TTLH_REQUIRE(!has_out || (aligned16(out) && out_ld % 8 == 0), TTLH_EUNSUPPORTED,
               "%s: the output does not admit 16-byte chunks", who);
  const int64_t oesz = out_dtype == TTLH_BF16 ? 2 : 4;
  const uintptr_t out_lo =
      has_out ? reinterpret_cast<uintptr_t>(out) + static_cast<uintptr_t>((y0 * out_ld + x0) * oesz)
              : 0;
  const uintptr_t out_hi =
      has_out ? reinterpret_cast<uintptr_t>(out) +
                    static_cast<uintptr_t>(((y0 + h - 1) * out_ld + x0 + w) * oesz)
              : 0;
  uintptr_t rlo[kRfRed], rhi[kRfRed];
  for (int j = 0; j < n_red; ++j) {
    row_result_span(red[j], h, &rlo[j], &rhi[j]);
    TTLH_REQUIRE(!overlap(rlo[j], rhi[j], out_lo, out_hi), TTLH_EUNSUPPORTED,
                 "%s: reduction %d's results overlap the output", who, j);
    for (int i = 0; i < j; ++i)
      TTLH_REQUIRE(!overlap(rlo[j], rhi[j], rlo[i], rhi[i]), TTLH_EUNSUPPORTED,
                   "%s: the results of reductions %d and %d overlap", who, i, j);
  }
  for (int j = 0; j < n_red; ++j) {
    if (!red[j].scaler) continue;
    const uintptr_t s0 = reinterpret_cast<uintptr_t>(red[j].scaler);
    const uintptr_t s1 = s0 + (red[j].scaler_dtype == TTLH_BF16 ? 2 : 4);
    bool clash = overlap(s0, s1, out_lo, out_hi);
    for (int i = 0; i < n_red; ++i) clash = clash || overlap(s0, s1, rlo[i], rhi[i]);
    TTLH_REQUIRE(!clash, TTLH_EUNSUPPORTED, "%s: reduction %d's scaler overlaps an output", who, j);
  }

  RfArgs a = {};
  a.out = out;
  a.out_ld = out_ld;
  a.out_dtype = out_dtype;
  a.y0 = y0;
  a.x0 = x0;
  a.h = h;
  a.w = w;
  a.n_red = n_red;
  int n_mem = 0, n_res = 0;
  for (int j = 0; j <= n_red; ++j) {
    const bool fin = j == n_red;
    if (fin && !has_out) {
      a.st[kRfRed].n_steps = 0;
      break;
    }
    const ttlh_instr* pj = fin ? prog : red[j].prog;
    const ttlh_operand* ij = fin ? in : red[j].in;
    const int nj = fin ? n_instr : red[j].n_instr;
    RfStage& st = a.st[fin ? kRfRed : j];
    EltArgs e = {};
    ProgInfo pi;
    const int rc = decode_program(who, pj, ij, nj, y0, x0, h, w, e, pi);
    if (rc != TTLH_OK) return rc;
    for (int k = 0; k < nj; ++k)
      TTLH_REQUIRE(is_inline_op(pj[k].form, pj[k].op), TTLH_EUNSUPPORTED,
                   "%s: step %d uses op %d (the fused set is + - * / max min exp sqrt rsqrt abs "
                   "neg relu recip)", who, k, pj[k].op);
    TTLH_REQUIRE(pi.vec, TTLH_EUNSUPPORTED, "%s: an operand does not admit 16-byte chunks", who);
    if (!fin) {
      const ttlh_row_reduce& r = red[j];
      st.kind = r.kind;
      st.out_dtype = r.out_dtype;
      st.out_pad = r.out_pad;
      st.scaler_dtype = r.scaler_dtype;
      st.scale_imm = r.scale_imm;
      st.scaler = r.scaler;
      st.out = r.out;
      st.out_ld = r.out_ld;
    }
    uint8_t src_of[TTLH_MAX_INSTR] = {};
    for (int i = 0; i < pi.n_ops; ++i) {
      const EltOperand& o = e.ops[i];
      int src = -1;
      for (int p = 0; p < j && p < n_red && src < 0; ++p)
        if (reads_row_result(o, red[p], y0, x0, h, w)) src = RS_SC + p;
      uintptr_t lo, hi;
      operand_span(o, y0, x0, h, w, &lo, &hi);
      if (src < 0) {
        for (int p = 0; p < n_red; ++p)
          TTLH_REQUIRE(!overlap(lo, hi, rlo[p], rhi[p]), TTLH_EUNSUPPORTED,
                       "%s: stage %d reads reduction %d's results other than as its rows' values",
                       who, j, p);
        // constant along the row (a column broadcast): a row scalar
        if (o.cs == 0 || o.cmask == 0 || w == 1) {
          for (int q = 0; q < a.n_row && src < 0; ++q)
            if (same_map(a.row[q], o)) src = RS_SC + kRfRed + q;
          if (src < 0 && a.n_row < kRfRow) {
            a.row[a.n_row] = o;
            src = RS_SC + kRfRed + a.n_row++;
          }
        }
        // rows held in registers: identity-mapped bf16 operands read once (a
        // row re-read by every row, stride 0, is left to the caches)
        if (src < 0 && o.dtype == TTLH_BF16 && o.rmask == -1 && o.cmask == -1 && o.cs == 1 &&
            o.vec && (o.rs != 0 || h == 1)) {
          for (int q = 0; q < n_res && src < 0; ++q)
            if (same_map(a.res[q], o)) src = RS_RES + q;
          if (src < 0 && n_res < kRfRes) {
            a.res[n_res] = o;
            src = RS_RES + n_res++;
          }
        }
      }
      if (src < 0) {
        TTLH_REQUIRE(n_mem < kRfMem, TTLH_EUNSUPPORTED, "%s: more than %d non-resident operands",
                     who, kRfMem);
        a.mem[n_mem] = o;
        src = RS_MEM + n_mem++;
      }
      src_of[i] = static_cast<uint8_t>(src);
      if (overlap(lo, hi, out_lo, out_hi)) {
        // only an operand read element for element in place (loaded before the store)
        const bool in_place = src < RS_MEM && out_dtype == TTLH_BF16 && o.rs == out_ld &&
                              reinterpret_cast<uintptr_t>(o.ptr) +
                                      static_cast<uintptr_t>((o.roff * o.rs + o.coff) * 2) ==
                                  reinterpret_cast<uintptr_t>(out);
        TTLH_REQUIRE(in_place, TTLH_EUNSUPPORTED,
                     "%s: stage %d reads the output other than element for element", who, j);
      }
    }
    TTLH_REQUIRE(rf_compile(e, nj, src_of, st), TTLH_EUNSUPPORTED,
                 "%s: stage %d is not a chain over the row (a binary op of two values computed "
                 "from the row's elements, or more than %d derived row values)", who, j, kRfNodes);
  }
  rf_choose_kept(a);
  const bool wide = w >= 2048;
  const int64_t groups = wide ? h : (h + 3) / 4;  // row groups: a workgroup's rows
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t lanes = wide ? 256 : 64;
  const int nch = static_cast<int>((w + 8 * lanes - 1) / (8 * lanes));  // 1..kRfChunks
  RfSoftmax sm;
  if (n_res == 1 && n_mem == 0 && a.n_row == 0 && rf_softmax_form(a, &sm)) {
    TTLH_REQUIRE(groups < (int64_t(1) << 31), TTLH_EUNSUPPORTED, "%s: region too large", who);
    const dim3 grid(static_cast<uint32_t>(groups)), block(256);
#define TTLH_SM(L)                                                                            \
  switch (nch) {                                                                              \
    case 1: hipLaunchKernelGGL((softmax_rows_kernel<L, 1>), grid, block, 0, s, a, sm); break; \
    case 2: hipLaunchKernelGGL((softmax_rows_kernel<L, 2>), grid, block, 0, s, a, sm); break; \
    case 3: hipLaunchKernelGGL((softmax_rows_kernel<L, 3>), grid, block, 0, s, a, sm); break; \
    default: hipLaunchKernelGGL((softmax_rows_kernel<L, 4>), grid, block, 0, s, a, sm); break; \
  }
    if (wide) {
      TTLH_SM(256)
    } else {
      TTLH_SM(64)
    }
#undef TTLH_SM
    return check_launch("softmax_rows_kernel");
  }
  if (n_res == 1 && rf_norm_form(a)) {
    TTLH_REQUIRE(groups < (int64_t(1) << 31), TTLH_EUNSUPPORTED, "%s: region too large", who);
    const dim3 grid(static_cast<uint32_t>(groups)), block(256);
#define TTLH_NORM(L)                                                                         \
  switch (nch) {                                                                             \
    case 1: hipLaunchKernelGGL((norm_rows_kernel<L, 1>), grid, block, 0, s, a); break;      \
    case 2: hipLaunchKernelGGL((norm_rows_kernel<L, 2>), grid, block, 0, s, a); break;      \
    case 3: hipLaunchKernelGGL((norm_rows_kernel<L, 3>), grid, block, 0, s, a); break;      \
    default: hipLaunchKernelGGL((norm_rows_kernel<L, 4>), grid, block, 0, s, a); break;     \
  }
    if (wide) {
      TTLH_NORM(256)
    } else {
      TTLH_NORM(64)
    }
#undef TTLH_NORM
    return check_launch("norm_rows_kernel");
  }
  // one instantiation per (lanes, resident operands, chunks per lane)
#define TTLH_RF3(L, R, C) return rf_launch<L, R, C>(a, groups, s)
#define TTLH_RF2(L, R)                   \
  switch (nch) {                         \
    case 1: TTLH_RF3(L, R, 1);           \
    case 2: TTLH_RF3(L, R, 2);           \
    case 3: TTLH_RF3(L, R, 3);           \
    default: TTLH_RF3(L, R, 4);          \
  }
#define TTLH_RF(L)                       \
  switch (n_res) {                       \
    case 0: TTLH_RF2(L, 0)               \
    case 1: TTLH_RF2(L, 1)               \
    case 2: TTLH_RF2(L, 2)               \
    default: TTLH_RF2(L, 3)              \
  }
  if (wide) TTLH_RF(256)
  TTLH_RF(64)
#undef TTLH_RF
#undef TTLH_RF2
#undef TTLH_RF3
}

}  // namespace
}  // namespace ttlh
