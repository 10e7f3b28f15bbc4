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

#include "ttlh_common.h"

namespace ttlh {
namespace {

typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef const __attribute__((address_space(1))) u32x4 gu32x4;

struct EltOperand {
  const void* ptr;
  int64_t rs, cs;          // row / col stride (elements)
  int64_t rmask, cmask;    // coordinate masks (-1 or 31)
  int64_t roff, coff;      // coordinate offsets
  int32_t dtype;
  int32_t vec;             // 1: 16-byte vector loads are legal for this operand
};

// Internal step encoding, decoded on the host from the ABI forms.
//   src:  where the step's input value comes from
//   kind: what the step does with it
enum : uint8_t { SRC_NONE = 0, SRC_OPERAND = 1, SRC_IMM = 2, SRC_POP = 3 };
enum : uint8_t { K_SET = 0, K_PUSH = 1, K_UNARY = 2, K_BIN = 3, K_BIN_REV = 4 };
struct Ins {
  uint8_t kind, src, op, rnd;
  uint8_t arg;  // operand index (consumption order) for SRC_OPERAND steps
  uint8_t pad[3];
  float imm;
};

struct EltArgs {
  Ins prog[TTLH_MAX_INSTR];
  EltOperand ops[TTLH_MAX_INSTR];  // in consumption order
  void* out;
  int64_t out_ld;
  int64_t y0, x0;
  uint32_t cpr;            // chunks per output row
  uint32_t total;          // total chunks
  uint32_t magic, shift;   // chunk / cpr == umulhi-based division (see divide())
  int32_t n_instr, n_ops, out_dtype;
};

__device__ __forceinline__ f32x8 splat(float s) { return f32x8{s, s, s, s, s, s, s, s}; }

// n / d for the host-chosen (magic, shift) pair, valid for n < 2^31
// (Granlund-Montgomery round-up method; d = 1 is magic 0, shift 0).
__device__ __forceinline__ uint32_t divide(uint32_t n, uint32_t magic, uint32_t shift) {
  const uint32_t t = __umulhi(n, magic);
  return (t + n) >> shift;
}

// Raw bits of one operand chunk: the aligned 16-byte block that holds it.
// bf16: q holds 8 packed values (vector operands) or the block containing the
// single element of a broadcast / 1-wide operand (picked by `sel`); f32
// vector operands also use q1.  Loading the aligned 16-byte block that holds a
// valid element cannot leave that element's page, so it cannot fault, and it
// keeps each operand load one unconditional global_load_dwordx4: no branch
// join between loads, so they all stay in flight together.
struct Raw {
  u32x4 q;
  u32x4 q1;
  uint32_t sel;
};

template <bool OFF32>
__device__ __forceinline__ uintptr_t operand_addr(const EltOperand& op, int64_t y, int64_t x) {
  if constexpr (OFF32) {
    const uint32_t iy = (static_cast<uint32_t>(y) & static_cast<uint32_t>(op.rmask)) +
                        static_cast<uint32_t>(op.roff);
    const uint32_t ix = (static_cast<uint32_t>(x) & static_cast<uint32_t>(op.cmask)) +
                        static_cast<uint32_t>(op.coff);
    const uint32_t e = iy * static_cast<uint32_t>(op.rs) + ix * static_cast<uint32_t>(op.cs);
    return reinterpret_cast<uintptr_t>(op.ptr) + (op.dtype == TTLH_BF16 ? 2ull : 4ull) * e;
  } else {
    const int64_t iy = (y & op.rmask) + op.roff;
    const int64_t ix = (x & op.cmask) + op.coff;
    const int64_t esz = op.dtype == TTLH_BF16 ? 2 : 4;
    return reinterpret_cast<uintptr_t>(op.ptr) + (iy * op.rs + ix * op.cs) * esz;
  }
}

template <int VEC, bool BF16>
__device__ __forceinline__ Raw load_raw(const EltOperand& op, uintptr_t u) {
  Raw r;
  r.q = *reinterpret_cast<gu32x4*>(u & ~uintptr_t(15));
  r.sel = static_cast<uint32_t>(u & 15u);
  if constexpr (!BF16) {
    if (VEC == 8 && op.dtype == TTLH_F32 && op.vec) r.q1 = *reinterpret_cast<gu32x4*>(u + 16);
  }
  return r;
}

__device__ __forceinline__ uint32_t pick_dword(const u32x4 q, uint32_t byte) {
  const uint32_t w = byte >> 2;
  const uint32_t lo = (w & 1) ? q.y : q.x;
  const uint32_t hi = (w & 1) ? q.w : q.z;
  return (w & 2) ? hi : lo;
}

// ALLVEC: the caller guarantees op.vec (8 distinct consecutive elements).
template <int VEC, bool BF16, bool ALLVEC = false>
__device__ __forceinline__ f32x8 to_f32(const EltOperand& op, const Raw& r) {
  if (BF16 || op.dtype == TTLH_BF16) {
    if (VEC == 8 && (ALLVEC || op.vec)) {
      const u32x4 q = r.q;
      return f32x8{__uint_as_float(q.x << 16), __uint_as_float(q.x & 0xffff0000u),
                   __uint_as_float(q.y << 16), __uint_as_float(q.y & 0xffff0000u),
                   __uint_as_float(q.z << 16), __uint_as_float(q.z & 0xffff0000u),
                   __uint_as_float(q.w << 16), __uint_as_float(q.w & 0xffff0000u)};
    }
    const uint32_t d = pick_dword(r.q, r.sel);
    return splat(__uint_as_float((r.sel & 2) ? (d & 0xffff0000u) : (d << 16)));
  }
  if (VEC == 8 && (ALLVEC || op.vec))
    return f32x8{__uint_as_float(r.q.x), __uint_as_float(r.q.y), __uint_as_float(r.q.z),
                 __uint_as_float(r.q.w), __uint_as_float(r.q1.x), __uint_as_float(r.q1.y),
                 __uint_as_float(r.q1.z), __uint_as_float(r.q1.w)};
  return splat(__uint_as_float(pick_dword(r.q, r.sel)));
}

// exp(x) = 2^(x log2 e), branch-free.  t = fl(x * log2e); the rounding
// error of that product and the tail of log2 e are recovered with two FMAs
// and folded back as 2^t * (1 + lo ln2), which keeps the result within about
// one fp32 ulp of exp(x).  Results below the normal range are computed as
// 2^(t + 64) * 2^-64 so v_exp_f32 never sees a subnormal output; inf / NaN
// inputs and overflow fall out of v_exp_f32 with the correction forced to 0.
template <typename F>
__device__ __forceinline__ f32x8 map8(f32x8 a, F f);

__device__ __forceinline__ float exp1(float x) {
  constexpr float kL2E = 1.44269502e+00f;     // log2(e) rounded to fp32
  constexpr float kL2ELo = 1.92596299e-08f;   // log2(e) - kL2E
  constexpr float kLn2 = 6.93147182e-01f;
  const float t = x * kL2E;
  float lo = __builtin_fmaf(x, kL2E, -t);
  lo = __builtin_fmaf(x, kL2ELo, lo);
  const bool fin = __builtin_fabsf(t) < 128.0f;  // false for inf / NaN / overflow
  const bool tiny = t < -125.0f;
  const float p = __builtin_amdgcn_exp2f(tiny ? t + 64.0f : t);
  // (no correction where p may be inf: inf * 0 would make a NaN)
  const float r = fin ? __builtin_fmaf(p, lo * kLn2, p) : p;
  return tiny ? r * 5.42101086e-20f : r;  // 2^-64
}

__device__ __forceinline__ f32x8 vexp(f32x8 x) {
  return map8(x, [](float v) { return exp1(v); });
}

// The same function with the range handling hoisted out: when every lane's
// 8 arguments satisfy |x log2 e| < 125 (no overflow, no subnormal result, no
// inf / NaN) the wave takes the straight-line FMA-split path, which computes
// exactly what exp1 computes for such arguments; otherwise it runs exp1.
__device__ __forceinline__ f32x8 vexp_uniform(f32x8 x) {
  constexpr float kL2E = 1.44269502e+00f;
  constexpr float kL2ELo = 1.92596299e-08f;
  constexpr float kLn2 = 6.93147182e-01f;
  const f32x8 t = x * kL2E;
  bool ok = true;
#pragma unroll
  for (int e = 0; e < 8; ++e) ok &= __builtin_fabsf(t[e]) < 125.0f;
  if (!__all(ok)) return vexp(x);
  f32x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float lo = __builtin_fmaf(x[e], kL2E, -t[e]);
    lo = __builtin_fmaf(x[e], kL2ELo, lo);
    const float p = __builtin_amdgcn_exp2f(t[e]);
    r[e] = __builtin_fmaf(p, lo * kLn2, p);
  }
  return r;
}

template <typename F>
__device__ __forceinline__ f32x8 map8(f32x8 a, F f) {
  f32x8 t;
#pragma unroll
  for (int e = 0; e < 8; ++e) t[e] = f(a[e]);
  return t;
}

// torch semantics: NaN-propagating maximum / minimum, floor division,
// Python-style remainder.
template <bool FULL>
__device__ __forceinline__ f32x8 binary(int op, f32x8 a, f32x8 b) {
  if constexpr (!FULL) {  // common ops only: keeps the fast variant inside 64 VGPRs
    switch (op) {
      case TTLH_OP_ADD: return a + b;
      case TTLH_OP_SUB: return a - b;
      default: return a * b;  // TTLH_OP_MUL
    }
  }
  switch (op) {
    case TTLH_OP_ADD: return a + b;
    case TTLH_OP_SUB: return a - b;
    case TTLH_OP_MUL: return a * b;
    case TTLH_OP_DIV: return a / b;
    case TTLH_OP_MAX:
    case TTLH_OP_MIN: {
      f32x8 t;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float m = op == TTLH_OP_MAX ? fmaxf(a[e], b[e]) : fminf(a[e], b[e]);
        t[e] = (a[e] != a[e] || b[e] != b[e]) ? __builtin_nanf("") : m;
      }
      return t;
    }
    case TTLH_OP_POW: {
      f32x8 t;
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = powf(a[e], b[e]);
      return t;
    }
    case TTLH_OP_FLOORDIV: return map8(a / b, [](float v) { return floorf(v); });
    default: {  // TTLH_OP_MOD
      f32x8 t;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float r = fmodf(a[e], b[e]);
        if (r != 0.0f && ((r < 0.0f) != (b[e] < 0.0f))) r += b[e];
        t[e] = r;
      }
      return t;
    }
  }
}

template <bool FULL>
__device__ __forceinline__ f32x8 unary(int op, f32x8 a, float imm) {
  if constexpr (!FULL) {
    switch (op) {
      case TTLH_OP_EXP: return vexp(a);
      case TTLH_OP_NEG: return -a;
      case TTLH_OP_ABS: return map8(a, [](float v) { return fabsf(v); });
      case TTLH_OP_RELU: return map8(a, [](float v) { return v != v ? v : fmaxf(v, 0.0f); });
      default: return 1.0f / a;  // TTLH_OP_RECIP
    }
  }
  switch (op) {
    case TTLH_OP_EXP: return vexp(a);
    case TTLH_OP_LOG: return map8(a, [](float v) { return logf(v); });
    case TTLH_OP_SQRT: return map8(a, [](float v) { return sqrtf(v); });
    case TTLH_OP_RSQRT: return map8(a, [](float v) { return 1.0f / sqrtf(v); });
    case TTLH_OP_TANH: return map8(a, [](float v) { return tanhf(v); });
    case TTLH_OP_ABS: return map8(a, [](float v) { return fabsf(v); });
    case TTLH_OP_NEG: return -a;
    case TTLH_OP_RELU: return map8(a, [](float v) { return v != v ? v : fmaxf(v, 0.0f); });
    case TTLH_OP_SIGMOID: return map8(a, [](float v) { return 1.0f / (1.0f + expf(-v)); });
    case TTLH_OP_RECIP: return 1.0f / a;
    default: return map8(a, [imm](float v) { return powf(v, imm); });  // TTLH_OP_POWI
  }
}

__device__ __forceinline__ f32x8 round_bf16x8(f32x8 a) {
  f32x8 r;
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const uint32_t u = cvt_pk_bf16x2(a[e], a[e + 1]);
    r[e] = __uint_as_float(u << 16);
    r[e + 1] = __uint_as_float(u & 0xffff0000u);
  }
  return r;
}

__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) { return cvt_pk_bf16x2(lo, hi); }

template <int VEC, bool BF16>
__device__ __forceinline__ f32x8 operand_value(const EltArgs& args, int idx, const Raw& q0,
                                               const Raw& q1, const Raw& q2, const Raw& q3) {
  switch (idx) {
    case 0: return to_f32<VEC, BF16>(args.ops[0], q0);
    case 1: return to_f32<VEC, BF16>(args.ops[1], q1);
    case 2: return to_f32<VEC, BF16>(args.ops[2], q2);
    default: return to_f32<VEC, BF16>(args.ops[3], q3);
  }
}

// One program step.  The operand a step consumes was numbered on the host
// (Ins.arg); with PRELOAD it is selected from q0..q3 by a uniform switch,
// otherwise it is loaded here.  s0 / s1 (the stack below acc) fold away when
// !STACK.
template <int VEC, bool PRELOAD, bool BF16, bool STACK, bool OFF32, bool FULL>
__device__ __forceinline__ void run_step(const EltArgs& args, const Ins ins, f32x8& acc, f32x8& s0,
                                         f32x8& s1, const Raw& q0, const Raw& q1, const Raw& q2,
                                         const Raw& q3, int64_t y, int64_t x) {
  f32x8 v = acc;
  if (ins.src == SRC_OPERAND) {
    if constexpr (PRELOAD) {
      v = operand_value<VEC, BF16>(args, ins.arg, q0, q1, q2, q3);
    } else {
      const EltOperand& op = args.ops[ins.arg];
      v = to_f32<VEC, BF16>(op, load_raw<VEC, BF16>(op, operand_addr<OFF32>(op, y, x)));
    }
  } else if (ins.src == SRC_IMM) {
    v = splat(ins.imm);
  } else if (STACK && ins.src == SRC_POP) {
    v = s0;
    s0 = s1;
  }
  switch (ins.kind) {
    case K_SET: acc = v; break;
    case K_PUSH:
      if constexpr (STACK) {
        s1 = s0;
        s0 = acc;
      }
      acc = v;
      break;
    case K_UNARY: acc = unary<FULL>(ins.op, acc, ins.imm); break;
    case K_BIN: acc = binary<FULL>(ins.op, acc, v); break;
    default: acc = binary<FULL>(ins.op, v, acc); break;  // K_BIN_REV
  }
  if (ins.rnd == TTLH_BF16) acc = round_bf16x8(acc);
}

// Runs the program on one chunk: a runtime step loop (one copy of the
// dispatch code; unrolling it raises register pressure past 8 waves/SIMD).
template <int VEC, bool PRELOAD, bool BF16, bool STACK, bool OFF32, bool FULL>
__device__ __forceinline__ f32x8 run_program(const EltArgs& args, const Raw& q0, const Raw& q1,
                                             const Raw& q2, const Raw& q3, int64_t y, int64_t x) {
  f32x8 acc = splat(0.0f), s0 = acc, s1 = acc;
  for (int k = 0; k < args.n_instr; ++k)
    run_step<VEC, PRELOAD, BF16, STACK, OFF32, FULL>(args, args.prog[k], acc, s0, s1, q0, q1, q2,
                                                     q3, y, x);
  return acc;
}

template <int VEC, typename Args>
__device__ __forceinline__ void store_chunk(const Args& args, int64_t y, int64_t x, f32x8 acc) {
  const int64_t off = y * args.out_ld + x;
  if (args.out_dtype == TTLH_BF16) {
    uint16_t* p = static_cast<uint16_t*>(args.out) + off;
    if constexpr (VEC == 8) {
      u32x4 q;
      q.x = cvt_pk_bf16(acc[0], acc[1]);
      q.y = cvt_pk_bf16(acc[2], acc[3]);
      q.z = cvt_pk_bf16(acc[4], acc[5]);
      q.w = cvt_pk_bf16(acc[6], acc[7]);
      __builtin_nontemporal_store(q, reinterpret_cast<u32x4*>(p));
    } else {
      *p = __builtin_bit_cast(uint16_t, static_cast<__bf16>(acc[0]));
    }
  } else {
    float* p = static_cast<float*>(args.out) + off;
    if constexpr (VEC == 8) {
      f32x4 a = {acc[0], acc[1], acc[2], acc[3]};
      f32x4 b = {acc[4], acc[5], acc[6], acc[7]};
      __builtin_nontemporal_store(a, reinterpret_cast<f32x4*>(p));
      __builtin_nontemporal_store(b, reinterpret_cast<f32x4*>(p + 4));
    } else {
      *p = acc[0];
    }
  }
}

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
    case C_RELU: return map8(acc, [](float t) { return t != t ? t : fmaxf(t, 0.0f); });
    default: return 1.0f / acc;  // C_RECIP
  }
}

// Each lane runs U chunks, 256 chunks apart (a wave's loads stay 1 KiB
// contiguous per operand); every load of every chunk is issued before the
// first arithmetic.  Lanes past the end clamp their chunk index for the loads
// (an in-bounds re-read) and skip the store.
#ifndef TTLH_CHAIN_U
#define TTLH_CHAIN_U 1
#endif
constexpr int kChainU = TTLH_CHAIN_U;

#ifndef TTLH_CHAIN_WAVES
#define TTLH_CHAIN_WAVES 8
#endif
template <int N, bool BF16, bool ALLVEC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(BF16 ? TTLH_CHAIN_WAVES : 6, BF16 ? TTLH_CHAIN_WAVES : 6)))
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

// Launches the stream kernel when `c` qualifies (see above); returns false
// to let the caller fall back to the chain kernel.
bool try_stream(const ChainArgs& c, int n, hipStream_t s, int* status) {
  if (n > 4 || c.out_ld >= (int64_t(1) << 31)) return false;
  StreamArgs a{};
  unsigned mask = 0;
  for (int k = 0; k < n; ++k) {
    const bool reads = k == 0 || c.imm_src[k] == 0;
    if (reads) {
      const EltOperand& o = c.ops[k];
      if (o.dtype != TTLH_BF16 || !o.vec || o.rs >= (int64_t(1) << 24)) return false;
      const int64_t ymax = o.rmask == -1 ? c.y0 + int64_t(c.total / c.cpr) - 1 + o.roff : 31 + o.roff;
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

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool is_binary(int op) { return op >= TTLH_OP_ADD && op <= TTLH_OP_MOD; }
bool is_unary(int op) { return op >= TTLH_OP_EXP && op <= TTLH_OP_POWI; }
// ops the common (fast) variants implement
bool is_common(int op) {
  return op == TTLH_OP_ADD || op == TTLH_OP_SUB || op == TTLH_OP_MUL || op == TTLH_OP_EXP || op == TTLH_OP_NEG || op == TTLH_OP_ABS || op == TTLH_OP_RELU ||
         op == TTLH_OP_RECIP;
}

// magic numbers for divide(): n / d == (umulhi(n, m) + n) >> s for n < 2^31,
// with s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1.
void division_magic(uint32_t d, uint32_t* m, uint32_t* s) {
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  *s = l;
  *m = static_cast<uint32_t>(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1);
  if (d == 1) *m = 0;
}

// largest element offset an operand can reach over the region (decides the
// 32-bit offset path)
int64_t max_offset(const ttlh_operand& o, int64_t y0, int64_t x0, int64_t h, int64_t w) {
  const int64_t ymax = o.row_mask == -1 ? y0 + h - 1 + o.row_off : 31 + o.row_off;
  const int64_t xmax = o.col_mask == -1 ? x0 + w - 1 + o.col_off : 31 + o.col_off;
  return ymax * o.row_stride + xmax * o.col_stride;
}

}  // namespace
}  // namespace ttlh

using namespace ttlh;

extern "C" int ttlh_eltwise(const ttlh_instr* prog, const ttlh_operand* in, int n_instr, void* out,
                            int out_dtype, int64_t out_ld, int64_t y0, int64_t x0, int64_t h,
                            int64_t w, void* stream) {
  clear_error();
  TTLH_REQUIRE(prog && in && n_instr > 0 && n_instr <= TTLH_MAX_INSTR, TTLH_EINVAL,
               "ttlh_eltwise: program must have 1..%d steps (got %d)", TTLH_MAX_INSTR, n_instr);
  TTLH_REQUIRE(out && (out_dtype == TTLH_BF16 || out_dtype == TTLH_F32), TTLH_EINVAL,
               "ttlh_eltwise: bad output pointer or dtype");
  TTLH_REQUIRE(h >= 0 && w >= 0 && y0 >= 0 && x0 >= 0 && out_ld >= x0 + w, TTLH_EINVAL,
               "ttlh_eltwise: bad output region");

  EltArgs a = {};
  int depth = 0;  // values on the stack including acc
  int max_depth = 0;
  bool all_bf16 = true;
  int n_ops = 0;
  bool full = false;  // program uses an op outside the common set
  bool off32 = (y0 + h) * out_ld < (int64_t(1) << 31);
  bool vec = (w % 8 == 0) && (x0 % 8 == 0) && (out_ld % 8 == 0) && aligned16(out);
  for (int k = 0; k < n_instr; ++k) {
    const ttlh_instr& p = prog[k];
    const int f = p.form;
    const bool uses_operand = f == TTLH_FORM_LOAD || f == TTLH_FORM_PUSH || f == TTLH_FORM_BIN ||
                              f == TTLH_FORM_BIN_REV;
    TTLH_REQUIRE(f >= TTLH_FORM_LOAD && f <= TTLH_FORM_BIN_POP, TTLH_EINVAL,
                 "ttlh_eltwise: bad form %d at step %d", f, k);
    TTLH_REQUIRE(p.rnd == TTLH_BF16 || p.rnd == TTLH_F32, TTLH_EINVAL,
                 "ttlh_eltwise: bad rounding mode at step %d", k);
    if (f == TTLH_FORM_UNARY)
      TTLH_REQUIRE(is_unary(p.op), TTLH_EINVAL, "ttlh_eltwise: step %d needs a unary opcode", k);
    if (f >= TTLH_FORM_BIN)
      TTLH_REQUIRE(is_binary(p.op), TTLH_EINVAL, "ttlh_eltwise: step %d needs a binary opcode", k);
    // stack discipline
    if (f == TTLH_FORM_LOAD || f == TTLH_FORM_CONST) {
      TTLH_REQUIRE(depth == 0, TTLH_EINVAL, "ttlh_eltwise: LOAD/CONST at step %d on a live stack", k);
      depth = 1;
    } else if (f == TTLH_FORM_PUSH || f == TTLH_FORM_PUSH_CONST) {
      TTLH_REQUIRE(depth >= 1 && depth < TTLH_MAX_STACK, TTLH_EINVAL,
                   "ttlh_eltwise: stack overflow at step %d", k);
      ++depth;
    } else if (f == TTLH_FORM_BIN_POP) {
      TTLH_REQUIRE(depth >= 2, TTLH_EINVAL, "ttlh_eltwise: stack underflow at step %d", k);
      --depth;
    } else {
      TTLH_REQUIRE(depth >= 1, TTLH_EINVAL, "ttlh_eltwise: step %d reads an empty stack", k);
    }
    max_depth = depth > max_depth ? depth : max_depth;
    if ((f == TTLH_FORM_UNARY || f >= TTLH_FORM_BIN) && !is_common(p.op)) full = true;
    Ins& q = a.prog[k];
    q.op = p.op;
    q.rnd = p.rnd;
    q.imm = p.imm;
    switch (f) {
      case TTLH_FORM_LOAD: q.kind = K_SET; q.src = SRC_OPERAND; break;
      case TTLH_FORM_PUSH: q.kind = K_PUSH; q.src = SRC_OPERAND; break;
      case TTLH_FORM_CONST: q.kind = K_SET; q.src = SRC_IMM; break;
      case TTLH_FORM_PUSH_CONST: q.kind = K_PUSH; q.src = SRC_IMM; break;
      case TTLH_FORM_UNARY: q.kind = K_UNARY; q.src = SRC_NONE; break;
      case TTLH_FORM_BIN: q.kind = K_BIN; q.src = SRC_OPERAND; break;
      case TTLH_FORM_BIN_REV: q.kind = K_BIN_REV; q.src = SRC_OPERAND; break;
      case TTLH_FORM_BIN_IMM: q.kind = K_BIN; q.src = SRC_IMM; break;
      case TTLH_FORM_BIN_IMM_REV: q.kind = K_BIN_REV; q.src = SRC_IMM; break;
      default: q.kind = K_BIN_REV; q.src = SRC_POP; break;  // BIN_POP: op(pop, acc)
    }
    if (!uses_operand) continue;
    q.arg = static_cast<uint8_t>(n_ops);
    const ttlh_operand& o = in[k];
    TTLH_REQUIRE(o.ptr && (o.dtype == TTLH_BF16 || o.dtype == TTLH_F32), TTLH_EINVAL,
                 "ttlh_eltwise: operand %d has a null pointer or bad dtype", k);
    TTLH_REQUIRE(o.row_mask == -1 || o.row_mask == 31, TTLH_EINVAL,
                 "ttlh_eltwise: operand %d row_mask must be -1 or 31", k);
    TTLH_REQUIRE(o.col_mask == -1 || o.col_mask == 31, TTLH_EINVAL,
                 "ttlh_eltwise: operand %d col_mask must be -1 or 31", k);
    TTLH_REQUIRE(o.row_stride >= 0 && o.col_stride >= 0, TTLH_EINVAL,
                 "ttlh_eltwise: operand %d has a negative stride", k);
    EltOperand& e = a.ops[n_ops++];
    e.ptr = o.ptr;
    e.rs = o.row_stride;
    e.cs = o.col_stride;
    e.rmask = o.row_mask;
    e.cmask = o.col_mask;
    e.roff = o.row_off;
    e.coff = o.col_off;
    e.dtype = o.dtype;
    all_bf16 = all_bf16 && o.dtype == TTLH_BF16;
    const int esz = o.dtype == TTLH_BF16 ? 2 : 4;
    e.vec = o.col_stride == 1 && aligned16(o.ptr) && ((o.row_stride * esz) % 16 == 0) &&
            ((o.col_off * esz) % 16 == 0) && ((x0 * esz) % 16 == 0);
    // stride-0 (broadcast) operands keep the 8-wide path; others need alignment
    if (o.col_stride != 0 && !e.vec) vec = false;
    const int64_t mo = max_offset(o, y0, x0, h, w);
    if (mo >= (int64_t(1) << 31) || o.row_off < 0 || o.col_off < 0) off32 = false;
  }
  TTLH_REQUIRE(depth == 1, TTLH_EINVAL, "ttlh_eltwise: program leaves %d values on the stack",
               depth);
  if (h == 0 || w == 0) return TTLH_OK;
  a.out = out;
  a.out_ld = out_ld;
  a.y0 = y0;
  a.x0 = x0;
  a.n_instr = n_instr;
  a.n_ops = n_ops;
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
  const bool preload = n_ops >= 1 && n_ops <= 4;  // preload reads operand 0 unconditionally
  // rare shapes: one generic variant each
  if (!off32) return vec ? launch<8, false, false, true, false, true>(a, s)
                         : launch<1, false, false, true, false, true>(a, s);
  if (!vec) return launch<1, false, false, true, true, true>(a, s);
  ChainArgs chain;
  if (make_chain(prog, n_instr, a, &chain)) {
    int status = TTLH_OK;
    if (all_bf16 && try_stream(chain, n_instr, s, &status)) return status;
    return all_bf16 ? dispatch_chain<true>(chain, n_instr, s) : dispatch_chain<false>(chain, n_instr, s);
  }
  if (!preload) return launch<8, false, false, true, true, true>(a, s);
  if (full) return launch<8, true, false, true, true, true>(a, s);
  // common ops, 8-wide, preloaded
  if (!all_bf16) return launch<8, true, false, true, true, false>(a, s);
  return max_depth > 1 ? launch<8, true, true, true, true, false>(a, s)
                       : launch<8, true, true, false, true, false>(a, s);
}
