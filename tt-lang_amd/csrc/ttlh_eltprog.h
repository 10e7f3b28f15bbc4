// The fused elementwise tile program shared by the kernels that evaluate it:
// ttlh_eltwise's interpreters and ttlh_reduce (eltwise.hip) and the GEMM whose
// epilogue runs it on the rounded product (matmul.hip).  Program format and
// operand addressing: include/ttlhip.h (ttlh_instr, ttlh_operand).  One
// definition of every op, so a fused epilogue rounds exactly as the
// elementwise launch it replaces.
#pragma once

#include <utility>

#include "ttlh_common.h"

namespace ttlh {
namespace {

typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef const __attribute__((address_space(1))) u32x4 gu32x4;

struct EltOperand {
  const void* ptr;
  int64_t rs, cs;          // row / col stride (elements)
  int64_t rmask, cmask;    // coordinate masks (-1, 31, 0 or ~31)
  int64_t roff, coff;      // coordinate offsets
  int32_t dtype;
  int32_t vec;             // 1: 16-byte vector loads are legal for this operand
};

// the operand coordinate masks: identity, a fixed tile re-used over the
// grid (31), one fixed row / column (0), row / column 0 of every tile (~31)
bool valid_mask(int64_t m) { return m == -1 || m == 31 || m == 0 || m == ~int64_t(31); }

// largest masked coordinate (before the offset) over [0, hi]
int64_t mask_max(int64_t m, int64_t hi) {
  if (m == -1) return hi;
  if (m == 31) return 31;
  if (m == 0) return 0;
  return hi & ~int64_t(31);
}

// Internal step encoding, decoded on the host from the ABI forms.
//   src:  where the step's input value comes from
//   kind: what the step does with it
enum : uint8_t { SRC_NONE = 0, SRC_OPERAND = 1, SRC_IMM = 2, SRC_POP = 3 };
enum : uint8_t { K_SET = 0, K_PUSH = 1, K_UNARY = 2, K_BIN = 3, K_BIN_REV = 4 };
struct Ins {
  uint8_t kind, src, op, rnd;
  uint8_t arg;  // operand index (consumption order) for SRC_OPERAND steps
  uint8_t pad[3];
  float imm, imm2;
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

template <typename F>
__device__ __forceinline__ f32x8 map8(f32x8 a, F f);

constexpr float kExpL2E = 1.44269502e+00f;    // log2(e) rounded to fp32
constexpr float kExpL2ELo = 1.92596299e-08f;  // log2(e) - kExpL2E
constexpr float kExpLn2 = 6.93147182e-01f;

// exp(x) = 2^(x log2 e), branch-free.  t = fl(x * log2e); the rounding
// error of that product and the tail of log2 e are recovered with two FMAs
// and folded back as 2^t * (1 + lo ln2), which keeps the result within about
// one fp32 ulp of exp(x).  Results below the normal range are computed as
// 2^(t + 64) * 2^-64 so v_exp_f32 never sees a subnormal output; inf / NaN
// inputs and overflow fall out of v_exp_f32 with the correction forced to 0.
__device__ __forceinline__ float exp1(float x) {
  const float t = x * kExpL2E;
  float lo = __builtin_fmaf(x, kExpL2E, -t);
  lo = __builtin_fmaf(x, kExpL2ELo, lo);
  const bool fin = __builtin_fabsf(t) < 128.0f;  // false for inf / NaN / overflow
  const bool tiny = t < -125.0f;
  const float p = __builtin_amdgcn_exp2f(tiny ? t + 64.0f : t);
  // (no correction where p may be inf: inf * 0 would make a NaN)
  const float r = fin ? __builtin_fmaf(p, lo * kExpLn2, p) : p;
  return tiny ? r * 5.42101086e-20f : r;  // 2^-64
}

// Arguments with |x log2 e| < 125 need none of exp1's range handling (no
// overflow, no subnormal result, no inf / NaN): exp1_in_range computes
// exactly what exp1 computes for them, straight-line.
__device__ __forceinline__ bool exp1_in_range(float x) {
  return __builtin_fabsf(x * kExpL2E) < 125.0f;
}
__device__ __forceinline__ float exp1_fast(float x) {
  const float t = x * kExpL2E;
  float lo = __builtin_fmaf(x, kExpL2E, -t);
  lo = __builtin_fmaf(x, kExpL2ELo, lo);
  const float p = __builtin_amdgcn_exp2f(t);
  return __builtin_fmaf(p, lo * kExpLn2, p);
}

__device__ __forceinline__ f32x8 vexp(f32x8 x) {
  return map8(x, [](float v) { return exp1(v); });
}

// exp1 with the range handling hoisted out: when every lane's 8 arguments
// are in exp1_in_range's range the wave takes the straight-line path.
__device__ __forceinline__ f32x8 vexp_uniform(f32x8 x) {
  bool ok = true;
#pragma unroll
  for (int e = 0; e < 8; ++e) ok &= exp1_in_range(x[e]);
  if (!__all(ok)) return vexp(x);
  return map8(x, [](float v) { return exp1_fast(v); });
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

// The spec's further math functions (TTLH_OP_EXP2 ..), out of line: they are
// rare, and inlining their libm expansions would grow every every-op
// interpreter copy.
__device__ __attribute__((noinline)) f32x8 unary_ext(int op, f32x8 a, float p, float q) {
  f32x8 t;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = a[e];
    float r;
    switch (op) {
      case TTLH_OP_EXP2: r = exp2f(x); break;
      case TTLH_OP_EXPM1: r = expm1f(x); break;
      case TTLH_OP_LOG1P: r = log1pf(x); break;
      case TTLH_OP_SIN: r = sinf(x); break;
      case TTLH_OP_COS: r = cosf(x); break;
      case TTLH_OP_TAN: r = tanf(x); break;
      case TTLH_OP_ASIN: r = asinf(x); break;
      case TTLH_OP_ACOS: r = acosf(x); break;
      case TTLH_OP_ATAN: r = atanf(x); break;
      case TTLH_OP_ASINH: r = asinhf(x); break;
      case TTLH_OP_ACOSH: r = acoshf(x); break;
      case TTLH_OP_ATANH: r = atanhf(x); break;
      // x / 2 (1 + erf(x / sqrt 2)) = x / 2 erfc(-x / sqrt 2): no cancellation for x << 0
      case TTLH_OP_GELU: r = 0.5f * x * erfcf(-x * 0.70710678118654752f); break;
      case TTLH_OP_SILU: r = x / (1.0f + expf(-x)); break;
      case TTLH_OP_SOFTSIGN: r = x / (1.0f + fabsf(x)); break;
      case TTLH_OP_HARDSIGMOID: r = fminf(fmaxf(x + 3.0f, 0.0f), 6.0f) / 6.0f; break;
      case TTLH_OP_ELU: r = x > 0.0f ? x : p * expm1f(x); break;
      case TTLH_OP_CELU: r = fmaxf(x, 0.0f) + fminf(p * expm1f(x / p), 0.0f); break;
      case TTLH_OP_SELU: r = p * (fmaxf(x, 0.0f) + fminf(q * expm1f(x), 0.0f)); break;
      default: r = p * x > q ? x : log1pf(expf(p * x)) / p; break;  // TTLH_OP_SOFTPLUS
    }
    t[e] = x != x ? x : r;  // NaN in, NaN out (fmaxf / fminf would drop it)
  }
  return t;
}

// relu as torch computes it (clamp_min(x, 0): x unless x < 0), so -0 stays
// -0 and a NaN passes through; a maximum with 0 would turn -0 into +0.
__device__ __forceinline__ float relu1(float v) { return v < 0.0f ? 0.0f : v; }

template <bool FULL>
__device__ __forceinline__ f32x8 unary(int op, f32x8 a, float imm, float imm2 = 0.0f) {
  if constexpr (!FULL) {
    switch (op) {
      case TTLH_OP_EXP: return vexp(a);
      case TTLH_OP_NEG: return -a;
      case TTLH_OP_ABS: return map8(a, [](float v) { return fabsf(v); });
      case TTLH_OP_RELU: return map8(a, [](float v) { return relu1(v); });
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
    case TTLH_OP_RELU: return map8(a, [](float v) { return relu1(v); });
    case TTLH_OP_SIGMOID: return map8(a, [](float v) { return 1.0f / (1.0f + expf(-v)); });
    case TTLH_OP_RECIP: return 1.0f / a;
    case TTLH_OP_POWI: return map8(a, [imm](float v) { return powf(v, imm); });
    default: return unary_ext(op, a, imm, imm2);
  }
}

// The ops a kernel that keeps live accumulators across the program may run:
// those whose definitions above expand inline (the others call out-of-line
// library code, and the call would spill the accumulators).  Same
// expressions as binary<true> / unary<true>.
inline bool is_inline_op(int form, int op) {
  if (form == TTLH_FORM_UNARY)
    return op == TTLH_OP_EXP || op == TTLH_OP_NEG || op == TTLH_OP_ABS || op == TTLH_OP_RELU ||
           op == TTLH_OP_RECIP || op == TTLH_OP_SQRT || op == TTLH_OP_RSQRT;
  if (form >= TTLH_FORM_BIN)
    return op == TTLH_OP_ADD || op == TTLH_OP_SUB || op == TTLH_OP_MUL || op == TTLH_OP_DIV ||
           op == TTLH_OP_MAX || op == TTLH_OP_MIN;
  return true;
}
// one element of binary_inline / unary_inline, the op fixed at compile time
template <int OP>
__device__ __forceinline__ float binary1(float a, float b) {
  if constexpr (OP == TTLH_OP_ADD) return a + b;
  else if constexpr (OP == TTLH_OP_SUB) return a - b;
  else if constexpr (OP == TTLH_OP_MUL) return a * b;
  else if constexpr (OP == TTLH_OP_DIV) return a / b;
  else {  // TTLH_OP_MAX, TTLH_OP_MIN (NaN-propagating)
    const float m = OP == TTLH_OP_MAX ? fmaxf(a, b) : fminf(a, b);
    return (a != a || b != b) ? __builtin_nanf("") : m;
  }
}
template <int OP>
__device__ __forceinline__ float unary1(float v) {
  if constexpr (OP == TTLH_OP_EXP) return exp1(v);
  else if constexpr (OP == TTLH_OP_SQRT) return sqrtf(v);
  else if constexpr (OP == TTLH_OP_RSQRT) return 1.0f / sqrtf(v);
  else if constexpr (OP == TTLH_OP_ABS) return fabsf(v);
  else if constexpr (OP == TTLH_OP_NEG) return -v;
  else if constexpr (OP == TTLH_OP_RELU) return relu1(v);
  else return 1.0f / v;  // TTLH_OP_RECIP
}
template <int OP>
__device__ __forceinline__ f32x8 binary8(f32x8 a, f32x8 b) {
  f32x8 t;
#pragma unroll
  for (int e = 0; e < 8; ++e) t[e] = binary1<OP>(a[e], b[e]);
  return t;
}
template <int OP>
__device__ __forceinline__ f32x8 unary8(f32x8 a) {
  f32x8 t;
#pragma unroll
  for (int e = 0; e < 8; ++e) t[e] = unary1<OP>(a[e]);
  return t;
}
__device__ __forceinline__ f32x8 binary_inline(int op, f32x8 a, f32x8 b) {
  switch (op) {
    case TTLH_OP_ADD: return binary8<TTLH_OP_ADD>(a, b);
    case TTLH_OP_SUB: return binary8<TTLH_OP_SUB>(a, b);
    case TTLH_OP_MUL: return binary8<TTLH_OP_MUL>(a, b);
    case TTLH_OP_DIV: return binary8<TTLH_OP_DIV>(a, b);
    case TTLH_OP_MAX: return binary8<TTLH_OP_MAX>(a, b);
    default: return binary8<TTLH_OP_MIN>(a, b);
  }
}
__device__ __forceinline__ f32x8 unary_inline(int op, f32x8 a) {
  switch (op) {
    case TTLH_OP_EXP: return unary8<TTLH_OP_EXP>(a);
    case TTLH_OP_SQRT: return unary8<TTLH_OP_SQRT>(a);
    case TTLH_OP_RSQRT: return unary8<TTLH_OP_RSQRT>(a);
    case TTLH_OP_ABS: return unary8<TTLH_OP_ABS>(a);
    case TTLH_OP_NEG: return unary8<TTLH_OP_NEG>(a);
    case TTLH_OP_RELU: return unary8<TTLH_OP_RELU>(a);
    default: return unary8<TTLH_OP_RECIP>(a);
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
    case K_UNARY: acc = unary<FULL>(ins.op, acc, ins.imm, ins.imm2); break;
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


// The program for one chunk with one operand held in registers: the operand
// whose pointer is null takes the values `reg` (the fused GEMM epilogue's
// rounded product), every other one is loaded as by the interpreters above.
// Same op definitions and per-step rounding as run_step, for the ops
// is_inline_op accepts (host code refuses the others).
template <bool OFF32>
__device__ __forceinline__ f32x8 run_program_reg(const EltArgs& args, f32x8 reg, int64_t y,
                                                 int64_t x) {
  f32x8 acc = splat(0.0f), s0 = acc, s1 = acc;
  for (int k = 0; k < args.n_instr; ++k) {
    const Ins ins = args.prog[k];
    f32x8 v = acc;
    if (ins.src == SRC_OPERAND) {
      const EltOperand& op = args.ops[ins.arg];
      v = op.ptr == nullptr
              ? reg
              : to_f32<8, false>(op, load_raw<8, false>(op, operand_addr<OFF32>(op, y, x)));
    } else if (ins.src == SRC_IMM) {
      v = splat(ins.imm);
    } else if (ins.src == SRC_POP) {
      v = s0;
      s0 = s1;
    }
    switch (ins.kind) {
      case K_SET: acc = v; break;
      case K_PUSH:
        s1 = s0;
        s0 = acc;
        acc = v;
        break;
      case K_UNARY: acc = unary_inline(ins.op, acc); break;
      case K_BIN: acc = binary_inline(ins.op, acc, v); break;
      default: acc = binary_inline(ins.op, v, acc); break;  // K_BIN_REV
    }
    if (ins.rnd == TTLH_BF16) acc = round_bf16x8(acc);
  }
  return acc;
}

// As run_program_reg, with every operand of the chunk loaded beforehand:
// q[i] holds operand i's raw bits (consumption order, at most 4 operands),
// the operand whose pointer is null (the product) takes `reg`.
__device__ __forceinline__ f32x8 run_program_reg_pre(const EltArgs& args, f32x8 reg,
                                                     const Raw (&q)[4]) {
  f32x8 acc = splat(0.0f), s0 = acc, s1 = acc;
  for (int k = 0; k < args.n_instr; ++k) {
    const Ins ins = args.prog[k];
    f32x8 v = acc;
    if (ins.src == SRC_OPERAND) {
      const int i = ins.arg;
      if (args.ops[i].ptr == nullptr) {
        v = reg;
      } else {
        switch (i) {  // uniform: no dynamic register indexing
          case 0: v = to_f32<8, false>(args.ops[0], q[0]); break;
          case 1: v = to_f32<8, false>(args.ops[1], q[1]); break;
          case 2: v = to_f32<8, false>(args.ops[2], q[2]); break;
          default: v = to_f32<8, false>(args.ops[3], q[3]); break;
        }
      }
    } else if (ins.src == SRC_IMM) {
      v = splat(ins.imm);
    } else if (ins.src == SRC_POP) {
      v = s0;
      s0 = s1;
    }
    switch (ins.kind) {
      case K_SET: acc = v; break;
      case K_PUSH:
        s1 = s0;
        s0 = acc;
        acc = v;
        break;
      case K_UNARY: acc = unary_inline(ins.op, acc); break;
      case K_BIN: acc = binary_inline(ins.op, acc, v); break;
      default: acc = binary_inline(ins.op, v, acc); break;  // K_BIN_REV
    }
    if (ins.rnd == TTLH_BF16) acc = round_bf16x8(acc);
  }
  return acc;
}

// ---------------------------------------------------------------------------
// host side: program validation and decoding

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool is_binary(int op) { return op >= TTLH_OP_ADD && op <= TTLH_OP_MOD; }
bool is_unary(int op) { return op >= TTLH_OP_EXP && op <= TTLH_OP_SOFTPLUS; }
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
  const int64_t ymax = mask_max(o.row_mask, y0 + h - 1) + o.row_off;
  const int64_t xmax = mask_max(o.col_mask, x0 + w - 1) + o.col_off;
  return ymax * o.row_stride + xmax * o.col_stride;
}


// What decode_program learned about a program and its operands.
struct ProgInfo {
  int n_ops = 0;
  int max_depth = 0;
  bool all_bf16 = true;  // every operand is bf16
  bool full = false;     // some step uses an op outside the common set
  bool vec = true;       // every contiguous operand allows 16-byte chunks at x0
  bool off32 = true;     // every operand offset over the region fits 31 bits
};

// Validates the ABI program `prog` / operands `in` over the iteration region
// (y0, x0, h, w) and decodes it into a.prog / a.ops / a.n_instr / a.n_ops.
// `who` prefixes the error messages.
int decode_program(const char* who, const ttlh_instr* prog, const ttlh_operand* in, int n_instr,
                   int64_t y0, int64_t x0, int64_t h, int64_t w, EltArgs& a, ProgInfo& pi) {
  TTLH_REQUIRE(prog && in && n_instr > 0 && n_instr <= TTLH_MAX_INSTR, TTLH_EINVAL,
               "%s: program must have 1..%d steps (got %d)", who, TTLH_MAX_INSTR, n_instr);
  int depth = 0;  // values on the stack including acc
  pi.vec = (w % 8 == 0) && (x0 % 8 == 0);
  for (int k = 0; k < n_instr; ++k) {
    const ttlh_instr& p = prog[k];
    const int f = p.form;
    const bool uses_operand = f == TTLH_FORM_LOAD || f == TTLH_FORM_PUSH || f == TTLH_FORM_BIN ||
                              f == TTLH_FORM_BIN_REV;
    TTLH_REQUIRE(f >= TTLH_FORM_LOAD && f <= TTLH_FORM_BIN_POP, TTLH_EINVAL,
                 "%s: bad form %d at step %d", who, f, k);
    TTLH_REQUIRE(p.rnd == TTLH_BF16 || p.rnd == TTLH_F32, TTLH_EINVAL,
                 "%s: bad rounding mode at step %d", who, k);
    if (f == TTLH_FORM_UNARY)
      TTLH_REQUIRE(is_unary(p.op), TTLH_EINVAL, "%s: step %d needs a unary opcode", who, k);
    if (f >= TTLH_FORM_BIN)
      TTLH_REQUIRE(is_binary(p.op), TTLH_EINVAL, "%s: step %d needs a binary opcode", who, k);
    // stack discipline
    if (f == TTLH_FORM_LOAD || f == TTLH_FORM_CONST) {
      TTLH_REQUIRE(depth == 0, TTLH_EINVAL, "%s: LOAD/CONST at step %d on a live stack", who, k);
      depth = 1;
    } else if (f == TTLH_FORM_PUSH || f == TTLH_FORM_PUSH_CONST) {
      TTLH_REQUIRE(depth >= 1 && depth < TTLH_MAX_STACK, TTLH_EINVAL,
                   "%s: stack overflow at step %d", who, k);
      ++depth;
    } else if (f == TTLH_FORM_BIN_POP) {
      TTLH_REQUIRE(depth >= 2, TTLH_EINVAL, "%s: stack underflow at step %d", who, k);
      --depth;
    } else {
      TTLH_REQUIRE(depth >= 1, TTLH_EINVAL, "%s: step %d reads an empty stack", who, k);
    }
    pi.max_depth = depth > pi.max_depth ? depth : pi.max_depth;
    if ((f == TTLH_FORM_UNARY || f >= TTLH_FORM_BIN) && !is_common(p.op)) pi.full = true;
    Ins& q = a.prog[k];
    q.op = p.op;
    q.rnd = p.rnd;
    q.imm = p.imm;
    q.imm2 = p.imm2;
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
    q.arg = static_cast<uint8_t>(pi.n_ops);
    const ttlh_operand& o = in[k];
    TTLH_REQUIRE(o.ptr && (o.dtype == TTLH_BF16 || o.dtype == TTLH_F32), TTLH_EINVAL,
                 "%s: operand %d has a null pointer or bad dtype", who, k);
    TTLH_REQUIRE(valid_mask(o.row_mask), TTLH_EINVAL,
                 "%s: operand %d row_mask must be -1, 31, 0 or ~31", who, k);
    TTLH_REQUIRE(valid_mask(o.col_mask), TTLH_EINVAL,
                 "%s: operand %d col_mask must be -1, 31, 0 or ~31", who, k);
    TTLH_REQUIRE(o.row_stride >= 0 && o.col_stride >= 0, TTLH_EINVAL,
                 "%s: operand %d has a negative stride", who, k);
    EltOperand& e = a.ops[pi.n_ops++];
    e.ptr = o.ptr;
    e.rs = o.row_stride;
    e.cs = o.col_stride;
    e.rmask = o.row_mask;
    e.cmask = o.col_mask;
    e.roff = o.row_off;
    e.coff = o.col_off;
    e.dtype = o.dtype;
    pi.all_bf16 = pi.all_bf16 && o.dtype == TTLH_BF16;
    const int esz = o.dtype == TTLH_BF16 ? 2 : 4;
    // column masks 0 / ~31 give every 8-element chunk (8-aligned, inside one
    // tile) a single column: such operands are splatted like stride-0 ones
    const bool col_uniform = o.col_stride == 0 || o.col_mask == 0 || o.col_mask == ~int64_t(31);
    e.vec = !col_uniform && o.col_stride == 1 && aligned16(o.ptr) &&
            ((o.row_stride * esz) % 16 == 0) && ((o.col_off * esz) % 16 == 0) &&
            ((x0 * esz) % 16 == 0);
    // chunk-uniform operands keep the 8-wide path; others need alignment
    if (!col_uniform && !e.vec) pi.vec = false;
    const int64_t mo = max_offset(o, y0, x0, h, w);
    if (mo >= (int64_t(1) << 31) || o.row_off < 0 || o.col_off < 0) pi.off32 = false;
  }
  TTLH_REQUIRE(depth == 1, TTLH_EINVAL, "%s: program leaves %d values on the stack", who, depth);
  a.n_instr = n_instr;
  a.n_ops = pi.n_ops;
  a.y0 = y0;
  a.x0 = x0;
  return TTLH_OK;
}


}  // namespace
}  // namespace ttlh
