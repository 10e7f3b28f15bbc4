/*
 * ttlhip.h — C ABI of libttlhip.so, the MI355X (gfx950) execution library
 * behind the drop-in `ttl` / `ttnn` Python modules.
 *
 * The reference (tenstorrent/tt-lang) exposes no C ABI for its kernels: its
 * host->device boundary is the Python call
 *     ttnn.generic_op(tensors, ProgramDescriptor)
 * made by run_kernel_on_device() (python/ttl/kernel_runner.py:188-255), which
 * launches compiled reader / compute / writer threads on the Tensix grid.
 * Each entry point below replaces one *class* of such launch: the Python
 * tracer turns a @ttl.kernel's circular-buffer / copy / store program into one
 * or a few calls here.  Every reference anchor is cited on the declaration.
 *
 * Conventions
 *  - All tensor pointers are DEVICE pointers (HIP), row-major storage.
 *    bf16 is stored as uint16_t bit patterns.  Exceptions: the *_host codec
 *    helpers, which take host pointers.
 *  - `stream` is a hipStream_t passed as void* (NULL = default stream).
 *    Every launch is stream-ordered and asynchronous; nothing here
 *    synchronises, allocates caller-visible memory or frees caller memory.
 *  - Return value: TTLH_OK (0) on success, a positive TTLH_E* code otherwise;
 *    ttlh_last_error() then returns a thread-local message (the Python layer
 *    raises ValueError / RuntimeError with it, mirroring the reference's
 *    error convention, python/ttl/ttl_api.py:733-737).
 */
#ifndef TTLHIP_H
#define TTLHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TTLH_ABI_VERSION 2

/* status codes */
#define TTLH_OK 0
#define TTLH_EINVAL 1       /* bad argument (shape, dtype, null pointer)  */
#define TTLH_EUNSUPPORTED 2 /* valid request this build does not handle  */
#define TTLH_EHIP 3         /* HIP runtime error                         */

/* element types (the reference's ttnn.bfloat16 / ttnn.float32,
 * python/ttl/dtype_utils.py:151-181) */
#define TTLH_BF16 0
#define TTLH_F32 1

/* Tile geometry (python/sim/constants.py:42-44: TILE_SHAPE = (32, 32)). */
#define TTLH_TILE 32

/* ------------------------------------------------------------------------
 * Fused elementwise / broadcast tile program
 *
 * Replaces the compute thread's DST-register tile ops
 * (include/ttlang/Dialect/TTL/TTLElementwiseOps.def:61-82; simulator:
 * Block._binary_op python/sim/block.py:870-1010 and broadcast_tensors
 * python/sim/ttnnsim.py:67-109) together with the reader / writer threads'
 * tile DMA (noc_async_read_tile / noc_async_write_tile, lowered in
 * lib/Dialect/TTL/Transforms/ConvertTTLToTTKernel.cpp:563-751).
 *
 * A program is a straight-line list of at most TTLH_MAX_INSTR steps of a
 * small stack machine evaluated per output element in fp32.  The value on
 * top of the stack is `acc`; at most two more values sit below it.  Step k
 * owns operand slot k (in[k]); steps that read no operand leave in[k].ptr
 * NULL.  After each step `acc` is rounded to `rnd` (TTLH_BF16 =
 * round-to-nearest-even to bfloat16, matching the simulator, which
 * materialises every intermediate tile in its torch dtype; TTLH_F32 = keep
 * fp32).  The result is `acc` after the last step.
 * ---------------------------------------------------------------------- */
enum ttlh_opcode {
  TTLH_OP_NONE = 0,
  TTLH_OP_ADD = 1,      /* binary: x + y                                   */
  TTLH_OP_SUB = 2,
  TTLH_OP_MUL = 3,
  TTLH_OP_DIV = 4,
  TTLH_OP_MAX = 5,      /* NaN-propagating (torch.maximum)                 */
  TTLH_OP_MIN = 6,
  TTLH_OP_POW = 7,      /* x ** y                                          */
  TTLH_OP_FLOORDIV = 8, /* floor(x / y)  (torch.floor_divide)              */
  TTLH_OP_MOD = 9,      /* x - floor(x / y) * y  (torch.remainder)         */
  TTLH_OP_EXP = 16,     /* unary: f(acc)                                   */
  TTLH_OP_LOG = 17,
  TTLH_OP_SQRT = 18,
  TTLH_OP_RSQRT = 19,
  TTLH_OP_TANH = 20,
  TTLH_OP_ABS = 21,
  TTLH_OP_NEG = 22,
  TTLH_OP_RELU = 23,
  TTLH_OP_SIGMOID = 24,
  TTLH_OP_RECIP = 25,
  TTLH_OP_POWI = 26,    /* acc ** imm (integer exponent, Block.__pow__)    */
  /* the spec's further math functions (docs/sphinx/specs/
   * TTLangSpecification.md:700-750; neither the reference compiler's op
   * table nor its simulator implements them): computed in fp32 and rounded
   * once, as the torch functions the spec links do on bfloat16 tensors */
  TTLH_OP_EXP2 = 27,
  TTLH_OP_EXPM1 = 28,
  TTLH_OP_LOG1P = 29,   /* ttl.math.logp1                                  */
  TTLH_OP_SIN = 30,
  TTLH_OP_COS = 31,
  TTLH_OP_TAN = 32,
  TTLH_OP_ASIN = 33,
  TTLH_OP_ACOS = 34,
  TTLH_OP_ATAN = 35,
  TTLH_OP_ASINH = 36,
  TTLH_OP_ACOSH = 37,
  TTLH_OP_ATANH = 38,
  TTLH_OP_GELU = 39,    /* x / 2 (1 + erf(x / sqrt 2)) (torch's exact GELU) */
  TTLH_OP_SILU = 40,    /* x / (1 + exp(-x))                               */
  TTLH_OP_SOFTSIGN = 41,/* x / (1 + |x|), rounded once (the drop-in's
                           ttl.math.softsign composes abs, add, div
                           instead, rounding per op like torch's)        */
  TTLH_OP_HARDSIGMOID = 42, /* min(max(x + 3, 0), 6) / 6                   */
  TTLH_OP_ELU = 43,     /* x > 0 ? x : imm (exp(x) - 1)                    */
  TTLH_OP_CELU = 44,    /* max(x, 0) + min(imm (exp(x / imm) - 1), 0)      */
  TTLH_OP_SELU = 45,    /* imm (max(x, 0) + min(imm2 (exp(x) - 1), 0))     */
  TTLH_OP_SOFTPLUS = 46 /* imm x > imm2 ? x : log(1 + exp(imm x)) / imm    */
};

enum ttlh_form {
  TTLH_FORM_LOAD = 0,        /* acc = in[k]            (stack was empty)   */
  TTLH_FORM_PUSH = 1,        /* push acc; acc = in[k]                      */
  TTLH_FORM_CONST = 2,       /* acc = imm              (stack was empty)   */
  TTLH_FORM_PUSH_CONST = 3,  /* push acc; acc = imm                        */
  TTLH_FORM_UNARY = 4,       /* acc = op(acc)                              */
  TTLH_FORM_BIN = 5,         /* acc = op(acc, in[k])                       */
  TTLH_FORM_BIN_REV = 6,     /* acc = op(in[k], acc)                       */
  TTLH_FORM_BIN_IMM = 7,     /* acc = op(acc, imm)                         */
  TTLH_FORM_BIN_IMM_REV = 8, /* acc = op(imm, acc)                         */
  TTLH_FORM_BIN_POP = 9      /* acc = op(pop(), acc)                       */
};

typedef struct ttlh_instr {
  uint8_t op;   /* ttlh_opcode (ignored by LOAD/PUSH/CONST forms) */
  uint8_t form; /* ttlh_form                                      */
  uint8_t rnd;  /* TTLH_BF16 or TTLH_F32                          */
  uint8_t pad;
  float imm;    /* CONST value / immediate operand / POWI exponent /
                   first parameter of ELU, CELU, SELU, SOFTPLUS   */
  float imm2;   /* second parameter of SELU (alpha), SOFTPLUS
                   (threshold); 0 otherwise                       */
} ttlh_instr;

#define TTLH_MAX_INSTR 12
#define TTLH_MAX_STACK 3

/* An input operand, addressed from the output element (y, x):
 *   iy = (y & row_mask) + row_off ;  ix = (x & col_mask) + col_off
 *   element = ptr[iy * row_stride + ix * col_stride]
 * row_mask/col_mask = -1 (identity), 31 (a fixed tile re-used across the
 * tile grid, simulator block broadcasting, python/sim/block.py:886-920),
 * ~31 (row / column 0 of every tile: the compiler's in-tile broadcast
 * tile_bcast Row / Col / Scalar, TTLElementwiseOps.def:82,
 * python/ttl/operators.py:333-360) or 0 (one fixed row / column: both at
 * once); a stride of 0 broadcasts a degenerate (size-1) tensor dimension
 * across the tile (python/sim/copyhandlers.py:103-131).  Offsets are
 * multiples of 32 for the masks other than -1.  The caller guarantees every
 * addressed element lies inside the allocation.                          */
typedef struct ttlh_operand {
  const void* ptr;
  int32_t dtype;      /* TTLH_BF16 / TTLH_F32 */
  int32_t pad;
  int64_t row_stride; /* elements */
  int64_t col_stride; /* elements: 1 (contiguous) or 0 (broadcast) */
  int64_t row_mask, col_mask;
  int64_t row_off, col_off;
} ttlh_operand;

/* Evaluate `prog` for every element of the out region
 * [y0, y0+h) x [x0, x0+w) of `out` (row stride out_ld elements) and store
 * the final `acc` (rounded RNE to out_dtype).  `in` has n_instr entries.
 * Replaces: the generated reader/compute/writer thread triple of a fused
 * elementwise kernel launched through ttnn.generic_op
 * (python/ttl/kernel_runner.py:188-255); simulator call stack
 * python/sim/program.py:363-647 -> block.py:805-1010. */
int ttlh_eltwise(const ttlh_instr* prog, const ttlh_operand* in, int n_instr,
                 void* out, int out_dtype, int64_t out_ld, int64_t y0,
                 int64_t x0, int64_t h, int64_t w, void* stream);

/* ------------------------------------------------------------------------
 * Scaled reductions of a tile program
 *
 * The spec's ttl.math.reduce_sum / reduce_max (docs/sphinx/specs/
 * TTLangSpecification.md:754-755: "scaled sum / maximum reduction over the
 * specified dimensions"); the reference has no implementation (neither the
 * compiler's op table nor the simulator), so the semantics are fixed here:
 *   v(y, x) = the value `prog` computes for iteration element (y, x) of the
 *             region [y0, y0+h) x [x0, x0+w), operands addressed exactly as
 *             in ttlh_eltwise (per-step rounding included);
 *   s       = scale_imm * (*scaler) (scaler NULL: s = scale_imm);
 *   result  = sum or NaN-propagating max of v * s over the reduced
 *             dimension(s), products and accumulation in fp32, rounded once
 *             (RNE) to out_dtype.
 * dims: TTLH_REDUCE_DIM0 reduces over rows (one value per column, written
 * at out[x - x0]), TTLH_REDUCE_DIM1 over columns (one value per row, at
 * out[(y - y0) * out_ld]), both bits: one value at out[0].  out_pad = 1
 * writes whole 32-wide result tiles instead, the reduced position(s) of
 * every tile being 0 (column reduce: rows 1..31 under each value zeroed;
 * row reduce: columns 1..31 after each value; both: the 32x32 tile).
 * Summation order is fixed by the launch shape, so results repeat exactly
 * for equal arguments.  Row reductions need no workspace; the others take
 * ttlh_reduce_workspace_bytes(dims, h, w) bytes of caller-owned device
 * memory (fp32 partial results).                                          */
#define TTLH_REDUCE_SUM 0
#define TTLH_REDUCE_MAX 1
#define TTLH_REDUCE_DIM0 1
#define TTLH_REDUCE_DIM1 2

int64_t ttlh_reduce_workspace_bytes(int dims, int64_t h, int64_t w);

int ttlh_reduce(const ttlh_instr* prog, const ttlh_operand* in, int n_instr,
                int kind, int dims, const void* scaler, int scaler_dtype,
                float scale_imm, void* out, int out_dtype, int64_t out_ld,
                int out_pad, int64_t y0, int64_t x0, int64_t h, int64_t w,
                void* workspace, int64_t workspace_bytes, void* stream);

/* ttlh_reduce without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference (its
 * kernels allocate nothing a caller sees).  The fp32 partial results live in
 * a fixed array of TTLH_REDUCE_SCRATCH_BYTES per GPU inside the library
 * (held until the process ends); reductions whose
 * ttlh_reduce_workspace_bytes() exceeds it are refused with TTLH_EUNSUPPORTED.
 * Nothing is allocated or freed.  Every call on one GPU shares that array:
 * calls that overlap on one GPU (different streams, or host threads racing
 * on one) race on it; calls ordered on one stream are safe.  The stream must
 * belong to the current device.  Results are identical to ttlh_reduce's. */
#define TTLH_REDUCE_SCRATCH_BYTES (4 << 20)

int ttlh_reduce_noalloc(const ttlh_instr* prog, const ttlh_operand* in,
                        int n_instr, int kind, int dims, const void* scaler,
                        int scaler_dtype, float scale_imm, void* out,
                        int out_dtype, int64_t out_ld, int out_pad, int64_t y0,
                        int64_t x0, int64_t h, int64_t w, void* stream);

/* ------------------------------------------------------------------------
 * Row reductions and the elementwise program that reads them, one launch
 *
 * One row reduction (the arguments of a ttlh_reduce call with dims =
 * TTLH_REDUCE_DIM1 and the region of ttlh_reduce_rows_eltwise).            */
typedef struct ttlh_row_reduce {
  const ttlh_instr* prog;
  const ttlh_operand* in;
  int32_t n_instr;
  int32_t kind;         /* TTLH_REDUCE_SUM / TTLH_REDUCE_MAX */
  const void* scaler;   /* NULL: scale_imm alone              */
  int32_t scaler_dtype;
  float scale_imm;
  void* out;            /* result of region row r at out[r * out_ld] */
  int32_t out_dtype;
  int32_t out_pad;
  int64_t out_ld;
} ttlh_row_reduce;

/* The same as ttlh_reduce(red[0]), ..., ttlh_reduce(red[n_red - 1]) (each a
 * row reduction over the region) followed by ttlh_eltwise(prog, in, n_instr,
 * out, ...) over that region, in one launch and with the same results in
 * every output, bit for bit: a row's operands are read from memory once and
 * a later program's operand that reads an earlier reduction's result for the
 * same row (its column 0) takes the value in registers.  For a store whose
 * expression reduces rows and then uses the results on the same rows, e.g.
 * softmax: exp(x - broadcast(reduce_max(x))) * broadcast(recip(reduce_sum(
 * exp(x - broadcast(reduce_max(x)))))) (spec ops reduce_max / reduce_sum /
 * broadcast, docs/sphinx/specs/TTLangSpecification.md:693-761; the
 * simulator materialises every intermediate block, python/sim/
 * block.py:870-920).  Returns TTLH_EUNSUPPORTED before launching, and the
 * caller makes the separate calls, unless: 1 <= n_red <= 3; every program
 * uses only + - * / max min exp sqrt rsqrt abs neg relu recip and is a chain
 * over the row (every binary op has at most one operand computed from the
 * row's elements; the other is an operand, an immediate, or computed from
 * earlier results and immediates alone, at most 8 such values per stage);
 * w <= 8192 and every operand admits 16-byte chunks (w, x0, offsets
 * 8-aligned), as does the output; at most three distinct identity-mapped
 * bf16 operands and four other operands; no output overlaps another output,
 * an operand or a scaler, except an elementwise output that is an operand
 * read element for element in place, and a later read of a reduction's
 * result maps every element of a row to that row's result.  ttlh_reduce
 * runs its row reductions of a program (anything but a single LOAD) on this
 * launch's kernel whenever it takes them, so a row reduction has the same
 * summation order alone and fused.                                         */
int ttlh_reduce_rows_eltwise(const ttlh_row_reduce* red, int n_red,
                             const ttlh_instr* prog, const ttlh_operand* in,
                             int n_instr, void* out, int out_dtype,
                             int64_t out_ld, int64_t y0, int64_t x0,
                             int64_t h, int64_t w, void* stream);

/* ------------------------------------------------------------------------
 * Tilized element order (the TILE_LAYOUT storage of ttnn tensors, which the
 * reference's compiled path requires: python/ttl/ttl_api.py:489-506; the
 * tilize itself lives in un-vendored tt-metal).  Tiles of 32x32 row-major
 * over the tile grid; a tile is four 16x16 faces (f0 rows 0-15 / cols 0-15,
 * f1 rows 0-15 / cols 16-31, f2 rows 16-31 / cols 0-15, f3 rows 16-31 /
 * cols 16-31), each face row-major: element (i, j) of a tensor with C
 * columns sits at tile (i / 32) * (C / 32) + j / 32, offset
 * 256 * (2 * ((i % 32) / 16) + (j % 32) / 16) + 16 * (i % 16) + j % 16.
 * rows, cols: multiples of 32; elem_bytes 2 (bf16) or 4 (f32); the
 * row-major side has row stride `ld` elements; device pointers, 16-byte
 * aligned.  Used to exchange tensors with tilized ttnn buffers.          */
int ttlh_tilize(const void* src, int64_t src_ld, void* dst, int64_t rows,
                int64_t cols, int elem_bytes, void* stream);
int ttlh_untilize(const void* src, void* dst, int64_t dst_ld, int64_t rows,
                  int64_t cols, int elem_bytes, void* stream);

/* dst[c, r] = src[r, c] for a bf16 [rows, cols] matrix (row strides in
 * elements).  No counterpart in the reference: it stages the K^T operand
 * [D, B*H*S] of an attention tile program (matmul of Q by K^T) as the K
 * [B*H*S, D] rows ttlh_sdpa_fwd reads, when K^T is not already the
 * transposed view of such rows.  rows, cols, strides: multiples of 8;
 * buffers 16-byte aligned and disjoint.                                  */
int ttlh_transpose_bf16(const void* src, int64_t src_ld, void* dst,
                        int64_t dst_ld, int64_t rows, int64_t cols,
                        void* stream);

/* ------------------------------------------------------------------------
 * Tile matmul:  C[M,N] (=|+=) A[M,K] . B[K,N]
 *
 * Replaces Block.__matmul__ + store(acc=True) over the K tiles
 * (python/sim/block.py:805-868,1012-1013; ttnnsim.py:454-459) and the
 * Tensix matmul_tiles loop (examples/metal_examples/singlecore_matmul/
 * metal/kernels/mm_compute.cpp:28-68).  bf16 inputs run on gfx950 bf16
 * MFMA, f32 inputs on f32 MFMA; accumulation is fp32 over the full K, the
 * result is rounded once to c_dtype.  accumulate = 1 adds into C.
 * M, N, K must be multiples of 32 (whole tiles); strides in elements.   */
int ttlh_matmul(const void* A, int a_dtype, int64_t lda, const void* B,
                int b_dtype, int64_t ldb, void* C, int c_dtype, int64_t ldc,
                int64_t M, int64_t N, int64_t K, int accumulate, void* stream);

/* ------------------------------------------------------------------------
 * Tile matmul with its store's elementwise program fused:
 *   out[y0 + i, x0 + j] = prog(round_bf16((A . B)[i, j]), operands...)
 * for the M x N product of bf16 A [M,K] and B [K,N] (fp32 accumulation).
 *
 * Replaces a store whose expression holds a tile / block matmul below its
 * root, e.g. store(relu(a @ b + c)) (spec TTLangSpecification.md:693-761):
 * the simulator materialises the product block in its dtype before the
 * other ops read it (python/sim/block.py:870-920, 1012-1013), so the product
 * is rounded to bf16, then the program runs with ttlh_eltwise's semantics
 * (same ops, per-step rounding) without the product passing through HBM.
 * `prog` / `in` / n_instr are ttlh_eltwise's, over the output region
 * (y0, x0, M, N); step `prod_step` reads the product: its in[] entry must
 * have a NULL pointer (the rest of that entry is ignored).  The program must
 * be stack-free (no PUSH / BIN_POP forms), may use + - * / max min exp sqrt
 * rsqrt abs neg relu recip and read at most 4 bf16 operands (the product
 * included); every operand must allow 8-wide chunks (16-byte aligned, unit
 * column stride or broadcast); the output is bf16.  Runs on the
 * large-problem GEMM only: >= 192 output blocks of 256 x 256.  Otherwise
 * returns TTLH_EUNSUPPORTED before launching, and the caller runs
 * ttlh_matmul into a buffer, then ttlh_eltwise.
 * M, N, K multiples of 32; A, B rows 16-byte aligned; out 16-byte aligned
 * with out_ld a multiple of 8; out must not overlap A, B or an operand.  */
int ttlh_matmul_eltwise(const void* A, int64_t lda, const void* B, int64_t ldb,
                        int64_t M, int64_t N, int64_t K, const ttlh_instr* prog,
                        const ttlh_operand* in, int n_instr, int prod_step,
                        void* out, int out_dtype, int64_t out_ld, int64_t y0,
                        int64_t x0, void* stream);

/* ------------------------------------------------------------------------
 * bfloat8_b weight tiles.  The reference only fixes the tile size
 * (32*32 + 64 = 1088 bytes, python/ttl/dtype_utils.py:174-175); the codec
 * lives in un-vendored tt-metal.  Format implemented here (byte layout of
 * one 32x32 tile; tiles stored row-major over the tile grid):
 *   bytes [0, 64):     shared exponents, face-major (faces f0 = rows 0-15 /
 *                      cols 0-15, f1 = rows 0-15 / cols 16-31, f2 = rows
 *                      16-31 / cols 0-15, f3 = rows 16-31 / cols 16-31),
 *                      byte 16*f + r for face row r;
 *   bytes [64, 1088):  one byte per element, byte 64 + 256*f + 16*r + c:
 *                      bit 7 = sign, bits 6..0 = magnitude m.
 *   value = (-1)^s * m * 2^(e - 133), exactly (m has at most 7 significant
 *   bits, so every value is a bfloat16, normal or subnormal; only e = 255,
 *   which packing finite data never produces, can overflow to +-inf).
 * Pack: e = largest biased fp32 exponent of the 16 values of a face row (0
 * when all are zero / subnormal), m = round-half-even(|x| * 2^(133 - e))
 * saturated to 127.  Inputs must be finite.  */
#define TTLH_BFP8_TILE_BYTES 1088

/* host codec (host pointers) */
int ttlh_bfp8_pack_host(const float* src, void* dst, int64_t rows,
                        int64_t cols);
int ttlh_bfp8_unpack_host(const void* src, uint16_t* dst_bf16, int64_t rows,
                          int64_t cols);
/* device dequant: tiles -> row-major bf16 (device pointers, both 16-byte
 * aligned; a tile's start is a multiple of 1088 = 68 x 16 bytes into the
 * tile array, so any tile-aligned view of an aligned array qualifies) */
int ttlh_bfp8_unpack(const void* src, void* dst_bf16, int64_t rows,
                     int64_t cols, void* stream);

/* C[M,N] = A[M,K] (bf16, row-major, lda) . dequant(Bq)[K,N], with Bq the
 * bfloat8_b tile array of a K x N matrix; dequantisation to bf16 happens in
 * LDS ahead of the bf16 MFMA; fp32 accumulate; bf16 out.                */
int ttlh_matmul_bfp8w(const void* A, int64_t lda, const void* Bq, void* C,
                      int64_t ldc, int64_t M, int64_t N, int64_t K,
                      void* stream);

/* The same product in two passes, for large M: Bq is dequantised once into
 * `workspace` (row-major bf16 [K, N], at least ttlh_matmul_bfp8w_workspace_bytes
 * bytes, 16-byte aligned, caller-owned) by ttlh_bfp8_unpack (so Bq must be
 * 16-byte aligned too), then multiplied by the bf16 GEMM of ttlh_matmul.
 * The fused entry point above decodes each
 * weight tile once per 256-row block of A, so it is the better choice when M
 * is small (one or two blocks); this one decodes each tile once.  Results are
 * identical to the fused path's within fp32 summation order.  Reference
 * counterpart: as ttlh_matmul_bfp8w (tile size dtype_utils.py:174-175).   */
int64_t ttlh_matmul_bfp8w_workspace_bytes(int64_t M, int64_t N, int64_t K);
int ttlh_matmul_bfp8w_ws(const void* A, int64_t lda, const void* Bq, void* C,
                         int64_t ldc, int64_t M, int64_t N, int64_t K,
                         void* workspace, int64_t workspace_bytes,
                         void* stream);

/* ------------------------------------------------------------------------
 * bfloat4_b tiles.  The reference fixes only the tile size, 64 + 512 = 576
 * bytes (python/ttl/dtype_utils.py:176-177); this build's format:
 *   bytes [0, 64):    exponent byte 16*f + r shared by face f, row r (faces
 *                     as for bfloat8_b);
 *   bytes [64, 576):  one nibble per element, byte 64 + 128*f + 8*r + c/2
 *                     (low nibble: even c, high nibble: odd c), bit 3 = sign,
 *                     bits 2..0 = magnitude m.
 *   value = (-1)^s * m * 2^(e - 129), exactly (at most 3 significant bits,
 *   always a bfloat16).
 * Pack: e = largest biased fp32 exponent of the face row's 16 values (0 when
 * all are zero / subnormal), m = round-half-even(|x| * 2^(129 - e)) capped at
 * 7.  Inputs must be finite.                                               */
#define TTLH_BFP4_TILE_BYTES 576

int ttlh_bfp4_pack_host(const float* src, void* dst, int64_t rows,
                        int64_t cols);
int ttlh_bfp4_unpack_host(const void* src, uint16_t* dst_bf16, int64_t rows,
                          int64_t cols);
/* device dequant: tiles -> row-major bf16 (device pointers, both 16-byte
 * aligned; a tile's start is a multiple of 1088 = 68 x 16 bytes into the
 * tile array, so any tile-aligned view of an aligned array qualifies) */
int ttlh_bfp4_unpack(const void* src, void* dst_bf16, int64_t rows,
                     int64_t cols, void* stream);
/* C[M,N] = A[M,K] (bf16, row-major) . dequant(Bq4)[K,N] in two passes: the
 * bfloat4_b weights are dequantised into `workspace` (row-major bf16 [K, N],
 * K*N*2 bytes, 16-byte aligned) and multiplied by the bf16 GEMM; bf16 out.
 * Reference counterpart: the bfloat4_b dtype (tile size as above).        */
int ttlh_matmul_bfp4w_ws(const void* A, int64_t lda, const void* Bq4, void* C,
                         int64_t ldc, int64_t M, int64_t N, int64_t K,
                         void* workspace, int64_t workspace_bytes,
                         void* stream);

/* ------------------------------------------------------------------------
 * Fused scaled-dot-product attention forward (no counterpart in the
 * reference: composed from spec ops @, exp, recip, reduce_max, reduce_sum,
 * broadcast, docs/sphinx/specs/TTLangSpecification.md:693-761).
 * Q, K, V, O: bf16 [B, H, S, D] contiguous; O = softmax(Q K^T * scale) V
 * with fp32 online softmax; D = 128 (or 64); S a multiple of 32 (whole
 * 32-row tiles; S not a multiple of 128 takes a masked tail). causal = 1
 * masks j > i.                                                            */
int ttlh_sdpa_fwd(const void* Q, const void* K, const void* V, void* O,
                  int64_t B, int64_t H, int64_t S, int64_t D, float scale,
                  int causal, void* stream);

/* ------------------------------------------------------------------------ */
const char* ttlh_last_error(void);
int ttlh_version(void);

#ifdef __cplusplus
}
#endif
#endif /* TTLHIP_H */
