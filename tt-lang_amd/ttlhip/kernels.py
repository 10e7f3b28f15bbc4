"""Python wrappers of the libttlhip.so entry points (torch tensors in, launch out).

Each wrapper validates shapes on the host (so that every address a kernel
forms is inside its allocation), converts torch tensors to raw device
pointers and calls the C ABI on the current torch stream.  None of them
synchronises; callers that need reference (synchronous) semantics call
torch.cuda.synchronize() themselves.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import List, Optional, Sequence

import torch

from . import _lib as L
from .expr import StackProgram


@dataclass
class OperandMap:
    """How an eltwise operand is addressed from output element (y, x):
    iy = (y & row_mask) + row_off, ix = (x & col_mask) + col_off with masks
    -1 (identity), 31 (one tile re-used), ~31 (row / column 0 of every tile)
    or 0 (one fixed row / column); a size-1 tensor dimension is broadcast
    (stride 0)."""

    tensor: torch.Tensor
    row_mask: int = -1
    col_mask: int = -1
    row_off: int = 0
    col_off: int = 0


def _check_device(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{what} must be a device (HIP) tensor; there is no CPU path")
    if t.dim() != 2:
        raise ValueError(f"{what} must be 2-D, got shape {tuple(t.shape)}")


# Device workspaces (column and full reductions, weight dequantisation), one
# per (device, stream), grown to the largest size asked for and then kept.
# Taking a fresh one from torch's caching allocator on every call costs about
# 10 us of host time (4096^2 column sums: 35 -> 25 us of host enqueue per
# call, against 17 us of kernels).  Calls on one stream run in stream
# order, so they share that stream's buffer safely; calls on different
# streams get different buffers.  A HIP graph captured over such a call
# keeps the buffer's address: replaying it while eager calls run on the
# same buffer from another stream races, as with any shared buffer.
_WORKSPACES: dict = {}


def _workspace(device: torch.device, stream, nbytes: int) -> torch.Tensor:
    sp = L.stream_ptr(stream)
    key = (device.index, sp)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
        if stream is not None:
            # allocated on the current stream, used on `stream`: keep the
            # block from being handed out again before that stream's work
            # on it has finished once this buffer is replaced
            ws.record_stream(stream)
        _WORKSPACES[key] = ws
    return ws


def release_workspaces() -> None:
    """Drop the cached workspaces (their memory returns to torch's caching
    allocator once the work queued on them has finished)."""
    _WORKSPACES.clear()


def _axis_range(lo: int, n: int, mask: int, off: int):
    """[min, max] of (c & mask) + off for c in [lo, lo + n)."""
    if n <= 0:
        return None
    if mask == -1:
        return lo + off, lo + n - 1 + off
    if mask == 0:
        return off, off
    if mask == ~31:
        return (lo & ~31) + off, ((lo + n - 1) & ~31) + off
    if mask != 31:
        raise ValueError(f"operand mask must be -1, 31, 0 or ~31, got {mask}")
    vals_lo, vals_hi = 31, 0
    if n >= 32:
        vals_lo, vals_hi = 0, 31
    else:
        for c in range(lo, lo + n):
            vals_lo, vals_hi = min(vals_lo, c & 31), max(vals_hi, c & 31)
    return vals_lo + off, vals_hi + off


def _operand_struct(m: OperandMap, y0: int, x0: int, h: int, w: int) -> L.Operand:
    t = m.tensor
    _check_device(t, "eltwise operand")
    rows, cols = t.shape
    rs = t.stride(0) if rows > 1 else 0
    cs = t.stride(1) if cols > 1 else 0
    if rows > 1:
        r = _axis_range(y0, h, m.row_mask, m.row_off)
        if r and (r[0] < 0 or r[1] >= rows):
            raise ValueError(f"eltwise operand rows {r} out of range for shape {tuple(t.shape)}")
    if cols > 1:
        r = _axis_range(x0, w, m.col_mask, m.col_off)
        if r and (r[0] < 0 or r[1] >= cols):
            raise ValueError(f"eltwise operand cols {r} out of range for shape {tuple(t.shape)}")
    return L.Operand(t.data_ptr(), L.dtype_code(t.dtype), 0, rs, cs, m.row_mask, m.col_mask,
                     m.row_off, m.col_off)


def eltwise(prog: StackProgram, operands: Sequence[Optional[OperandMap]], out: torch.Tensor,
            region=None, stream=None) -> None:
    """Runs a compiled stack program over `region` = (y0, x0, h, w) of `out`.

    operands[k] is the operand of step k (None for steps without one).
    """
    _check_device(out, "eltwise output")
    if out.stride(1) != 1:
        raise ValueError("eltwise output must have unit column stride")
    n = len(prog.steps)
    if len(operands) != n:
        raise ValueError(f"{n} steps but {len(operands)} operand slots")
    y0, x0, h, w = region if region is not None else (0, 0, out.shape[0], out.shape[1])
    if y0 < 0 or x0 < 0 or y0 + h > out.shape[0] or x0 + w > out.shape[1]:
        raise ValueError(f"region {(y0, x0, h, w)} outside output {tuple(out.shape)}")
    instrs = (L.Instr * n)()
    ops = (L.Operand * n)()
    for k, (s, m) in enumerate(zip(prog.steps, operands)):
        instrs[k] = L.Instr(s.op, s.form, s.rnd, 0, s.imm, s.imm2)
        if s.form in (L.FORM_LOAD, L.FORM_PUSH, L.FORM_BIN, L.FORM_BIN_REV):
            if m is None:
                raise ValueError(f"step {k} needs an operand")
            ops[k] = _operand_struct(m, y0, x0, h, w)
    L.call("ttlh_eltwise", instrs, ops, n, out.data_ptr(), L.dtype_code(out.dtype),
           out.stride(0), y0, x0, h, w, L.stream_ptr(stream))


def reduce(prog: StackProgram, operands: Sequence[Optional[OperandMap]], kind: str,
           dims: Sequence[int], out: torch.Tensor, region, out_origin=(0, 0),
           out_pad: bool = False, scaler: Optional[torch.Tensor] = None, scale: float = 1.0,
           stream=None, noalloc: bool = False) -> None:
    """Scaled reduction (kind "sum" or "max") of a stack program over the
    iteration `region` = (y0, x0, h, w), operands addressed as in eltwise()
    from iteration element (y, x).  dims: the reduced axes (0: over rows, 1:
    over columns).  The results are written into `out` from `out_origin`
    (one per column, one per row, or one value; out_pad: whole zero-padded
    32-wide result tiles).  scaler: a device tensor whose first element
    multiplies every value (times `scale`).  noalloc: run through
    ttlh_reduce_noalloc (partial results in the library's fixed per-GPU
    scratch array, nothing allocated; calls overlapping on one GPU race)."""
    _check_device(out, "reduce output")
    if out.stride(1) != 1:
        raise ValueError("reduce output must have unit column stride")
    if kind not in ("sum", "max"):
        raise ValueError(f"reduce kind must be 'sum' or 'max', got {kind!r}")
    dset = set(int(d) for d in dims)
    if not dset or not dset <= {0, 1}:
        raise ValueError(f"reduce dims must be a non-empty subset of [0, 1], got {list(dims)}")
    dbits = (L.REDUCE_DIM0 if 0 in dset else 0) | (L.REDUCE_DIM1 if 1 in dset else 0)
    n = len(prog.steps)
    if len(operands) != n:
        raise ValueError(f"{n} steps but {len(operands)} operand slots")
    y0, x0, h, w = region
    if h <= 0 or w <= 0 or y0 < 0 or x0 < 0:
        raise ValueError(f"bad reduce region {tuple(region)}")
    oy, ox = out_origin
    # output extent: the result rows / columns (plus the tile padding)
    rows = (1 if 0 in dset else h) if not out_pad else (32 if 0 in dset else h)
    cols = (1 if 1 in dset else w) if not out_pad else (32 if 1 in dset else w)
    if oy < 0 or ox < 0 or oy + rows > out.shape[0] or ox + cols > out.shape[1]:
        raise ValueError(f"reduce result ({rows}x{cols} at {(oy, ox)}) outside output "
                         f"{tuple(out.shape)}")
    instrs = (L.Instr * n)()
    ops = (L.Operand * n)()
    for k, (s, m) in enumerate(zip(prog.steps, operands)):
        instrs[k] = L.Instr(s.op, s.form, s.rnd, 0, s.imm, s.imm2)
        if s.form in (L.FORM_LOAD, L.FORM_PUSH, L.FORM_BIN, L.FORM_BIN_REV):
            if m is None:
                raise ValueError(f"step {k} needs an operand")
            ops[k] = _operand_struct(m, y0, x0, h, w)
    sp, sdt = 0, 0
    if scaler is not None:
        if not scaler.is_cuda or scaler.numel() < 1:
            raise ValueError("reduce scaler must be a non-empty device tensor")
        sp, sdt = scaler.data_ptr(), L.dtype_code(scaler.dtype)
    optr = out.data_ptr() + (oy * out.stride(0) + ox) * out.element_size()
    kcode = L.REDUCE_SUM if kind == "sum" else L.REDUCE_MAX
    if noalloc:
        L.call("ttlh_reduce_noalloc", instrs, ops, n, kcode, dbits, sp, sdt, float(scale), optr,
               L.dtype_code(out.dtype), out.stride(0), int(bool(out_pad)), y0, x0, h, w,
               L.stream_ptr(stream))
        return
    ws_bytes = int(L.load().ttlh_reduce_workspace_bytes(dbits, h, w))
    ws = _workspace(out.device, stream, ws_bytes) if ws_bytes else None
    L.call("ttlh_reduce", instrs, ops, n, kcode,
           dbits, sp, sdt, float(scale), optr, L.dtype_code(out.dtype), out.stride(0),
           int(bool(out_pad)), y0, x0, h, w, ws.data_ptr() if ws is not None else 0, ws_bytes,
           L.stream_ptr(stream))


def _program_structs(prog: StackProgram, operands: Sequence[Optional[OperandMap]], region):
    y0, x0, h, w = region
    n = len(prog.steps)
    if len(operands) != n:
        raise ValueError(f"{n} steps but {len(operands)} operand slots")
    instrs = (L.Instr * n)()
    ops = (L.Operand * n)()
    for k, (s, m) in enumerate(zip(prog.steps, operands)):
        instrs[k] = L.Instr(s.op, s.form, s.rnd, 0, s.imm, s.imm2)
        if s.form in (L.FORM_LOAD, L.FORM_PUSH, L.FORM_BIN, L.FORM_BIN_REV):
            if m is None:
                raise ValueError(f"step {k} needs an operand")
            ops[k] = _operand_struct(m, y0, x0, h, w)
    return instrs, ops, n


@dataclass
class RowReduce:
    """One row reduction of reduce_rows_eltwise(): the arguments of a
    reduce(prog, operands, kind, [1], out, region, out_origin, out_pad,
    scaler, scale) call over the common region."""

    prog: StackProgram
    operands: Sequence[Optional[OperandMap]]
    kind: str
    out: torch.Tensor
    out_origin: tuple = (0, 0)
    out_pad: bool = False
    scaler: Optional[torch.Tensor] = None
    scale: float = 1.0


def reduce_rows_eltwise(reds: Sequence[RowReduce], prog: StackProgram,
                        operands: Sequence[Optional[OperandMap]], out: torch.Tensor, region,
                        stream=None) -> bool:
    """The row reductions `reds` (each a reduce(..., dims=[1]) over
    `region`), then eltwise(prog, operands, out, region), as one launch of
    ttlh_reduce_rows_eltwise: the same values in every output, each row's
    operands read once, a later program reading an earlier result for its
    own row from registers.  Returns False, having launched nothing, where
    the library refuses the combination (TTLH_EUNSUPPORTED); the caller then
    makes the separate calls."""
    y0, x0, h, w = region
    if h <= 0 or w <= 0 or y0 < 0 or x0 < 0:
        raise ValueError(f"bad region {tuple(region)}")
    _check_device(out, "eltwise output")
    if out.stride(1) != 1:
        raise ValueError("eltwise output must have unit column stride")
    if y0 + h > out.shape[0] or x0 + w > out.shape[1]:
        raise ValueError(f"region {tuple(region)} outside output {tuple(out.shape)}")
    keep = []  # ctypes arrays the structs point into, alive until the call returns
    rr = (L.RowReduce * len(reds))()
    for j, r in enumerate(reds):
        _check_device(r.out, "reduce output")
        if r.out.stride(1) != 1:
            raise ValueError("reduce output must have unit column stride")
        if r.kind not in ("sum", "max"):
            raise ValueError(f"reduce kind must be 'sum' or 'max', got {r.kind!r}")
        oy, ox = r.out_origin
        cols = 32 if r.out_pad else 1
        if oy < 0 or ox < 0 or oy + h > r.out.shape[0] or ox + cols > r.out.shape[1]:
            raise ValueError(f"reduce result ({h}x{cols} at {(oy, ox)}) outside output "
                             f"{tuple(r.out.shape)}")
        instrs, ops, n = _program_structs(r.prog, r.operands, region)
        keep += [instrs, ops]
        sp, sdt = 0, 0
        if r.scaler is not None:
            if not r.scaler.is_cuda or r.scaler.numel() < 1:
                raise ValueError("reduce scaler must be a non-empty device tensor")
            sp, sdt = r.scaler.data_ptr(), L.dtype_code(r.scaler.dtype)
        optr = r.out.data_ptr() + (oy * r.out.stride(0) + ox) * r.out.element_size()
        rr[j] = L.RowReduce(instrs, ops, n, L.REDUCE_SUM if r.kind == "sum" else L.REDUCE_MAX,
                            sp, sdt, float(r.scale), optr, L.dtype_code(r.out.dtype),
                            int(bool(r.out_pad)), r.out.stride(0))
    instrs, ops, n = _program_structs(prog, operands, region)
    st = L.load().ttlh_reduce_rows_eltwise(rr, len(reds), instrs, ops, n, out.data_ptr(),
                                           L.dtype_code(out.dtype), out.stride(0), y0, x0, h, w,
                                           L.stream_ptr(stream))
    if st == L.TTLH_EUNSUPPORTED:
        return False
    L.check("ttlh_reduce_rows_eltwise", st)
    return True


def matmul(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, accumulate: bool = False,
           stream=None) -> None:
    """c (=|+=) a @ b on the GPU, fp32 accumulation (bf16 or f32 MFMA)."""
    for t, nm in ((a, "A"), (b, "B"), (c, "C")):
        _check_device(t, f"matmul {nm}")
        if t.stride(1) != 1:
            raise ValueError(f"matmul {nm} must be row-major with unit column stride")
    M, K = a.shape
    K2, N = b.shape
    if K2 != K or tuple(c.shape) != (M, N):
        raise ValueError(f"matmul shapes {tuple(a.shape)} @ {tuple(b.shape)} -> {tuple(c.shape)}")
    L.call("ttlh_matmul", a.data_ptr(), L.dtype_code(a.dtype), a.stride(0), b.data_ptr(),
           L.dtype_code(b.dtype), b.stride(0), c.data_ptr(), L.dtype_code(c.dtype), c.stride(0),
           M, N, K, int(bool(accumulate)), L.stream_ptr(stream))


# Ops the fused GEMM epilogue (ttlh_matmul_eltwise) runs: + - * / max min
# and the unary exp sqrt rsqrt abs neg relu recip.
EPILOGUE_OPS = {1, 2, 3, 4, 5, 6, 16, 18, 19, 21, 22, 23, 25}


def matmul_eltwise_supported(M: int, N: int, K: int, prog: StackProgram) -> bool:
    """Whether ttlh_matmul_eltwise takes a problem of this shape and program:
    the large-problem GEMM (>= 192 output blocks of 256 x 256), a stack-free
    program of at most four operand reads (the product included) and the
    epilogue's op set (bf16 operands and output, and their alignment, are
    checked by the call)."""
    if M % 32 or N % 32 or K % 32 or ((M + 255) // 256) * ((N + 255) // 256) < 192:
        return False
    if any(s.form in (L.FORM_PUSH, L.FORM_PUSH_CONST, L.FORM_BIN_POP) for s in prog.steps):
        return False
    if sum(s.form in (L.FORM_LOAD, L.FORM_BIN, L.FORM_BIN_REV) for s in prog.steps) > 4:
        return False
    return all(s.op in EPILOGUE_OPS for s in prog.steps
               if s.form in (L.FORM_UNARY, L.FORM_BIN, L.FORM_BIN_REV, L.FORM_BIN_IMM,
                             L.FORM_BIN_IMM_REV))


def matmul_eltwise_preferred(prog: StackProgram) -> bool:
    """Whether the executor runs the fused epilogue rather than the GEMM +
    eltwise pair it replaces: programs of one op after the product load, and
    of two without exp whose only other operand is one tensor (the
    bias-and-activation form, at parity and one launch with the product's
    HBM round trip gone).

    The fused kernel runs its epilogue after the MFMA loop with one wave per
    SIMD and, at the sizes it takes, one output block per CU, so the whole
    chip runs the epilogue at once and nothing hides its VALU work or its
    operand reads; the pair pays the product's round trip through HBM
    (write + read, 4 bytes per element) instead.  Measured at 4096^3
    (fused / two launches; buffer sets rotated over 1.5 GB or not, the same
    ratios within 1%): one op after the load 0.99-1.11x faster (bias
    add 1.03, row / column broadcast 1.00 / 1.01, scale 1.03, relu 1.02,
    max 1.11, div 1.09, sqrt 1.08, rsqrt 1.06, recip 1.00, exp 0.99); two or
    more ops 0.92-0.99x (relu(x + c) 0.99, x + c + d 0.98, exp(x s) c 0.94,
    relu(x s + row) 0.93, three operands 0.92)."""
    steps = prog.steps
    if len(steps) <= 2:
        return True
    reads = sum(s.form in (L.FORM_LOAD, L.FORM_BIN, L.FORM_BIN_REV) for s in steps)
    return (len(steps) == 3 and reads <= 2
            and not any(s.form == L.FORM_UNARY and s.op == L.OP["exp"] for s in steps))


def matmul_eltwise(a: torch.Tensor, b: torch.Tensor, prog: StackProgram,
                   operands: Sequence[Optional[OperandMap]], prod_step: int, out: torch.Tensor,
                   region, stream=None) -> None:
    """out[region] = prog(round_bf16(a @ b), operands): step `prod_step`
    reads the product (its operands[] entry is ignored), the other steps'
    operands are addressed as in eltwise() from the output element.  region
    = (y0, x0, M, N) with (M, N) the product's shape."""
    for t, nm in ((a, "A"), (b, "B")):
        _check_device(t, f"matmul_eltwise {nm}")
        if t.dtype != torch.bfloat16 or t.stride(1) != 1:
            raise ValueError(f"matmul_eltwise {nm} must be row-major bf16")
    _check_device(out, "matmul_eltwise output")
    if out.stride(1) != 1:
        raise ValueError("matmul_eltwise output must have unit column stride")
    M, K = a.shape
    K2, N = b.shape
    y0, x0, h, w = region
    if K2 != K or (h, w) != (M, N) or y0 + h > out.shape[0] or x0 + w > out.shape[1]:
        raise ValueError(f"matmul_eltwise shapes {tuple(a.shape)} @ {tuple(b.shape)} -> region "
                         f"{tuple(region)} of {tuple(out.shape)}")
    n = len(prog.steps)
    instrs = (L.Instr * n)()
    ops = (L.Operand * n)()
    for k, (s, m) in enumerate(zip(prog.steps, operands)):
        instrs[k] = L.Instr(s.op, s.form, s.rnd, 0, s.imm, s.imm2)
        if k != prod_step and s.form in (L.FORM_LOAD, L.FORM_PUSH, L.FORM_BIN, L.FORM_BIN_REV):
            if m is None:
                raise ValueError(f"step {k} needs an operand")
            ops[k] = _operand_struct(m, y0, x0, h, w)
    L.call("ttlh_matmul_eltwise", a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), M, N, K,
           instrs, ops, n, prod_step, out.data_ptr(), L.dtype_code(out.dtype), out.stride(0),
           y0, x0, L.stream_ptr(stream))


def tilize(x: torch.Tensor, stream=None) -> torch.Tensor:
    """Row-major bf16 / f32 [rows, cols] (device) -> its tilized element order
    (tiles row-major over the tile grid, four 16x16 faces per tile), as a 1-D
    device tensor of rows * cols elements."""
    _check_device(x, "tilize input")
    if x.dtype not in (torch.bfloat16, torch.float32) or x.stride(1) != 1:
        raise ValueError("tilize takes a bf16 / f32 tensor with unit column stride")
    rows, cols = x.shape
    out = torch.empty(rows * cols, dtype=x.dtype, device=x.device)
    L.call("ttlh_tilize", x.data_ptr(), x.stride(0), out.data_ptr(), rows, cols,
           x.element_size(), L.stream_ptr(stream))
    return out


def untilize(data: torch.Tensor, rows: int, cols: int, out: Optional[torch.Tensor] = None,
             stream=None) -> torch.Tensor:
    """Tilized elements (device, rows * cols of them) -> row-major [rows, cols]
    (into `out` when given, which may have a row stride larger than cols)."""
    if not data.is_cuda:
        raise RuntimeError("untilize input must be a device (HIP) tensor; there is no CPU path")
    if data.dtype not in (torch.bfloat16, torch.float32) or data.numel() != rows * cols:
        raise ValueError(f"untilize needs {rows * cols} bf16 / f32 elements, got "
                         f"{data.numel()} {data.dtype}")
    if out is None:
        out = torch.empty(rows, cols, dtype=data.dtype, device=data.device)
    _check_device(out, "untilize output")
    if out.dtype != data.dtype or tuple(out.shape) != (rows, cols) or out.stride(1) != 1:
        raise ValueError("untilize output must match the data dtype and [rows, cols] shape")
    L.call("ttlh_untilize", data.contiguous().data_ptr(), out.data_ptr(), out.stride(0), rows,
           cols, data.element_size(), L.stream_ptr(stream))
    return out


def transpose(src: torch.Tensor, dst: torch.Tensor, stream=None) -> None:
    """dst = src^T for bf16 device matrices with unit column stride."""
    for t, nm in ((src, "source"), (dst, "destination")):
        _check_device(t, f"transpose {nm}")
        if t.dtype != torch.bfloat16 or t.dim() != 2 or t.stride(1) != 1:
            raise ValueError(f"transpose {nm} must be a bf16 matrix with unit column stride")
    rows, cols = src.shape
    if tuple(dst.shape) != (cols, rows):
        raise ValueError(f"transpose of {tuple(src.shape)} into {tuple(dst.shape)}")
    L.call("ttlh_transpose_bf16", src.data_ptr(), src.stride(0), dst.data_ptr(), dst.stride(0),
           rows, cols, L.stream_ptr(stream))


def bfp8_tiles_bytes(rows: int, cols: int) -> int:
    if rows % 32 or cols % 32:
        raise ValueError(f"bfloat8_b needs whole 32x32 tiles, got {rows}x{cols}")
    return (rows // 32) * (cols // 32) * L.TTLH_BFP8_TILE_BYTES


def bfp8_pack_host(x: torch.Tensor) -> torch.Tensor:
    """fp32 [rows, cols] (host) -> uint8 bfloat8_b tile bytes (host)."""
    x = x.detach().to("cpu", torch.float32).contiguous()
    rows, cols = x.shape
    out = torch.empty(bfp8_tiles_bytes(rows, cols), dtype=torch.uint8)
    L.call("ttlh_bfp8_pack_host", x.data_ptr(), out.data_ptr(), rows, cols)
    return out


def bfp8_unpack_host(q: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    q = q.detach().to("cpu", torch.uint8).contiguous()
    if q.numel() != bfp8_tiles_bytes(rows, cols):
        raise ValueError("bfloat8_b byte count does not match the shape")
    out = torch.empty((rows, cols), dtype=torch.bfloat16)
    L.call("ttlh_bfp8_unpack_host", q.data_ptr(), out.data_ptr(), rows, cols)
    return out


def bfp8_unpack(q: torch.Tensor, rows: int, cols: int, stream=None) -> torch.Tensor:
    if not q.is_cuda:
        raise RuntimeError("bfp8_unpack takes device tiles")
    if q.numel() != bfp8_tiles_bytes(rows, cols) or q.dtype != torch.uint8:
        raise ValueError("bfloat8_b byte count does not match the shape")
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=q.device)
    L.call("ttlh_bfp8_unpack", q.data_ptr(), out.data_ptr(), rows, cols, L.stream_ptr(stream))
    return out


# At and above this many rows of A the weight tiles are dequantised once into a
# bf16 workspace and multiplied by the bf16 GEMM (ttlh_matmul_bfp8w_ws); below
# it the fused kernel, which decodes each tile once per 256-row block of A, is
# used (ttlh_matmul_bfp8w).
BFP8_TWO_PASS_MIN_M = 512


def matmul_bfp8w(a: torch.Tensor, bq: torch.Tensor, c: torch.Tensor, stream=None,
                 two_pass: Optional[bool] = None) -> None:
    """c[M,N] = a[M,K] (bf16) @ dequant(bq)[K,N]; bf16 out.  `two_pass`
    forces the path (None: by M, see BFP8_TWO_PASS_MIN_M); the two-pass
    workspace is the cached one of c's device and the stream."""
    _check_device(a, "matmul_bfp8w A")
    _check_device(c, "matmul_bfp8w C")
    M, K = a.shape
    M2, N = c.shape
    if M2 != M or a.dtype != torch.bfloat16 or c.dtype != torch.bfloat16:
        raise ValueError("matmul_bfp8w takes bf16 A [M,K] and bf16 C [M,N]")
    if not bq.is_cuda or bq.dtype != torch.uint8 or bq.numel() != bfp8_tiles_bytes(K, N):
        raise ValueError("matmul_bfp8w: Bq must be device uint8 tiles of a K x N matrix")
    if a.stride(1) != 1 or c.stride(1) != 1:
        raise ValueError("matmul_bfp8w: A and C must be row-major")
    if two_pass is None:  # the two-pass decode reads Bq in 16-byte words
        two_pass = M >= BFP8_TWO_PASS_MIN_M and bq.data_ptr() % 16 == 0
    if not two_pass:
        L.call("ttlh_matmul_bfp8w", a.data_ptr(), a.stride(0), bq.data_ptr(), c.data_ptr(),
               c.stride(0), M, N, K, L.stream_ptr(stream))
        return
    nbytes = int(L.load().ttlh_matmul_bfp8w_workspace_bytes(M, N, K))
    ws = _workspace(c.device, stream, nbytes)
    L.call("ttlh_matmul_bfp8w_ws", a.data_ptr(), a.stride(0), bq.data_ptr(), c.data_ptr(),
           c.stride(0), M, N, K, ws.data_ptr(), nbytes, L.stream_ptr(stream))


def bfp4_tiles_bytes(rows: int, cols: int) -> int:
    if rows % 32 or cols % 32:
        raise ValueError(f"bfloat4_b needs whole 32x32 tiles, got {rows}x{cols}")
    return (rows // 32) * (cols // 32) * L.TTLH_BFP4_TILE_BYTES


def bfp4_pack_host(x: torch.Tensor) -> torch.Tensor:
    """fp32 [rows, cols] (host) -> uint8 bfloat4_b tile bytes (host)."""
    x = x.detach().to("cpu", torch.float32).contiguous()
    rows, cols = x.shape
    out = torch.empty(bfp4_tiles_bytes(rows, cols), dtype=torch.uint8)
    L.call("ttlh_bfp4_pack_host", x.data_ptr(), out.data_ptr(), rows, cols)
    return out


def bfp4_unpack_host(q: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    q = q.detach().to("cpu", torch.uint8).contiguous()
    if q.numel() != bfp4_tiles_bytes(rows, cols):
        raise ValueError("bfloat4_b byte count does not match the shape")
    out = torch.empty((rows, cols), dtype=torch.bfloat16)
    L.call("ttlh_bfp4_unpack_host", q.data_ptr(), out.data_ptr(), rows, cols)
    return out


def bfp4_unpack(q: torch.Tensor, rows: int, cols: int, stream=None) -> torch.Tensor:
    if not q.is_cuda:
        raise RuntimeError("bfp4_unpack takes device tiles")
    if q.numel() != bfp4_tiles_bytes(rows, cols) or q.dtype != torch.uint8:
        raise ValueError("bfloat4_b byte count does not match the shape")
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=q.device)
    L.call("ttlh_bfp4_unpack", q.data_ptr(), out.data_ptr(), rows, cols, L.stream_ptr(stream))
    return out


def matmul_bfp4w(a: torch.Tensor, bq: torch.Tensor, c: torch.Tensor, stream=None) -> None:
    """c[M,N] = a[M,K] (bf16) @ dequant(bq)[K,N] with bfloat4_b weights; the
    dequantised weights go through a bf16 workspace (the cached one of c's
    device and the stream)."""
    _check_device(a, "matmul_bfp4w A")
    _check_device(c, "matmul_bfp4w C")
    M, K = a.shape
    M2, N = c.shape
    if M2 != M or a.dtype != torch.bfloat16 or c.dtype != torch.bfloat16:
        raise ValueError("matmul_bfp4w takes bf16 A [M,K] and bf16 C [M,N]")
    if not bq.is_cuda or bq.dtype != torch.uint8 or bq.numel() != bfp4_tiles_bytes(K, N):
        raise ValueError("matmul_bfp4w: Bq must be device uint8 tiles of a K x N matrix")
    if a.stride(1) != 1 or c.stride(1) != 1:
        raise ValueError("matmul_bfp4w: A and C must be row-major")
    ws = _workspace(c.device, stream, K * N * 2)
    L.call("ttlh_matmul_bfp4w_ws", a.data_ptr(), a.stride(0), bq.data_ptr(), c.data_ptr(),
           c.stride(0), M, N, K, ws.data_ptr(), K * N * 2, L.stream_ptr(stream))


def sdpa_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor, scale: float,
             causal: bool = False, stream=None) -> None:
    for t, nm in ((q, "Q"), (k, "K"), (v, "V"), (o, "O")):
        if not t.is_cuda or t.dtype != torch.bfloat16 or t.dim() != 4 or not t.is_contiguous():
            raise ValueError(f"sdpa {nm} must be a contiguous bf16 device tensor [B,H,S,D]")
        if tuple(t.shape) != tuple(q.shape):
            raise ValueError("sdpa Q, K, V, O must share one shape")
    B, H, S, D = q.shape
    L.call("ttlh_sdpa_fwd", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, S, D,
           float(scale), int(bool(causal)), L.stream_ptr(stream))
