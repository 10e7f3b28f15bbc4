"""Per-store-site profile of a kernel call, the MI355X counterpart of the
reference's auto-profiler (TTLANG_AUTO_PROFILE=1, python/ttl/_src/
auto_profile.py:52-54): there every source line of every Tensix thread gets
device cycles; here the threads are traced away and each store() site of the
kernel becomes one grid-wide launch, so the report gives, per store line,
the launch it became, its time (HIP events on the launch stream) and the
achieved rate against that launch's roofline (HBM bytes for elementwise
launches, MFMA flops for tile matmuls).
"""

from __future__ import annotations

import linecache
import os
from typing import Any, Dict, List, Sequence, Tuple

from . import plan as P

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0    # dense bf16 MFMA
F32_PEAK_TFLOPS = 157.3      # dense fp32 MFMA


def enabled() -> bool:
    return os.environ.get("TTLANG_AUTO_PROFILE", "0") == "1"


def _elem_size(dtype) -> int:
    return getattr(dtype, "itemsize", 2)


def launch_work(l, args: Dict[Any, Any]) -> Tuple[float, str, float]:
    """(algorithmic work, unit, peak) of one launch: bytes read + written for
    an elementwise launch (an operand counted over the rows / columns it
    actually spans), 2 M N K flops for a tile matmul, 4 S^2 D per head for
    fused attention; a matmul with its store's program fused counts as the
    matmul (MFMA-bound)."""
    if isinstance(l, P.FusedMatmulLaunch):
        return launch_work(l.mm, args)
    if isinstance(l, P.ReduceEltwiseLaunch):  # each operand once, every output
        total, seen = 0.0, set()
        for x in l.reds + [l.ew]:
            _, _, h, w = x.region
            out = x.out.resolve(args)
            total += (h if isinstance(x, P.ReduceLaunch) else h * w) * _elem_size(out.dtype)
            for spec in x.operands:
                if spec is None:
                    continue
                t = spec.ref.resolve(args)
                key = (t.data_ptr(), spec.row_mask, spec.col_mask, spec.row_off, spec.col_off)
                if key in seen or any(t.data_ptr() == r.out.resolve(args).data_ptr()
                                      for r in l.reds):
                    continue  # a reduction's result is read from registers
                seen.add(key)
                rows = 1 if t.shape[0] == 1 else (32 if spec.row_mask == 31 else h)
                cols = 1 if t.shape[1] == 1 else (32 if spec.col_mask == 31 else w)
                total += rows * cols * _elem_size(t.dtype)
        return float(total), "GB/s", HBM_PEAK_GBS
    if isinstance(l, (P.EltwiseLaunch, P.ReduceLaunch)):
        _, _, h, w = l.region
        out = l.out.resolve(args)
        if isinstance(l, P.ReduceLaunch):  # one result per kept row / column
            nres = (1 if 0 in l.dims else h) * (1 if 1 in l.dims else w)
            total = nres * _elem_size(out.dtype)
        else:
            total = h * w * _elem_size(out.dtype)
        seen = set()
        for spec in l.operands:
            if spec is None or id(spec.ref) in seen:
                continue
            seen.add(id(spec.ref))
            t = spec.ref.resolve(args)
            rows = 1 if t.shape[0] == 1 else (32 if spec.row_mask == 31 else h)
            cols = 1 if t.shape[1] == 1 else (32 if spec.col_mask == 31 else w)
            total += rows * cols * _elem_size(t.dtype)
        return float(total), "GB/s", HBM_PEAK_GBS
    if isinstance(l, P.SdpaLaunch):  # Q K^T and P V: 4 S^2 D flops per head
        d = l.q.resolve(args).shape[1]
        return 4.0 * l.heads * l.seq * l.seq * d, "TFLOP/s", BF16_PEAK_TFLOPS
    m = l.rows[1] - l.rows[0]
    n = l.cols[1] - l.cols[0]
    a = l.a.resolve(args)
    peak = F32_PEAK_TFLOPS if getattr(a, "dtype", None) is not None and str(a.dtype) == "torch.float32" \
        else BF16_PEAK_TFLOPS
    return 2.0 * m * n * l.k, "TFLOP/s", peak


def _launch_name(l, args) -> str:
    if isinstance(l, P.FusedMatmulLaunch):
        return (f"ttlh_matmul_eltwise {_launch_name(l.mm, args)[len('ttlh_matmul '):]} + "
                f"{len(l.ew.prog.steps)}-step epilogue")
    if isinstance(l, P.ReduceEltwiseLaunch):
        _, _, h, w = l.ew.region
        kinds = "+".join(r.kind for r in l.reds)
        return (f"ttlh_reduce_rows_eltwise {h}x{w}: row {kinds}, then "
                f"{len(l.ew.prog.steps)} steps")
    if isinstance(l, P.ReduceLaunch):
        _, _, h, w = l.region
        return f"ttlh_reduce {l.kind} dims {list(l.dims)} over {h}x{w}, {len(l.prog.steps)} steps"
    if isinstance(l, P.EltwiseLaunch):
        _, _, h, w = l.region
        nops = len({id(s.ref) for s in l.operands if s is not None})
        return f"ttlh_eltwise {h}x{w}, {len(l.prog.steps)} steps, {nops} operands"
    if isinstance(l, P.SdpaLaunch):
        return f"ttlh_sdpa_fwd {l.heads} heads x {l.seq} rows, D {l.q.resolve(args).shape[1]}"
    m = l.rows[1] - l.rows[0]
    n = l.cols[1] - l.cols[0]
    fmt = f" x {l.b.resolve_obj(args).dtype.name}" if l.b_block else ""
    return f"ttlh_matmul{fmt} {m}x{n}x{l.k}"


def report(kernel_name: str, grid: Sequence[int], plan: P.Plan, args: Dict[Any, Any],
           times_us: List[float]) -> str:
    width = 100
    lines = ["=" * width, "TTLANG AUTO-PROFILE REPORT (MI355X, HIP event time per launch)", "=" * width,
             f"kernel {kernel_name}  grid {tuple(grid)}  {len(plan.launches)} launch(es)  "
             f"total {sum(times_us):.2f} us", "",
             f"{'LINE':>6}  {'TIME':>10}  {'RATE':>22}  LAUNCH / SOURCE", "-" * width]
    for l, us in zip(plan.launches, times_us):
        work, unit, peak = launch_work(l, args)
        rate = work / (us * 1e-6) / (1e9 if unit == "GB/s" else 1e12) if us > 0 else 0.0
        frac = 100.0 * rate / peak if peak else 0.0
        fname, lineno = l.loc if l.loc else ("?", 0)
        src = linecache.getline(fname, lineno).strip() if lineno else ""
        lines.append(f"{lineno:>6}  {us:>7.2f} us  {rate:>9.1f} {unit:<7} ({frac:3.0f}%)  "
                     f"{_launch_name(l, args)}")
        lines.append(f"{'':>6}  {'':>10}  {'':>22}  {src}   [{os.path.basename(fname)}]")
    lines.append("(device time per launch; the first call of a kernel in a process also loads "
                 "its code object)")
    lines.append("=" * width)
    return "\n".join(lines)
