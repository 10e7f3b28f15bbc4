#!/usr/bin/env python3
"""Benchmark of the TTL tile-op hot path on one MI355X.

`python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAMES]` prints ONE
JSON line.  The headline workload is BASELINE.json configs[1], the fused
elementwise + broadcast pipe Y = exp(A + b_row) * C on bf16 4096x4096 tiles,
written as a tt-lang kernel (tests/kernel_lib.py: make_exp_row_pipe) and run
through the drop-in `ttl`; `value` is its HBM throughput in GB/s.  The other
configs are measured in the same run and listed under "workloads" with their
own roofline figures:
  C1 eltwise add 2048^2       tt-lang kernel (eltwise_add style)   HBM GB/s
  C3 bf16 matmul 4096^3       tt-lang kernel (multicore style)     TFLOP/s
  C4 bf16 x bfp8 4096x4096x11008   tt-lang kernel (multicore style, ttnn.bfloat8_b B)
                              -> ttlh_matmul_bfp8w_ws (two-pass)   TFLOP/s
  C4, weights dequantised in LDS   ttlh_matmul_bfp8w (mm_dq_kernel)  TFLOP/s
  C5 SDPA [4,32,4096,128]     tt-lang attention program -> ttlh_sdpa_fwd   TFLOP/s
  row sums 4096^2 (spec reduce_sum)  tt-lang kernel (reduce_rows)  HBM GB/s
  row softmax 4096^2 in one store   tt-lang kernel -> ttlh_reduce_rows_eltwise  HBM GB/s
                              (and the same plan as three launches, for comparison)
  tilize 4096^2 bf16 (TILE_LAYOUT)   ttlh_tilize                  HBM GB/s

A "step" is one pass of the hot path over one batch of synthetic input: one
execution of the kernel's launch plan over one resident buffer set.  Inputs
are in HBM before the timed region; every workload rotates buffer sets
spanning > 1.2 GB (ROTATE_BYTES) so the 256 MB Infinity Cache cannot serve them.
Every workload times exactly K steps, at steady state: a HIP graph of the K
steps is first replayed back to back, without a host synchronisation, over at
least PREROLL_MS (MFMA workloads MFMA_PREROLL_MS) and PREROLL_MIN_STEPS
steps; behind that queued work the K launches of each of SAMPLES samples are
enqueued between their own HIP events, so the engine clock has ramped and no
idle gap, host delay or graph start-up lies inside a timed sample.  The
median per-step time is reported.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "tests"), os.path.join(ROOT, "tt-lang_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
PREROLL_MS = 10.0              # steady work queued ahead of the timed steps (ms), at least
PREROLL_MIN_STEPS = 50         # ... and at least this many steps
MFMA_PREROLL_MS = 30.0         # MFMA workloads: the clock settles at the power cap
SAMPLES = 5                    # timed samples of K steps each (median reported)
ROTATE_BYTES = 1.2e9           # the buffer sets a workload cycles through span at least this
                               # (> 4 x the 256 MB Infinity Cache: every step's data comes from
                               # HBM; with ~300 MB of sets the cache served part of it, C2 ran
                               # 15.7 against 18.2 us)
COPY_BYTES = 8192 * 16384 * 2  # bytes the copy-ceiling kernel reads (and writes) per launch
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _timed(fn, threads=None):
    """(seconds, result) of fn() on the host, with torch limited to `threads`."""
    nthr = torch.get_num_threads()
    if threads is not None:
        torch.set_num_threads(threads)
    try:
        t0 = time.perf_counter()
        r = fn()
        return time.perf_counter() - t0, r
    finally:
        torch.set_num_threads(nthr)


CPU_SAMPLE_S = 10.0  # host seconds each CPU baseline aims for (repeated samples)


def _repeat(fn, threads=None, min_s: float = CPU_SAMPLE_S, max_reps: int = 64):
    """(seconds per repetition, repetitions) of fn() repeated on the host until
    min_s seconds have passed (at least once, at most max_reps times)."""
    total, reps = 0.0, 0
    while reps < max_reps and (reps == 0 or total < min_s):
        dt, _ = _timed(fn, threads)
        total += dt
        reps += 1
    return total / reps, reps


def _eager(make, tensors):
    """The oracle's eager executor (simulator execution model: threads
    blocking on circular-buffer rings, one torch op per 32x32 tile) running a
    tt-lang kernel over CPU tensors on 1 thread, repeated to about
    CPU_SAMPLE_S seconds; returns (seconds per run, runs)."""
    from oracle import sim_exec
    k = make(sim_exec.make_ttl())
    args = [sim_exec.OracleTensor(t) for t in tensors]
    return _repeat(lambda: k(*args), threads=1)


# --------------------------------------------------------------------------
# workloads


class Workload:
    name = ""
    bound = "hbm"
    unit = "GB/s"
    config = ""

    def setup(self):
        raise NotImplementedError

    def launch(self, i: int):
        raise NotImplementedError

    def work_per_step(self) -> float:
        raise NotImplementedError

    def kernel_name(self) -> str:
        raise NotImplementedError

    def check(self) -> dict:
        raise NotImplementedError

    def cpu_baseline(self):
        """The reference's CPU path for this workload (the oracle's
        restatement of the simulator), timed on a bounded sample."""
        return None

    def traffic_kernels(self):
        """(kernel-name substring, workgroup count or None) of every kernel a
        step launches, for the HBM byte counters."""
        return [(self.kernel_name(), None)]

    def algorithmic_bytes(self) -> float:
        """Bytes a step must move at least: every operand read once, every
        result written once."""
        return self.work_per_step()


def n_sets(bytes_per_set: float) -> int:
    """Buffer sets to cycle through: at least 3, spanning ROTATE_BYTES."""
    return max(3, math.ceil(ROTATE_BYTES / bytes_per_set))


def _clone(t):
    """Another device copy of a ttnn tensor with the same layout (strides of
    a transposed view, packed block-float tiles)."""
    import ttnn
    x = t._tensor.clone(memory_format=torch.preserve_format)
    return ttnn.Tensor(x, block=t._block, logical_shape=t._logical_shape, layout=t._layout)


class PlanWorkload(Workload):
    """A tt-lang kernel traced once by the drop-in `ttl`; each step executes
    its launch plan on one of the resident buffer sets."""

    def make_sets(self):  # -> list of arg lists (ttnn tensors)
        raise NotImplementedError

    def setup(self):
        from ttlhip import plan as P

        self.sets = self.make_sets()
        self.plan = self.kernel.trace(*self.sets[0])
        assert len(self.plan.launches) == 1, self.plan.describe()
        while len(self.sets) < n_sets(self.algorithmic_bytes()):
            self.sets.append([_clone(t) for t in self.sets[0]])
        self.amaps = [dict(enumerate(s)) for s in self.sets]
        self._execute = P.execute

    def launch(self, i):
        self._execute(self.plan, self.amaps[i % len(self.amaps)])


class EltwiseWorkload(PlanWorkload):
    """C1 / C2 through the drop-in.  `cols` (default n) other than a power of
    two times 8 makes C2's row vector fall outside the flat kernel's 1-D
    indexing (a row vector is read through a mask of its chunk count), so
    the launch is the general 2-D `stream_kernel` (any region, masks and
    offsets)."""

    def __init__(self, name, n, kind, seed=1234, cols=None):
        self.name, self.n, self.kind, self.seed = name, n, kind, seed
        self.cols = n if cols is None else cols
        shape = "%dx%d" % (n, self.cols)
        self.config = ("eltwise add C = A + B, bf16 %s, U[-1,1] (BASELINE configs[0])" % shape
                       if kind == "add" else
                       "fused eltwise pipe + broadcast Y = exp(A + b_row) * C, bf16 %s, "
                       "b_row 1x%d, U[-2,2]%s" % (
                           shape, self.cols, " (BASELINE configs[1])" if cols is None else
                           " (C2's program at a row length that is not a power of two)"))

    def flat(self):
        cpr = self.cols // 8
        return self.kind == "add" or (cpr & (cpr - 1)) == 0

    def kernel_name(self):
        return "flat_kernel" if self.flat() else "stream_kernel"

    def traffic_kernels(self):  # the kernel's instantiation for this program
        if self.kind == "add":
            return [("flat_kernel<2, 3u, true>", None)]
        return [("flat_kernel<4, 11u, true>" if self.flat() else "stream_kernel<4, 11u>", None)]

    def work_per_step(self):
        e = self.n * self.cols * 2
        return 3 * e if self.kind == "add" else 3 * e + self.cols * 2

    def expr(self):
        if self.kind == "add":
            return ("add", ("leaf", "a"), ("leaf", "b"))
        return ("mul", ("exp", ("add", ("leaf", "a"), ("leaf", "b"))), ("leaf", "c"))

    def cpu_inputs(self):
        from oracle.tile_ops import seeded
        n, m, s = self.n, self.cols, self.seed
        if self.kind == "add":
            return [seeded((n, m), "uniform", s, lo=-1, hi=1),
                    seeded((n, m), "uniform", s + 1, lo=-1, hi=1)]
        return [seeded((n, m), "uniform", s, lo=-2, hi=2),
                seeded((1, m), "uniform", s + 1, lo=-2, hi=2),
                seeded((n, m), "uniform", s + 2, lo=-2, hi=2)]

    def make_kernel(self, ttl_ns):
        import kernel_lib as KL
        return KL.make_eltwise_add(ttl_ns) if self.kind == "add" else KL.make_exp_row_pipe(ttl_ns)

    def make_sets(self):
        import ttl
        import ttnn

        self.kernel = self.make_kernel(ttl)
        base = [ttnn.from_torch(t) for t in self.cpu_inputs()]
        nsets = n_sets(self.work_per_step())
        sets = []
        for i in range(nsets):
            ins = base if i == 0 else [ttnn.Tensor(t._tensor.clone()) for t in base]
            sets.append(ins + [ttnn.empty((self.n, self.cols), dtype=torch.bfloat16)])
        return sets

    def check(self):
        from oracle import tile_ops as O
        self.launch(0)
        torch.cuda.synchronize()
        ref = O.eval_expr(self.expr(), dict(zip("abc", self.cpu_inputs())))
        ulp = O.bf16_ulp_diff(self.sets[0][-1].to_torch(), ref)
        return {"max_ulp": int(ulp.max()), "mismatch_frac": float((ulp > 0).float().mean()),
                "oracle": "vectorised simulator semantics (per-op bf16 rounding)"}

    def cpu_baseline(self):
        """The oracle's eager executor (one torch op per 32x32 tile, CB ring
        bookkeeping, three threads per core under the GIL: the simulator's
        execution model) on the same tt-lang kernel and the full-size input."""
        from oracle import tile_ops as O
        ins = self.cpu_inputs()
        out = torch.zeros(self.n, self.cols, dtype=torch.bfloat16)
        dt, reps = _eager(self.make_kernel, ins + [out])
        env = dict(zip("abc", ins))
        dtv, _ = _repeat(lambda: O.eval_expr(self.expr(), env), min_s=1.0)
        return {"value": round(self.work_per_step() / dt / 1e9, 4), "unit": "GB/s", "cores": 1,
                "kind": "port",
                "sample": f"the full {self.n}x{self.cols} workload through the eager tile-by-tile "
                          f"oracle executor (simulator execution model, 1 thread), {reps} runs "
                          f"of {dt:.2f} s",
                "host_cpu_count": os.cpu_count(),
                "vectorised_torch_cpu": {"value": round(self.work_per_step() / dtv / 1e9, 3),
                                         "unit": "GB/s", "cores": torch.get_num_threads()}}


class ReduceWorkload(PlanWorkload):
    """Row sums of a bf16 matrix through a tt-lang kernel
    (ttl.math.reduce_sum(x, s, dims=[1]) over (2, 16)-tile blocks accumulated
    with store(acc=True), 8x8 grid) -> one ttlh_reduce launch; HBM-bound."""

    def __init__(self, name, n, seed=4321):
        self.name, self.n, self.seed = name, n, seed
        self.config = (f"row sums out[r] = sum_c x[r, c] * s, x bf16 {n}x{n} U[-2,2], s = 1, "
                       f"bf16 out {n}x1 (spec reduce_sum, dims=[1])")

    def kernel_name(self):
        return "reduce_rows_bf16_kernel"

    def traffic_kernels(self):  # the plain variant (the product one serves row_dot)
        return [("reduce_rows_bf16_kernel<0, false, true, false>", self.n)]

    def work_per_step(self):
        return self.n * self.n * 2 + self.n * 2

    def make_sets(self):
        import kernel_lib as KL
        import ttl
        import ttnn
        from oracle.tile_ops import seeded
        self.kernel = KL.make_reduce_rows(ttl, kind="sum", gr=2, gc=16, grid=(8, 8))
        self.x = seeded((self.n, self.n), "uniform", self.seed, lo=-2, hi=2)
        x = ttnn.from_torch(self.x)
        sc = ttnn.from_torch(torch.ones(32, 32, dtype=torch.bfloat16))
        nsets = n_sets(self.work_per_step())
        sets = []
        for i in range(nsets):
            xi = x if i == 0 else ttnn.Tensor(x._tensor.clone())
            sets.append([xi, sc, ttnn.empty((self.n, 1), dtype=torch.bfloat16)])
        return sets

    def check(self):
        from oracle import tile_ops as O
        self.launch(0)
        torch.cuda.synchronize()
        exact = self.x.double().sum(1, keepdim=True).float().bfloat16()
        ulp = O.bf16_ulp_diff(self.sets[0][-1].to_torch(), exact)
        return {"max_ulp": int(ulp.max()), "mismatch_frac": float((ulp > 0).float().mean()),
                "oracle": "float64 row sums rounded once to bf16"}

    def cpu_baseline(self):
        import kernel_lib as KL
        from oracle.tile_ops import seeded
        x = seeded((self.n, self.n), "uniform", self.seed, lo=-2, hi=2)
        t = [x, torch.ones(32, 32, dtype=torch.bfloat16),
             torch.zeros(self.n, 1, dtype=torch.bfloat16)]
        dt, reps = _eager(lambda ns: KL.make_reduce_rows(ns, kind="sum", gr=2, gc=16,
                                                         grid=(8, 8)), t)
        return {"value": round(self.work_per_step() / dt / 1e9, 4), "unit": "GB/s", "cores": 1,
                "kind": "port",
                "sample": f"the full {self.n}x{self.n} workload through the eager tile-by-tile "
                          f"oracle executor (1 thread), {reps} runs of {dt:.2f} s"}


class RowDotWorkload(PlanWorkload):
    """Row dot products out[r] = sum_c a[r, c] * b[r, c] through a tt-lang
    kernel (tests/kernel_lib.py make_row_dot: ttl.math.reduce_sum(a * b, 1,
    dims=[1]) over whole rows, 8x8 grid): the reduction fused with the
    elementwise stage that produces its operand, one launch (the bf16 row
    kernel's product variant) reading both operands once; HBM-bound."""

    def __init__(self, name, n, seed=4322):
        self.name, self.n, self.seed = name, n, seed
        self.config = (f"row dot products out[r] = sum_c a[r, c] * b[r, c], a, b bf16 {n}x{n} "
                       f"U[-2,2], bf16 out {n}x32 (spec reduce_sum of a product, dims=[1])")

    def kernel_name(self):
        return "reduce_rows_bf16_kernel"

    def traffic_kernels(self):
        return [("reduce_rows_bf16_kernel<0, false, true, true>", self.n)]

    def work_per_step(self):
        return 2 * self.n * self.n * 2 + self.n * 32 * 2

    def _make(self, ns, grid=(8, 8)):
        import kernel_lib as KL
        return KL.make_row_dot(ns, gr=2, gc=self.n // 32, grid=grid)

    def _inputs(self):
        from oracle.tile_ops import seeded
        return (seeded((self.n, self.n), "uniform", self.seed, lo=-2, hi=2),
                seeded((self.n, self.n), "uniform", self.seed + 1, lo=-2, hi=2))

    def make_sets(self):
        import ttl
        import ttnn
        self.kernel = self._make(ttl)
        self.a, self.b = self._inputs()
        a, b = ttnn.from_torch(self.a), ttnn.from_torch(self.b)
        nsets = n_sets(self.work_per_step())
        sets = []
        for i in range(nsets):
            ai = a if i == 0 else ttnn.Tensor(a._tensor.clone())
            bi = b if i == 0 else ttnn.Tensor(b._tensor.clone())
            sets.append([ai, bi, ttnn.empty((self.n, 32), dtype=torch.bfloat16)])
        return sets

    def check(self):
        from oracle import tile_ops as O
        self.launch(0)
        torch.cuda.synchronize()
        got = self.sets[0][-1].to_torch()
        # the simulator rounds the product to bf16 before the sum
        prod = (self.a.float() * self.b.float()).bfloat16().double()
        exact = prod.sum(1).float().bfloat16()
        ulp = O.bf16_ulp_diff(got[:, 0], exact)
        return {"max_ulp": int(ulp.max()), "mismatch_frac": float((ulp > 0).float().mean()),
                "padding_zero": bool((got[:, 1:] == 0).all()),
                "oracle": "float64 row sums of the bf16-rounded products, rounded once to bf16"}

    def cpu_baseline(self):
        a, b = self._inputs()
        t = [a, b, torch.zeros(self.n, 32, dtype=torch.bfloat16)]
        dt, reps = _eager(lambda ns: self._make(ns, grid=(1, 1)), t)
        return {"value": round(self.work_per_step() / dt / 1e9, 4), "unit": "GB/s", "cores": 1,
                "kind": "port",
                "sample": f"the full {self.n}x{self.n} workload through the eager tile-by-tile "
                          f"oracle executor running the same kernel (1 thread), {reps} runs of "
                          f"{dt:.2f} s"}


class SoftmaxWorkload(PlanWorkload):
    """Row softmax of a bf16 matrix written as one tt-lang store whose
    expression holds the spec's reduce_max and reduce_sum
    (tests/kernel_lib.py make_softmax_one_store: y = e * broadcast(recip(
    reduce_sum(e))), e = exp(x - broadcast(reduce_max(x))), one block per
    row band of 128 tiles, 8x8 grid).  Planned as two row reductions and the
    elementwise program: one ttlh_reduce_rows_eltwise launch reading x once,
    which runs the row softmax on its dedicated kernel
    (`separate`: the same plan run as its three launches, x read three
    times, for comparison).  HBM-bound; algorithmic bytes = x read once, y
    written once, the two reduction result tiles written once."""

    form = "softmax"

    def __init__(self, name, n, separate=False, seed=2468):
        self.name, self.n, self.separate, self.seed = name, n, separate, seed
        how = ("the plan's three launches (ttlh_reduce x2, ttlh_eltwise)" if separate else
               "one ttlh_reduce_rows_eltwise launch")
        self.config = (f"row softmax y = exp(x - max_r) / sum_r exp(x - max_r) in one store "
                       f"(spec reduce_max / reduce_sum / broadcast), x bf16 {n}x{n} U[-4,4], "
                       f"per-op bf16 rounding; {how}")

    def kernel_name(self):
        return "reduce_rows_bf16_kernel" if self.separate else "softmax_rows_kernel"

    def traffic_kernels(self):
        # separate: the row sum and the final program both run as
        # reduce_rows_eltwise_kernel<256, 1, 2, false> over 4096 workgroups,
        # which the per-kernel counter medians cannot tell apart: not listed
        if self.separate:
            return []
        return [("softmax_rows_kernel<256, 2>", None)]

    def work_per_step(self):
        return 2 * self.n * self.n * 2 + 2 * self.n * 32 * 2

    def make_sets(self):
        import kernel_lib as KL
        import ttl
        import ttnn
        from oracle.tile_ops import seeded
        self.kernel = KL.make_softmax_one_store(ttl, gc=self.n // 32, grid=(8, 8), form=self.form)
        self.x = seeded((self.n, self.n), "uniform", self.seed, lo=-4, hi=4)
        x = ttnn.from_torch(self.x)
        sc = ttnn.from_torch(torch.ones(32, 32, dtype=torch.bfloat16))
        sets = []
        for i in range(n_sets(self.work_per_step())):
            xi = x if i == 0 else ttnn.Tensor(x._tensor.clone())
            sets.append([xi, sc, ttnn.empty((self.n, self.n), dtype=torch.bfloat16)])
        return sets

    def setup(self):
        from ttlhip import plan as P
        super().setup()
        (l,) = self.plan.launches
        assert isinstance(l, P.ReduceEltwiseLaunch), self.plan.describe()
        if self.separate:
            self.plan = P.Plan(launches=list(l.reds) + [l.ew], created=self.plan.created,
                               uses_created=self.plan.uses_created)

    def check(self):
        from oracle import tile_ops as O
        from ttlhip import plan as P
        self.launch(0)
        torch.cuda.synchronize()
        got = self.sets[0][-1].to_torch()
        # the other execution of the same plan, bit for bit
        other = P.Plan(launches=list(self.plan.launches[0].reds) + [self.plan.launches[0].ew]) \
            if not self.separate else P.Plan(launches=[P.ReduceEltwiseLaunch(
                self.plan.launches[:-1], self.plan.launches[-1])])
        P.execute(other, self.amaps[0])
        torch.cuda.synchronize()
        again = self.sets[0][-1].to_torch()
        ex = self.exact()
        return {"bit_equal_fused_and_separate": bool(torch.equal(got.view(torch.int16),
                                                                 again.view(torch.int16))),
                "max_abs_err_vs_exact": float((got.double() - ex).abs().max()),
                "max_exact": float(ex.abs().max()),
                "oracle": f"float64 {self.form} (the per-op bf16 roundings bound the error by "
                          "2^-6 max); fused and separate launches compared bit for bit"}

    def exact(self):
        return torch.softmax(self.x.double(), 1)

    def cpu_baseline(self):
        import kernel_lib as KL
        from oracle.tile_ops import seeded
        rows = 1024  # a bounded sample: 32 tile rows of the full width (~10 s in all)
        x = seeded((rows, self.n), "uniform", self.seed, lo=-4, hi=4)
        t = [x, torch.ones(32, 32, dtype=torch.bfloat16),
             torch.zeros(rows, self.n, dtype=torch.bfloat16)]
        dt, reps = _eager(lambda ns: KL.make_softmax_one_store(ns, gc=self.n // 32, grid=(1, 1),
                                                               form=self.form), t)
        nbytes = self.work_per_step() * rows / self.n  # the step's bytes for `rows` rows
        return {"value": round(nbytes / dt / 1e9, 5), "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{rows} of the {self.n} rows through the eager tile-by-tile oracle "
                          f"executor running the same kernel (1 thread), {reps} runs of {dt:.2f} s"}


class RmsNormWorkload(SoftmaxWorkload):
    """RMS normalisation of a bf16 matrix written as one tt-lang store
    (tests/kernel_lib.py make_softmax_one_store, form "rms": y = x *
    rsqrt(broadcast(reduce_sum(x * x)) / W + 1e-5), one block per row band
    of 128 tiles, 8x8 grid): one row reduction and the program in one
    ttlh_reduce_rows_eltwise launch, on its dedicated kernel; HBM-bound;
    algorithmic bytes = x read once, y written once, the result tiles."""

    form = "rms"

    def __init__(self, name, n, separate=False, seed=1357):
        self.name, self.n, self.separate, self.seed = name, n, separate, seed
        self.config = (f"row RMS normalisation y = x * rsqrt(sum_r x^2 / W + 1e-5) in one store "
                       f"(spec reduce_sum / broadcast / rsqrt), x bf16 {n}x{n} U[-4,4], per-op "
                       f"bf16 rounding; one ttlh_reduce_rows_eltwise launch")

    def kernel_name(self):
        return "norm_rows_kernel"

    def traffic_kernels(self):
        return [("norm_rows_kernel<256, 2>", None)]

    def work_per_step(self):
        return 2 * self.n * self.n * 2 + self.n * 32 * 2

    def exact(self):
        x = self.x.double()
        return x * torch.rsqrt((x * x).mean(1, keepdim=True) + 1e-5)


class TilizeWorkload(Workload):
    """Row-major bf16 -> tilized element order (ttnn TILE_LAYOUT storage,
    16x16 faces) through ttlh_tilize; HBM-bound byte permutation, buffer sets
    rotated over > 1.2 GB."""

    def __init__(self, name, n, seed=5678):
        self.name, self.n, self.seed = name, n, seed
        self.config = (f"tilize bf16 {n}x{n} row-major -> 32x32 tiles of four 16x16 faces "
                       "(ttnn TILE_LAYOUT storage order)")

    def kernel_name(self):
        return "layout_kernel"

    def work_per_step(self):
        return 2 * self.n * self.n * 2

    def setup(self):
        from oracle.tile_ops import seeded
        from ttlhip import _lib as L
        self.L = L
        self.x = seeded((self.n, self.n), "uniform", self.seed, lo=-1, hi=1)
        x = self.x.cuda()
        nsets = n_sets(self.work_per_step())
        self.sets = [(x if i == 0 else x.clone(),
                      torch.empty(self.n * self.n, dtype=torch.bfloat16, device="cuda"))
                     for i in range(nsets)]

    def launch(self, i):
        src, dst = self.sets[i % len(self.sets)]
        self.L.call("ttlh_tilize", src.data_ptr(), self.n, dst.data_ptr(), self.n, self.n, 2,
                    self.L.stream_ptr())

    def check(self):
        from oracle import tile_ops as O
        self.launch(0)
        torch.cuda.synchronize()
        ok = torch.equal(self.sets[0][1].cpu(), O.tilize_ref(self.x))
        return {"bit_exact": bool(ok), "oracle": "reshape / permute restatement (tilize_ref)"}

    def cpu_baseline(self):
        from oracle import tile_ops as O
        dt, reps = _repeat(lambda: O.tilize_ref(self.x).contiguous(), max_reps=2000)
        return {"value": round(self.work_per_step() / dt / 1e9, 4), "unit": "GB/s",
                "cores": torch.get_num_threads(), "kind": "port",
                "sample": f"the full {self.n}x{self.n} tilize through the oracle's reshape / "
                          f"permute restatement, {reps} runs of {dt * 1e3:.2f} ms"}


class MatmulWorkload(PlanWorkload):
    """C3 through the multicore-style tt-lang kernel (13x10 grid, (1,1) CBs,
    store(acc=True) over K) -> one MFMA GEMM launch."""

    bound = "mfma"
    unit = "TFLOP/s"

    def __init__(self, name, M, N, K, seed=99):
        self.name, self.M, self.N, self.K, self.seed = name, M, N, K, seed
        self.config = (f"tiled matmul C = A.B bf16 {M}x{K}x{N}, N(0,1)/sqrt(K), fp32 accumulate, "
                       "bf16 out, 4x4-tile output blocks (BASELINE configs[2])")

    def kernel_name(self):
        return "mm_dma_kernel"

    def work_per_step(self):
        return 2.0 * self.M * self.N * self.K

    def traffic_kernels(self):
        return [("mm_dma_kernel", (self.M // 256) * (self.N // 256))]

    def algorithmic_bytes(self):
        return 2.0 * (self.M * self.K + self.K * self.N + self.M * self.N)

    def make_sets(self):
        import kernel_lib as KL
        import ttl
        import ttnn
        from oracle.tile_ops import seeded
        self.kernel = KL.make_matmul_multi(ttl, ttnn)
        std = 1.0 / math.sqrt(self.K)
        a = ttnn.from_torch(seeded((self.M, self.K), "normal", self.seed, std=std))
        b = ttnn.from_torch(seeded((self.K, self.N), "normal", self.seed + 1, std=std))
        c = ttnn.empty((self.M, self.N), dtype=torch.bfloat16)
        return [[a, b, c]]

    def check(self):
        self.launch(0)
        torch.cuda.synchronize()
        a, b, c = (t.to_torch() for t in self.sets[0])
        rows = torch.arange(0, self.M, max(1, self.M // 64))
        exact = a[rows].double() @ b.double()
        got = c[rows].double()
        return {"max_abs_err_rel": float((got - exact).abs().max() / exact.abs().max()),
                "rows_checked": int(rows.numel()), "oracle": "float64 product"}

    def cpu_baseline(self):
        import kernel_lib as KL
        import ttnn
        from oracle.tile_ops import seeded
        n = 1024
        std = 1.0 / math.sqrt(n)
        t = [seeded((n, n), "normal", self.seed, std=std),
             seeded((n, n), "normal", self.seed + 1, std=std),
             torch.zeros(n, n, dtype=torch.bfloat16)]
        dt, reps = _eager(lambda ns: KL.make_matmul_multi(ns, ttnn), t)
        steps = (n // 32) ** 3
        full = (self.M // 32) * (self.N // 32) * (self.K // 32)
        return {"value": round(2.0 * n ** 3 / dt / 1e12, 8), "unit": "TFLOP/s", "cores": 1,
                "kind": "port",
                "sample": f"{n}^3 ({steps} tile steps) through the eager tile-by-tile oracle "
                          f"executor (1 thread), {reps} runs of {dt:.2f} s; extrapolated to "
                          f"{self.M}x{self.K}x{self.N} ({full} tile steps) at the same rate: "
                          f"{dt * full / steps:.0f} s"}


class MatmulEpilogueWorkload(PlanWorkload):
    """relu(A.B + C) at C3's shape through the drop-in: one store per output
    block of the spec's block matmul plus a bias and an activation, planned
    as one fused launch (the GEMM with the store's program in its epilogue,
    the product never written to HBM)."""

    bound = "mfma"
    unit = "TFLOP/s"

    def __init__(self, name, M, N, K, seed=71):
        self.name, self.M, self.N, self.K, self.seed = name, M, N, K, seed
        self.config = (f"relu(A.B + C) bf16 {M}x{K}x{N}, N(0,1)/sqrt(K) operands, C N(0,1), "
                       "product rounded to bf16 before the bias (simulator semantics), "
                       "4x4-tile output blocks, (4, K/32) @ (K/32, 4) block matmuls")

    def kernel_name(self):
        return "mm_dma_epi_kernel"

    def work_per_step(self):
        return 2.0 * self.M * self.N * self.K

    def algorithmic_bytes(self):  # A, B, the bias and the output once (no product)
        return 2.0 * (self.M * self.K + self.K * self.N + 2 * self.M * self.N)

    def make_sets(self):
        import kernel_lib as KL
        import ttl
        import ttnn
        from oracle.tile_ops import seeded
        self.kernel = KL.make_matmul_epilogue(ttl, 4, self.K // 32, 4, "relu_bias")
        std = 1.0 / math.sqrt(self.K)
        a = ttnn.from_torch(seeded((self.M, self.K), "normal", self.seed, std=std))
        b = ttnn.from_torch(seeded((self.K, self.N), "normal", self.seed + 1, std=std))
        c = ttnn.from_torch(seeded((self.M, self.N), "normal", self.seed + 2))
        out = ttnn.empty((self.M, self.N), dtype=torch.bfloat16)
        return [[a, b, c, out]]

    def setup(self):
        super().setup()
        from ttlhip import plan as P
        (fl,) = self.plan.launches
        assert isinstance(fl, P.FusedMatmulLaunch), self.plan.describe()

    def check(self):
        self.launch(0)
        torch.cuda.synchronize()
        a, b, c, out = (t.to_torch() for t in self.sets[0])
        rows = torch.arange(0, self.M, max(1, self.M // 64))
        prod = (a[rows].double() @ b.double()).to(torch.bfloat16)
        exact = torch.relu((prod.double() + c[rows].double()).to(torch.bfloat16).double())
        got = out[rows].double()
        return {"max_abs_err_rel": float((got - exact).abs().max() / exact.abs().max()),
                "rows_checked": int(rows.numel()),
                "oracle": "float64 product rounded to bf16, bf16 bias add, relu"}

    def cpu_baseline(self):
        import kernel_lib as KL
        from oracle.tile_ops import seeded
        n = 1024
        std = 1.0 / math.sqrt(n)
        t = [seeded((n, n), "normal", self.seed, std=std),
             seeded((n, n), "normal", self.seed + 1, std=std),
             seeded((n, n), "normal", self.seed + 2), torch.zeros(n, n, dtype=torch.bfloat16)]
        dt, reps = _eager(lambda ns: KL.make_matmul_epilogue(ns, 4, n // 32, 4, "relu_bias"), t)
        return {"value": round(2.0 * n ** 3 / dt / 1e12, 8), "unit": "TFLOP/s", "cores": 1,
                "kind": "port",
                "sample": f"{n}^3 through the eager tile-by-tile oracle executor running the "
                          f"same kernel (1 thread), {reps} runs of {dt:.2f} s"}


class Bfp8MatmulWorkload(PlanWorkload):
    """C4 through the drop-in: the multicore tt-lang matmul kernel (13x10
    grid, store(acc=True) over K) with B a ttnn.bfloat8_b tensor, C = A (bf16
    [M,K], N(0,1)) . dequant(Bq), Bq the bfloat8_b tiles of an N(0, 0.02)
    fp32 [K,N] matrix.  The plan is one bf16 x bfloat8_b GEMM launch; at M =
    4096 that is the two-pass entry point (one dequantisation pass into a
    bf16 workspace from torch's caching allocator, then the bf16 GEMM), both
    kernels inside the timed step."""

    bound = "mfma"
    unit = "TFLOP/s"

    def __init__(self, name, M, N, K, seed=77):
        self.name, self.M, self.N, self.K, self.seed = name, M, N, K, seed
        self.config = (f"weight-quantised matmul bf16 [{M},{K}] x bfloat8_b [{K},{N}], fp32 "
                       "accumulate, bf16 out (BASELINE configs[3])")

    def kernel_name(self):
        from ttlhip import kernels as K
        return ("bfp8_unpack_kernel + mm_dma_kernel" if self.M >= K.BFP8_TWO_PASS_MIN_M
                else "mm256_kernel<bfp8>")

    def work_per_step(self):
        return 2.0 * self.M * self.N * self.K

    def traffic_kernels(self):
        blocks = ((self.M + 255) // 256) * ((self.N + 255) // 256)
        return [("bfp8_unpack_kernel", None), ("mm_dma_kernel", blocks)]

    def algorithmic_bytes(self):  # A, the packed weight tiles and C once
        return (2.0 * self.M * self.K + (self.K // 32) * (self.N // 32) * 1088
                + 2.0 * self.M * self.N)

    def make_sets(self):
        import kernel_lib as KL
        import ttl
        import ttnn
        from oracle.tile_ops import seeded
        self.kernel = KL.make_matmul_multi(ttl, ttnn)
        self.a = seeded((self.M, self.K), "normal", self.seed)
        self.w = seeded((self.K, self.N), "normal", self.seed + 1, torch.float32, std=0.02)
        wq = ttnn.from_torch(self.w, dtype=ttnn.bfloat8_b)
        c = ttnn.empty((self.M, self.N), dtype=torch.bfloat16)
        return [[ttnn.from_torch(self.a), wq, c]]

    def setup(self):
        super().setup()
        (l,) = self.plan.launches
        assert l.b_block, self.plan.describe()

    def check(self):
        from oracle import bfp8 as OB
        self.launch(0)
        torch.cuda.synchronize()
        rows = torch.arange(0, self.M, max(1, self.M // 32))
        wd = OB.unpack_c(OB.pack_c(self.w), self.K, self.N).double()
        exact = self.a[rows].double() @ wd
        got = self.sets[0][2].to_torch()[rows].double()
        return {"max_abs_err_rel": float((got - exact).abs().max() / exact.abs().max()),
                "rows_checked": int(rows.numel()),
                "oracle": "float64 product of the C oracle's dequantisation"}

    def cpu_baseline(self):
        from oracle import bfp8 as OB
        rows = 256
        bq = OB.pack_c(self.w)
        a = self.a[:rows]

        def work():
            w = OB.unpack_c(bq, self.K, self.N)
            return (a.float() @ w.float()).bfloat16()
        dt, reps = _repeat(work)
        return {"value": round(2.0 * rows * self.N * self.K / dt / 1e12, 6), "unit": "TFLOP/s",
                "cores": torch.get_num_threads(), "kind": "port",
                "sample": f"{rows} of the {self.M} rows of A: the C oracle's bfloat8_b decode of "
                          f"all of Bq plus a float32 torch CPU product, {reps} runs of {dt:.2f} s "
                          "(no simulator path exists for bfloat8_b)"}


class Bfp8LdsMatmulWorkload(Bfp8MatmulWorkload):
    """C4 on the north-star design: the same operands as the plan's launch,
    through the fused entry point ttlh_matmul_bfp8w (no workspace): the
    bfloat8_b tiles go into LDS packed and are dequantised there between the
    MFMAs (mm_dq_kernel).  At M = 4096 every weight tile is decoded once per
    256-row block of A (16 times), which is why the two-pass launch of the
    plan is faster at this M; this line reports the kernel itself."""

    def kernel_name(self):
        return "mm_dq_kernel"

    def traffic_kernels(self):
        return [("mm_dq_kernel", None)]

    def setup(self):
        super().setup()
        from ttlhip import kernels as Kn
        self._ops = [tuple(t._tensor for t in s) for s in self.sets]
        self._mm = Kn.matmul_bfp8w

    def launch(self, i):
        a, q, c = self._ops[i % len(self._ops)]
        self._mm(a, q, c, two_pass=False)


class SdpaWorkload(PlanWorkload):
    """C5 through the drop-in: attention written tile by tile with the spec's
    ops (tests/kernel_lib.py make_attention: @, reduce_max, exp, broadcast,
    reduce_sum, recip over intermediate CBs, 8x8 grid), planned onto one
    fused ttlh_sdpa_fwd launch; Q, V, out [B*H*S, D] and K^T as the
    transposed view of K rows (no staging copy)."""

    bound = "mfma"
    unit = "TFLOP/s"

    def __init__(self, name, B, H, S, D, seed=7):
        self.name, self.B, self.H, self.S, self.D, self.seed = name, B, H, S, D, seed
        self.config = (f"fused SDPA fwd Q,K,V bf16 [{B},{H},{S},{D}], N(0,1), scale 1/sqrt({D}), "
                       "non-causal, fp32 online softmax (BASELINE configs[4]); tile program "
                       "of @ / reduce_max / exp / broadcast / reduce_sum / recip through the "
                       "drop-in")

    def kernel_name(self):
        # the eight-wave kernel serves D = 128, non-causal, positive scale,
        # S % 256 == 0; the ping-pong kernel the other multiples of 256
        if self.D == 128 and self.S % 256 == 0:
            return "sdpa_w8_kernel"
        return "sdpa_pp_kernel" if self.S % 256 == 0 else "sdpa_fwd_kernel"

    def work_per_step(self):
        return 4.0 * self.B * self.H * self.S * self.S * self.D

    def algorithmic_bytes(self):  # Q, K, V and O once
        return 4.0 * 2 * self.B * self.H * self.S * self.D

    def make_sets(self):
        import kernel_lib as KL
        import ttl
        import ttnn
        from oracle.tile_ops import seeded
        n = self.B * self.H * self.S
        self.scale = 1.0 / math.sqrt(self.D)
        self.kernel = KL.make_attention(ttl, self.S, self.scale, grid=(8, 8))
        q, k, v = (seeded((n, self.D), "normal", self.seed + i).cuda() for i in range(3))
        return [[ttnn.Tensor(q), ttnn.Tensor(k.t()), ttnn.Tensor(v),
                 ttnn.empty((n, self.D), dtype=torch.bfloat16)]]

    def setup(self):
        super().setup()
        from ttlhip import plan as P
        assert isinstance(self.plan.launches[0], P.SdpaLaunch), self.plan.describe()

    def check(self):
        from oracle.tile_ops import sdpa_ref
        self.launch(0)
        torch.cuda.synchronize()
        q, kt, v, o = (x._tensor for x in self.sets[0])
        S, D = self.S, self.D
        h = self.B * self.H - 1  # the last (batch, head) pair
        rows = slice(h * S, (h + 1) * S)
        ref = sdpa_ref(*(x[rows].cpu().view(1, 1, S, D) for x in (q, kt.t(), v)), self.scale)
        got = o[rows].cpu().double().view(1, 1, S, D)
        return {"max_abs_err_rel": float((got - ref).abs().max() / ref.abs().max()),
                "heads_checked": 1, "oracle": "float64 softmax(QK^T s)V"}

    def cpu_baseline(self):
        import kernel_lib as KL
        from oracle.tile_ops import seeded
        S, D = self.S, self.D
        q, k, v = (seeded((S, D), "normal", self.seed + 10 + i) for i in range(3))
        t = [q, k.t().contiguous(), v, torch.zeros(S, D, dtype=torch.bfloat16)]
        dt, reps = _eager(lambda ns: KL.make_attention(ns, S, self.scale, grid=(1, 1)), t)
        return {"value": round(4.0 * S * S * D / dt / 1e12, 8), "unit": "TFLOP/s", "cores": 1,
                "kind": "port",
                "sample": f"one of the {self.B * self.H} (batch, head) pairs (S {S}, D {D}) "
                          f"through the eager tile-by-tile oracle executor running the same "
                          f"attention tile program (1 thread), {reps} run(s) of {dt:.2f} s"}


WORKLOADS = {
    "exp_bcast_mul_4096": lambda: EltwiseWorkload("exp_bcast_mul_4096", 4096, "pipe"),
    "eltwise_add_2048": lambda: EltwiseWorkload("eltwise_add_2048", 2048, "add"),
    "exp_bcast_mul_4096x3072": lambda: EltwiseWorkload("exp_bcast_mul_4096x3072", 4096, "pipe",
                                                       cols=3072),
    "matmul_bf16_4096": lambda: MatmulWorkload("matmul_bf16_4096", 4096, 4096, 4096),
    "matmul_bfp8w_4096x11008": lambda: Bfp8MatmulWorkload("matmul_bfp8w_4096x11008", 4096,
                                                          11008, 4096),
    "matmul_bfp8w_lds_4096x11008": lambda: Bfp8LdsMatmulWorkload("matmul_bfp8w_lds_4096x11008",
                                                                 4096, 11008, 4096),
    "matmul_bias_relu_4096": lambda: MatmulEpilogueWorkload("matmul_bias_relu_4096", 4096, 4096,
                                                            4096),
    "sdpa_4x32x4096x128": lambda: SdpaWorkload("sdpa_4x32x4096x128", 4, 32, 4096, 128),
    "reduce_sum_rows_4096": lambda: ReduceWorkload("reduce_sum_rows_4096", 4096),
    "row_dot_4096": lambda: RowDotWorkload("row_dot_4096", 4096),
    "softmax_rows_4096": lambda: SoftmaxWorkload("softmax_rows_4096", 4096),
    "rms_norm_rows_4096": lambda: RmsNormWorkload("rms_norm_rows_4096", 4096),
    "softmax_rows_4096_separate": lambda: SoftmaxWorkload("softmax_rows_4096_separate", 4096,
                                                          separate=True),
    "tilize_4096": lambda: TilizeWorkload("tilize_4096", 4096),
}
HEADLINE = "exp_bcast_mul_4096"


def measure(w: Workload, steps: int, warmup: int, use_graph: bool = True,
            samples: int = SAMPLES) -> dict:
    """Times exactly `steps` steps, `samples` times, at steady state.

    Each timed sample is `steps` launches of the plan enqueued on the launch
    stream between a pair of HIP events.  Before them, back-to-back work of
    at least PREROLL_MS (MFMA workloads: MFMA_PREROLL_MS) and
    PREROLL_MIN_STEPS steps is queued (replays of a HIP graph of the same
    steps, no host synchronisation), and at least three times the host's
    enqueue time of every timed launch: so the engine clock has ramped, the
    host has enqueued every timed launch before the GPU reaches the first
    event, and no idle gap or graph start-up lies inside a timed sample.  The
    reported per-step time is the median over the samples (all listed)."""
    w.setup()
    for i in range(warmup):
        w.launch(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    p0 = torch.cuda.Event(enable_timing=True)
    p1 = torch.cuda.Event(enable_timing=True)
    p0.record(stream)
    t0 = time.perf_counter()
    for i in range(3):
        w.launch(i)
    host = (time.perf_counter() - t0) / 3 * 1e3  # ms of host time per launch
    p1.record(stream)
    torch.cuda.synchronize()
    est = max(p0.elapsed_time(p1) / 3, 1e-4)  # ms per step on the GPU
    pre_ms = max(MFMA_PREROLL_MS if w.unit != "GB/s" else PREROLL_MS,
                 3.0 * host * steps * samples)
    pre_steps = max(PREROLL_MIN_STEPS, math.ceil(pre_ms / est))
    g = None
    if use_graph:
        s = torch.cuda.Stream()
        s.wait_stream(stream)
        with torch.cuda.stream(s):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                for i in range(steps):
                    w.launch(i)
        torch.cuda.synchronize()
        g.replay()  # untimed warm replay
        torch.cuda.synchronize()
    pre_reps = math.ceil(pre_steps / steps)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(samples)]
    torch.cuda.synchronize()
    for _ in range(pre_reps):
        if g is not None:
            g.replay()
        else:
            for i in range(steps):
                w.launch(i)
    for e0, e1 in ev:
        e0.record(stream)
        for i in range(steps):
            w.launch(i)
        e1.record(stream)
    torch.cuda.synchronize()
    per_s = sorted(e0.elapsed_time(e1) / steps for e0, e1 in ev)
    per = per_s[len(per_s) // 2]
    work = w.work_per_step()
    scale = 1e9 if w.unit == "GB/s" else 1e12
    achieved = work / (per * 1e-3) / scale
    peak = HBM_PEAK_GBS if w.unit == "GB/s" else BF16_PEAK_TFLOPS
    return {"name": w.name, "config": w.config, "kernel": w.kernel_name(), "bound": w.bound,
            "steps": steps, "samples": samples, "preroll_steps": pre_reps * steps,
            "host_ms_per_launch": host,
            "ms_total": per * steps * samples, "ms_per_step": per,
            "ms_per_step_min": per_s[0], "ms_per_step_max": per_s[-1], "achieved": achieved,
            "unit": w.unit, "peak": peak, "frac": achieved / peak, "work_per_step": work}


def copy_ceiling(reps: int = 50) -> dict:
    """Empirical HBM ceiling: a plain copy (the one-step program `load a`,
    which ttlh_eltwise runs on its flat streaming kernel) of 256 MiB, read +
    write counted, two buffer pairs alternating so the 256 MB Infinity Cache
    cannot serve them, timed with HIP events on the launch stream."""
    from ttlhip import expr as X
    from ttlhip import kernels as K
    rows, cols = 8192, 16384  # bf16: COPY_BYTES (256 MiB)
    pairs = [(torch.ones(rows, cols, dtype=torch.bfloat16, device="cuda"),
              torch.empty(rows, cols, dtype=torch.bfloat16, device="cuda")) for _ in range(2)]
    prog = X.compile_expr(X.Leaf(0, torch.bfloat16))
    for src, dst in pairs:
        K.eltwise(prog, [K.OperandMap(src)], dst)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        src, dst = pairs[i % 2]
        K.eltwise(prog, [K.OperandMap(src)], dst)
    e1.record(stream)
    torch.cuda.synchronize()
    per = e0.elapsed_time(e1) / reps
    nbytes = 2 * rows * cols * 2
    ok = bool(torch.equal(pairs[1][1][:64], pairs[1][0][:64]))
    del pairs
    torch.cuda.empty_cache()
    return {"value": round(nbytes / (per * 1e-3) / 1e9, 1), "unit": "GB/s", "copy_ok": ok,
            "how": "plain copy of 256 MiB of bf16 through ttlh_eltwise's flat streaming kernel "
                   f"(read + write), two buffer pairs alternating, {reps} copies timed with HIP "
                   "events"}


def traffic_for(name: str):
    """HBM bytes per launch measured by rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
    (scaled by a copy kernel's readings), from the committed profile summary."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f).get(name)
        return None if t is None else t.get("hbm_bytes_per_launch")  # measured for t["kernel"]
    except (OSError, ValueError):
        return None


def summarize_traffic(fetch_csv: str, write_csv: str):
    """(markdown, json) of HBM bytes per step from two rocprofv3 --pmc passes
    over a bench.py run (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch).
    Each counter is scaled by what it reads for the run's copy-ceiling
    kernel, which moves COPY_BYTES each way; per workload the medians over
    the dispatches of each kernel it launches (traffic_kernels) are summed
    and compared with its algorithmic bytes."""
    import csv
    import statistics

    def read(path, counter):
        per = {}
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                if row["Counter_Name"] != counter:
                    continue
                name = row["Kernel_Name"].replace("(anonymous namespace)::", "")
                name = name.removeprefix("void ").removeprefix("ttlh::").split("(")[0]
                wgs = int(row["Grid_Size"]) // max(1, int(row["Workgroup_Size"]))
                per.setdefault((name, wgs), []).append(float(row["Counter_Value"]))
        return per

    fetch, write = read(fetch_csv, "FETCH_SIZE"), read(write_csv, "WRITE_SIZE")
    cal = next(k for k in fetch if k[0].startswith("flat_kernel<1, 1u, true>"))
    f_kib, w_kib = statistics.median(fetch[cal]), statistics.median(write[cal])
    fs, ws = COPY_BYTES / (f_kib * 1024), COPY_BYTES / (w_kib * 1024)
    out = {"_calibration": {"kernel": cal[0], "bytes_each_way": COPY_BYTES,
                            "fetch_size_kib": round(f_kib, 1), "write_size_kib": round(w_kib, 1),
                            "fetch_scale": round(fs, 5), "write_scale": round(ws, 5)}}
    lines = ["| workload | kernels | HBM bytes / step | algorithmic bytes | ratio |",
             "|---|---|---|---|---|"]
    for name, make in WORKLOADS.items():
        w = make()
        ks, total = [], 0.0
        if not w.traffic_kernels():
            continue
        for sub, wgs in w.traffic_kernels():
            hits = [k for k in fetch if sub in k[0] and (wgs is None or k[1] == wgs) and k in write]
            if not hits:
                break
            k = max(hits, key=lambda k: len(fetch[k]))
            fm, wm = statistics.median(fetch[k]), statistics.median(write[k])
            b = (fm * fs + wm * ws) * 1024
            total += b
            ks.append({"kernel": k[0], "workgroups": k[1], "dispatches": len(fetch[k]),
                       "fetch_size_kib_median": round(fm, 1), "write_size_kib_median": round(wm, 1),
                       "hbm_bytes": round(b)})
        else:
            alg = w.algorithmic_bytes()
            out[name] = {"hbm_bytes_per_launch": round(total), "algorithmic_bytes": round(alg),
                         "traffic_over_algorithmic": round(total / alg, 4), "kernels": ks}
            names = " + ".join(f"`{k['kernel']}` ({k['workgroups']} WGs)" for k in ks)
            lines.append(f"| {name} | {names} | {round(total):,} | {round(alg):,} | "
                         f"{total / alg:.4f} |")
    return "\n".join(lines), out


def summarize_counters(paths, kernel: str, wgs: int = 0) -> dict:
    """Median per dispatch of every counter in rocprofv3 --pmc passes
    (`*_counter_collection.csv`) over the dispatches of the kernel whose name
    contains `kernel` (and that has `wgs` workgroups, if given)."""
    import csv
    import statistics
    per = {}
    for path in paths:
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                name = row["Kernel_Name"]
                n_wg = int(row["Grid_Size"]) // max(1, int(row["Workgroup_Size"]))
                if kernel not in name or (wgs and n_wg != wgs):
                    continue
                per.setdefault(row["Counter_Name"], []).append(float(row["Counter_Value"]))
    return {c: {"median": statistics.median(v), "dispatches": len(v)} for c, v in per.items()}


def summarize_trace(path: str, steps: int, samples: int = SAMPLES, gap_us: float = 200.0) -> str:
    """Markdown table of kernel durations from a rocprofv3 kernel trace
    (`*_kernel_trace.csv`) of a bench.py run, taken from its steady stretch.
    All dispatches, in start order, are split into bursts that run back to
    back (less than `gap_us` between one dispatch's end and the next one's
    start, whatever the kernels).  Per kernel (name and workgroup count), the
    burst holding most of its dispatches is the pre-roll plus the timed
    samples; its last `samples * steps` dispatches of that kernel (fewer if
    the burst is shorter) are reported.  Warm-up, probe and check dispatches,
    which run at a cold clock or behind a host synchronisation, fall outside
    it."""
    import csv
    rows_in = []
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            name = row["Kernel_Name"].replace("(anonymous namespace)::", "")
            name = name.removeprefix("void ").removeprefix("ttlh::").split("(")[0][:72]
            wgs = int(row["Grid_Size_X"]) * int(row["Grid_Size_Y"]) * int(row["Grid_Size_Z"]) // max(
                1, int(row["Workgroup_Size_X"]) * int(row["Workgroup_Size_Y"]) * int(row["Workgroup_Size_Z"]))
            rows_in.append((int(row["Start_Timestamp"]), int(row["End_Timestamp"]), (name, wgs)))
    rows_in.sort()
    burst, prev_end = 0, None
    per = {}  # kernel -> {burst: [durations in start order]}
    for s, e, key in rows_in:
        if prev_end is not None and (s - prev_end) * 1e-3 >= gap_us:
            burst += 1
        prev_end = e if prev_end is None else max(prev_end, e)
        per.setdefault(key, {}).setdefault(burst, []).append((e - s) * 1e-3)
    lines = ["| kernel | workgroups | dispatches | in its longest back-to-back burst | reported | "
             "median us | mean us | min us | max us |", "|---|---|---|---|---|---|---|---|---|"]
    rows = []
    for (name, wgs), bursts in per.items():
        best = max(bursts.values(), key=len)
        if len(best) < PREROLL_MIN_STEPS:
            continue  # not a timed workload kernel (set-up, fills, copies)
        timed = best[-samples * steps:]
        us = sorted(timed)
        rows.append((name, wgs, sum(map(len, bursts.values())), len(best), len(timed),
                     us[len(us) // 2], sum(us) / len(us), us[0], us[-1]))
    for r in sorted(rows, key=lambda r: -r[5]):
        lines.append(f"| `{r[0]}` | {r[1]} | {r[2]} | {r[3]} | {r[4]} | {r[5]:.2f} | {r[6]:.2f} | "
                     f"{r[7]:.2f} | {r[8]:.2f} |")
    return "\n".join(lines)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", default="", help="comma-separated workload names")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="print the timed-replay kernel durations of a rocprofv3 kernel trace of "
                         "a bench.py run made with the same --steps, then exit (no GPU used)")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the HBM traffic table of two rocprofv3 --pmc passes (FETCH_SIZE, "
                         "WRITE_SIZE) over a bench.py run and write profiles/traffic.json, then "
                         "exit (no GPU used)")
    ap.add_argument("--counter-summary", nargs="+", metavar="ARG",
                    help="KERNEL[:WORKGROUPS] CSV...: medians per dispatch of the counters of "
                         "rocprofv3 --pmc passes for one kernel, as JSON, then exit (no GPU used)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run one 256 MiB device copy (PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.counter_summary:
        kern, _, wg = args.counter_summary[0].partition(":")
        print(json.dumps(summarize_counters(args.counter_summary[1:], kern, int(wg or 0)),
                         indent=1))
        return 0
    if args.traffic_summary:
        md, js = summarize_traffic(*args.traffic_summary)
        with open(TRAFFIC_FILE, "w") as f:
            json.dump(js, f, indent=1)
            f.write("\n")
        print(md)
        return 0
    if args.trace_summary:
        print(summarize_trace(args.trace_summary, args.steps))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"--gpus {args.gpus}). Every config would shard without communication: the "
              "elementwise ones by tile rows, the matmuls by output columns, attention by "
              "(batch, head).", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (no HIP device visible)", file=sys.stderr)
        return 1
    if args.copy_calibration:
        src = torch.ones(128 * 1024 * 1024, dtype=torch.int16, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    names = [n for n in (args.only.split(",") if args.only else WORKLOADS) if n]
    if HEADLINE not in names:
        names.insert(0, HEADLINE)
    ceiling = copy_ceiling()
    log(f"[bench] empirical copy ceiling {ceiling['value']} GB/s")
    results = {}
    for n in names:
        w = WORKLOADS[n]()
        log(f"[bench] {n}: steps={args.steps} warmup={args.warmup}")
        r = measure(w, args.steps, args.warmup, use_graph=not args.no_graph)
        r["parity"] = w.check()
        r["traffic"] = traffic_for(n)
        if w.unit == "GB/s":
            r["empirical_peak"] = ceiling["value"]
            r["frac_of_empirical"] = r["achieved"] / ceiling["value"]
        results[n] = r
        log(f"[bench] {n}: {r['steps']} steps, {r['ms_per_step'] * 1e3:.2f} us/step {r['achieved']:.1f} {r['unit']} "
            f"({r['frac'] * 100:.1f}%) parity={r['parity']}")
        if not args.no_cpu:
            r["cpu_baseline"] = w.cpu_baseline()
            log(f"[bench] {n}: cpu baseline {r['cpu_baseline']['value']} {r['unit']} "
                f"({r['cpu_baseline']['sample']})")
        del w
        torch.cuda.empty_cache()
    h = results[HEADLINE]
    cpu = h.get("cpu_baseline")
    line = {
        "metric": "eltwise GB/s (% HBM peak); matmul/SDPA bf16 TFLOP/s (% MFMA peak) @1 GPU",
        "value": round(h["achieved"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded; resident in HBM; every workload's buffer sets rotated over > 1.2 GB)",
        "config": {"workload": h["config"], "kernel": "tt-lang kernel via drop-in ttl -> "
                   "ttlh_eltwise flat_kernel", "tiles": "32x32", "cb_block": "4x4 tiles",
                   "grid": "(8, 8) tt-lang cores -> one grid-wide launch"},
        "roofline": {"bound": h["bound"], "achieved": round(h["achieved"], 2), "peak": h["peak"],
                     "unit": h["unit"], "frac": round(h["frac"], 4), "traffic": h["traffic"],
                     "empirical_peak": ceiling["value"],
                     "frac_of_empirical": round(h["achieved"] / ceiling["value"], 4)},
        "copy_ceiling": ceiling,
        "cpu_baseline": cpu,
        "workloads": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()
                       if k != "cpu_baseline" or n != HEADLINE}
                      for n, r in results.items()],
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
