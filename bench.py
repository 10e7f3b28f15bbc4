#!/usr/bin/env python3
"""Benchmark of the TTL tile-op hot path on one MI355X.

`python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAMES]` prints ONE
JSON line.  The headline workload is BASELINE.json configs[1], the fused
elementwise + broadcast pipe Y = exp(A + b_row) * C on bf16 4096x4096 tiles;
`value` is its whole-job HBM throughput in GB/s.  The other configs are
measured in the same run and reported under "workloads".

A "step" is one pass of the hot path over one batch of synthetic input: one
kernel launch over one resident buffer set.  Inputs live in HBM before the
timed region starts; eltwise configs rotate buffer sets totalling > 256 MB so
the 256 MB Infinity Cache cannot serve them.  The K timed launches are
captured once into a HIP graph and replayed, so host launch overhead does not
pad the small kernels; HIP events on the launch stream bracket the replay.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tt-lang_amd"))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, TFLOP/s


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# --------------------------------------------------------------------------
# workloads
# --------------------------------------------------------------------------

class Workload:
    name = ""
    bound = "hbm"
    unit = "GB/s"

    def setup(self):  # allocate resident inputs
        raise NotImplementedError

    def launch(self, i: int):  # enqueue step i on the current stream
        raise NotImplementedError

    def work_per_step(self) -> float:  # algorithmic bytes or flops of one launch
        raise NotImplementedError

    def kernel_name(self) -> str:
        raise NotImplementedError


class EltwiseWorkload(Workload):
    """C1 (eltwise add 2048^2) and C2 (exp(A + b_row) * C, 4096^2)."""

    def __init__(self, name, rows, cols, expr_kind, seed=1234):
        self.name = name
        self.rows, self.cols = rows, cols
        self.kind = expr_kind
        self.seed = seed

    def kernel_name(self):
        return "eltwise_kernel"

    def work_per_step(self):
        n = self.rows * self.cols * 2
        return 3 * n if self.kind == "add" else 3 * n + self.cols * 2

    def build_expr(self, t):
        from ttlhip import expr as X
        from ttlhip.kernels import OperandMap

        bf = torch.bfloat16
        if self.kind == "add":
            a, b = X.Leaf(OperandMap(t["a"]), bf), X.Leaf(OperandMap(t["b"]), bf)
            return X.Binary("add", a, b, bf)
        a = X.Leaf(OperandMap(t["a"]), bf)
        b = X.Leaf(OperandMap(t["b"]), bf)
        c = X.Leaf(OperandMap(t["c"]), bf)
        return X.Binary("mul", X.Unary("exp", X.Binary("add", a, b, bf), bf), c, bf)

    def cpu_inputs(self, seed):
        from oracle.tile_ops import seeded
        r, c = self.rows, self.cols
        if self.kind == "add":
            return {"a": seeded((r, c), "uniform", seed, lo=-1, hi=1),
                    "b": seeded((r, c), "uniform", seed + 1, lo=-1, hi=1)}
        return {"a": seeded((r, c), "uniform", seed, lo=-2, hi=2),
                "b": seeded((1, c), "uniform", seed + 1, lo=-2, hi=2),
                "c": seeded((r, c), "uniform", seed + 2, lo=-2, hi=2)}

    def setup(self):
        from ttlhip import expr as X

        per_set = self.work_per_step()
        self.nsets = max(3, math.ceil(300e6 / per_set))
        self.sets = []
        base = {k: v.cuda() for k, v in self.cpu_inputs(self.seed).items()}
        for s in range(self.nsets):
            t = base if s == 0 else {k: v.clone() for k, v in base.items()}
            out = torch.empty((self.rows, self.cols), dtype=torch.bfloat16, device="cuda")
            e = self.build_expr(t)
            prog = X.compile_expr(e)
            self.sets.append((t, out, prog))
        self._prepared = [self._prepare(t, out, prog) for (t, out, prog) in self.sets]

    def _prepare(self, t, out, prog):
        from ttlhip import _lib as L
        from ttlhip.kernels import _operand_struct

        n = len(prog.steps)
        instrs = (L.Instr * n)()
        ops = (L.Operand * n)()
        for k, s in enumerate(prog.steps):
            instrs[k] = L.Instr(s.op, s.form, s.rnd, 0, s.imm)
            if s.leaf is not None:
                ops[k] = _operand_struct(s.leaf.ref, 0, 0, self.rows, self.cols)
        return (instrs, ops, n, out.data_ptr(), L.TTLH_BF16, out.stride(0), 0, 0, self.rows,
                self.cols)

    def launch(self, i):
        from ttlhip import _lib as L
        args = self._prepared[i % self.nsets]
        L.call("ttlh_eltwise", *args, L.stream_ptr())

    def check(self):
        """Parity of set 0 against the oracle (bit-exact except exp: <= 1 ulp)."""
        from oracle import tile_ops as O
        t, out, _ = self.sets[0]
        self.launch(0)
        torch.cuda.synchronize()
        env = {k: v.cpu() for k, v in t.items()}
        if self.kind == "add":
            ref = O.eval_expr(("add", ("leaf", "a"), ("leaf", "b")), env)
        else:
            ref = O.eval_expr(("mul", ("exp", ("add", ("leaf", "a"), ("leaf", "b"))),
                               ("leaf", "c")), env)
        ulp = O.bf16_ulp_diff(out.cpu(), ref)
        return {"max_ulp": int(ulp.max()), "mismatch_frac": float((ulp > 0).float().mean())}

    def cpu_baseline(self, budget_s=8.0):
        """Oracle timed tile-by-tile, one torch op per 32x32 tile on one
        thread (the simulator's execution granularity), on a sample of tiles."""
        from oracle import tile_ops as O
        env = self.cpu_inputs(self.seed)
        nthreads = torch.get_num_threads()
        torch.set_num_threads(1)
        try:
            rt, ct = self.rows // 32, self.cols // 32
            done, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < budget_s and done < rt * ct:
                r, c = divmod(done, ct)
                a = env["a"][r * 32:(r + 1) * 32, c * 32:(c + 1) * 32]
                b = env["b"][0:1, c * 32:(c + 1) * 32] if self.kind != "add" else \
                    env["b"][r * 32:(r + 1) * 32, c * 32:(c + 1) * 32]
                if self.kind == "add":
                    y = a + b
                else:
                    y = torch.exp(a + b) * env["c"][r * 32:(r + 1) * 32, c * 32:(c + 1) * 32]
                done += 1
            dt = time.perf_counter() - t0
        finally:
            torch.set_num_threads(nthreads)
        bytes_per_tile = self.work_per_step() / (rt * ct)
        return {"value": done * bytes_per_tile / dt / 1e9, "unit": "GB/s", "cores": 1,
                "kind": "port",
                "sample": f"{done} of {rt * ct} output tiles, tile-by-tile torch CPU ops "
                          f"(simulator granularity), {dt:.1f} s"}


class MatmulWorkload(Workload):
    """C3: C[M,N] = A[M,K] . B[K,N], bf16 in, fp32 accumulate, bf16 out."""

    bound = "mfma"
    unit = "TFLOP/s"

    def __init__(self, name, M, N, K, seed=99):
        self.name, self.M, self.N, self.K, self.seed = name, M, N, K, seed

    def kernel_name(self):
        return "mm_bf16_kernel"

    def work_per_step(self):
        return 2.0 * self.M * self.N * self.K

    def setup(self):
        from oracle.tile_ops import seeded
        std = 1.0 / math.sqrt(self.K)
        self.a = seeded((self.M, self.K), "normal", self.seed, std=std).cuda()
        self.b = seeded((self.K, self.N), "normal", self.seed + 1, std=std).cuda()
        self.c = torch.empty((self.M, self.N), dtype=torch.bfloat16, device="cuda")
        from ttlhip import _lib as L
        self._args = (self.a.data_ptr(), L.TTLH_BF16, self.K, self.b.data_ptr(), L.TTLH_BF16,
                      self.N, self.c.data_ptr(), L.TTLH_BF16, self.N, self.M, self.N, self.K, 0)

    def launch(self, i):
        from ttlhip import _lib as L
        L.call("ttlh_matmul", *self._args, L.stream_ptr())

    def check(self):
        """64 sampled rows against float64: max error relative to max |C|."""
        self.launch(0)
        torch.cuda.synchronize()
        rows = torch.arange(0, self.M, max(1, self.M // 64))
        exact = self.a.cpu()[rows].double() @ self.b.cpu().double()
        got = self.c.cpu()[rows].double()
        return {"max_abs_err_rel": float((got - exact).abs().max() / exact.abs().max()),
                "rows_checked": int(rows.numel())}


class Bfp8MatmulWorkload(MatmulWorkload):
    """C4: C = A (bf16 [M,K], N(0,1)) . dequant(Bq) with Bq the bfloat8_b
    tiles of a N(0, 0.02) fp32 [K,N] matrix; dequantised in LDS."""

    def kernel_name(self):
        return "mm_bf16_kernel<bfp8>"

    def setup(self):
        from oracle.tile_ops import seeded
        from ttlhip import kernels as K
        self.a = seeded((self.M, self.K), "normal", self.seed).cuda()
        w = seeded((self.K, self.N), "normal", self.seed + 1, torch.float32, std=0.02)
        self.bq = K.bfp8_pack_host(w).cuda()
        self.c = torch.empty((self.M, self.N), dtype=torch.bfloat16, device="cuda")
        self._args = (self.a.data_ptr(), self.K, self.bq.data_ptr(), self.c.data_ptr(), self.N,
                      self.M, self.N, self.K)

    def launch(self, i):
        from ttlhip import _lib as L
        L.call("ttlh_matmul_bfp8w", *self._args, L.stream_ptr())

    def check(self):
        from oracle import bfp8 as OB
        self.launch(0)
        torch.cuda.synchronize()
        rows = torch.arange(0, self.M, max(1, self.M // 32))
        wd = OB.unpack_c(self.bq.cpu(), self.K, self.N).double()
        exact = self.a.cpu()[rows].double() @ wd
        got = self.c.cpu()[rows].double()
        return {"max_abs_err_rel": float((got - exact).abs().max() / exact.abs().max()),
                "rows_checked": int(rows.numel())}


class SdpaWorkload(Workload):
    """C5: softmax(Q K^T / sqrt(128)) V, bf16 [4, 32, 4096, 128], non-causal."""

    bound = "mfma"
    unit = "TFLOP/s"

    def __init__(self, name, B, H, S, D, seed=7):
        self.name, self.B, self.H, self.S, self.D, self.seed = name, B, H, S, D, seed

    def kernel_name(self):
        return "sdpa_fwd_kernel"

    def work_per_step(self):
        return 4.0 * self.B * self.H * self.S * self.S * self.D

    def setup(self):
        from oracle.tile_ops import seeded
        shape = (self.B, self.H, self.S, self.D)
        self.q, self.k, self.v = (seeded(shape, "normal", self.seed + i).cuda() for i in range(3))
        self.o = torch.empty_like(self.q)
        self.scale = 1.0 / math.sqrt(self.D)
        self._args = (self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(), self.o.data_ptr(),
                      self.B, self.H, self.S, self.D, self.scale, 0)

    def launch(self, i):
        from ttlhip import _lib as L
        L.call("ttlh_sdpa_fwd", *self._args, L.stream_ptr())

    def check(self):
        from oracle.tile_ops import sdpa_ref
        self.launch(0)
        torch.cuda.synchronize()
        ref = sdpa_ref(self.q[:1, :1].cpu(), self.k[:1, :1].cpu(), self.v[:1, :1].cpu(), self.scale)
        got = self.o[:1, :1].cpu().double()
        return {"max_abs_err_rel": float((got - ref).abs().max() / ref.abs().max()),
                "heads_checked": 1}


WORKLOADS = {
    "eltwise_add_2048": lambda: EltwiseWorkload("eltwise_add_2048", 2048, 2048, "add"),
    "exp_bcast_mul_4096": lambda: EltwiseWorkload("exp_bcast_mul_4096", 4096, 4096, "pipe"),
    "matmul_bf16_4096": lambda: MatmulWorkload("matmul_bf16_4096", 4096, 4096, 4096),
    "matmul_bfp8w_4096x11008": lambda: Bfp8MatmulWorkload("matmul_bfp8w_4096x11008", 4096, 11008,
                                                          4096),
    "sdpa_4x32x4096x128": lambda: SdpaWorkload("sdpa_4x32x4096x128", 4, 32, 4096, 128),
}
HEADLINE = "exp_bcast_mul_4096"


def measure(w: Workload, steps: int, warmup: int, use_graph: bool = True):
    w.setup()
    for i in range(warmup):
        w.launch(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
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
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    if g is not None:
        g.replay()
    else:
        for i in range(steps):
            w.launch(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    per = ms / steps
    work = w.work_per_step()
    achieved = work / (per * 1e-3) / (1e9 if w.unit == "GB/s" else 1e12)
    peak = HBM_PEAK_GBS if w.unit == "GB/s" else BF16_PEAK_TFLOPS
    return {"name": w.name, "ms_total": ms, "ms_per_step": per, "achieved": achieved,
            "unit": w.unit, "peak": peak, "frac": achieved / peak, "work_per_step": work,
            "kernel": w.kernel_name(), "bound": w.bound}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", default="", help="comma-separated workload names")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"--gpus {args.gpus}); the per-GPU work shards without communication, "
              f"see DESIGN.md.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (no HIP device visible)", file=sys.stderr)
        return 1
    names = [n for n in (args.only.split(",") if args.only else WORKLOADS) if n]
    if HEADLINE not in names:
        names.insert(0, HEADLINE)
    results = {}
    checks = {}
    for n in names:
        w = WORKLOADS[n]()
        log(f"[bench] {n}: steps={args.steps} warmup={args.warmup}")
        results[n] = measure(w, args.steps, args.warmup, use_graph=not args.no_graph)
        checks[n] = w.check()
        results[n]["parity"] = checks[n]
        log(f"[bench] {n}: {results[n]['ms_per_step']*1e3:.2f} us/step "
            f"{results[n]['achieved']:.1f} {results[n]['unit']} ({results[n]['frac']*100:.1f}%) "
            f"parity={checks[n]}")
        if n == HEADLINE:
            headline_w = w
        del w
        torch.cuda.empty_cache()
    h = results[HEADLINE]
    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline ...")
        cpu = WORKLOADS[HEADLINE]().cpu_baseline()
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
        "data": "synthetic (seeded U[-2,2] bf16; resident in HBM; buffer sets rotated)",
        "config": {"workload": "fused eltwise pipe + broadcast: Y = exp(A + b_row) * C, "
                               "A,C bf16 4096x4096, b_row 1x4096 (BASELINE configs[1])",
                   "tiles": "32x32", "grid": "whole tensor, one launch"},
        "roofline": {"bound": h["bound"], "achieved": round(h["achieved"], 2),
                     "peak": h["peak"], "unit": h["unit"], "frac": round(h["frac"], 4),
                     "traffic": None},
        "cpu_baseline": cpu,
        "workloads": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
                      for r in results.values()],
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
