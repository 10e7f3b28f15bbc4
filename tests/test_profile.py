"""The auto-profile report (TTLANG_AUTO_PROFILE=1): store sites carry their
kernel source line, the per-launch work model equals the algorithmic bytes /
flops bench.py uses, and the report names line, launch and rate."""

import linecache

import pytest
import torch

import kernel_lib as KL
import ttl
import ttnn
from oracle import tile_ops as O
from ttlhip import plan as P
from ttlhip import profile


def _args(ts):
    return {i: ttnn.Tensor(t) for i, t in enumerate(ts)}


def test_store_sites_carry_source_lines_and_work():
    n = 256
    ts = [O.seeded((n, n), "uniform", 1), O.seeded((1, n), "uniform", 2),
          O.seeded((n, n), "uniform", 3), torch.zeros(n, n, dtype=torch.bfloat16)]
    args = _args(ts)
    plan = KL.make_exp_row_pipe(ttl, g=2, grid=(2, 2)).trace(*args.values())
    (l,) = plan.launches
    fname, line = l.loc
    assert fname.endswith("kernel_lib.py") and ".store(" in linecache.getline(fname, line)
    work, unit, peak = profile.launch_work(l, args)
    # exp(a + b_row) * c: a, c and y in full, the row vector once (bench.py's C2 formula)
    assert (work, unit, peak) == (3 * n * n * 2 + n * 2, "GB/s", 8000.0)
    text = profile.report("exp_row_pipe", (2, 2), plan, args, [10.0])
    assert f"{line:>6}" in text and ".store(" in text and "GB/s" in text
    rate = work / 10e-6 / 1e9
    assert f"{rate:9.1f}" in text


def test_matmul_work_is_2mnk():
    a, b = torch.rand(128, 256).bfloat16(), torch.rand(256, 96).bfloat16()
    args = _args([a, b, torch.zeros(128, 96, dtype=torch.bfloat16)])
    plan = KL.make_matmul_single(ttl).trace(*args.values())
    (l,) = plan.launches
    assert profile.launch_work(l, args) == (2.0 * 128 * 96 * 256, "TFLOP/s", 2500.0)
    assert "ttlh_matmul 128x96x256" in profile.report("mm", (1, 1), plan, args, [3.0])


@pytest.mark.gpu
def test_auto_profile_report_on_device(monkeypatch, capsys):
    monkeypatch.setenv("TTLANG_AUTO_PROFILE", "1")
    n = 512
    ts = [O.seeded((n, n), "uniform", 4), O.seeded((1, n), "uniform", 5),
          O.seeded((n, n), "uniform", 6), torch.zeros(n, n, dtype=torch.bfloat16)]
    k = KL.make_exp_row_pipe(ttl, g=2, grid=(2, 2))
    args = [ttnn.from_torch(t) for t in ts]
    k(*args)
    out = capsys.readouterr().out
    assert "TTLANG AUTO-PROFILE REPORT" in out and ".store(" in out and "GB/s" in out
    # the profiled call still computed the result
    ref = torch.exp(ts[0] + ts[1]) * ts[2]
    assert int(O.bf16_ulp_diff(ttnn.to_torch(args[3]), ref).max()) <= 1


def test_fused_row_launch_work_reads_each_operand_once():
    # a softmax in one store: one ReduceEltwiseLaunch whose work is x read
    # once, y written once and one result per row of each reduction (the
    # report's model for reductions), not x read three times
    rows, cols = 64, 512
    ts = [O.seeded((rows, cols), "uniform", 7, lo=-4, hi=4),
          torch.ones(32, 32, dtype=torch.bfloat16), torch.zeros(rows, cols, dtype=torch.bfloat16)]
    args = _args(ts)
    plan = KL.make_softmax_one_store(ttl, gc=cols // 32, grid=(2, 1)).trace(*args.values())
    (l,) = plan.launches
    assert isinstance(l, P.ReduceEltwiseLaunch)
    work, unit, _ = profile.launch_work(l, args)
    assert unit == "GB/s" and work == 2 * rows * cols * 2 + 2 * rows * 2
    text = profile.report("softmax", (2, 1), plan, args, [5.0])
    assert "ttlh_reduce_rows_eltwise 64x512: row max+sum" in text
