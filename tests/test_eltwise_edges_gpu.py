"""Signed zeros, NaN, infinities and subnormals through the elementwise
kernels, against torch, whose CPU ops are the simulator's arithmetic
(python/sim/ttnnsim.py:384-452).

relu is clamp_min(x, 0) in torch: -0 stays -0 on both of torch's CPU paths
(scalar and vectorised), so the kernels must return it bit for bit.  NaN
results are compared as NaN (torch's own payloads differ between its scalar
and vectorised paths: 0x7fc0 against 0xffff for relu / maximum of a NaN), and
so is the order of +0 and -0 under maximum / minimum, which torch's two paths
also resolve differently: both are parity unpinned at those points.
"""

import pytest
import torch

from ttlhip import expr as X
from ttlhip import kernels as Kn

pytestmark = pytest.mark.gpu

B16 = torch.bfloat16
EDGES = [-0.0, 0.0, float("nan"), -float("nan"), -1.0, 1.0, float("inf"), -float("inf"),
         1e-40, -1e-40, 3.0e38, -2.5]


def _edge_tensor(rows=32, cols=4096):
    v = torch.tensor(EDGES * (cols // len(EDGES) + 1), dtype=B16)[:cols]
    return v.reshape(1, cols).repeat(rows, 1).contiguous()


def _run(prog_expr, operands, shape):
    p = X.compile_expr(prog_expr)
    out = torch.empty(shape, dtype=B16, device="cuda")
    ops = [Kn.OperandMap(operands[s.leaf.ref]) if s.leaf is not None else None for s in p.steps]
    Kn.eltwise(p, ops, out)
    torch.cuda.synchronize()
    return out.cpu()


def _same(got, ref):
    gn, rn = torch.isnan(got.float()), torch.isnan(ref.float())
    assert torch.equal(gn, rn)
    g, r = got.view(torch.int16), ref.view(torch.int16)
    assert torch.equal(g[~gn], r[~rn])


@pytest.mark.parametrize("op", ["relu", "abs", "neg"])
def test_unary_edges_bit_exact_with_torch(op):
    x = _edge_tensor()
    got = _run(X.Unary(op, X.Leaf(0, B16), B16), {0: x.cuda()}, x.shape)
    ref = {"relu": torch.relu, "abs": torch.abs, "neg": torch.neg}[op](x)
    _same(got, ref)
    if op == "relu":  # -0 kept, as torch's scalar and vectorised paths both do
        assert int(got[0, 0].view(torch.int16)) & 0xffff == 0x8000


@pytest.mark.parametrize("op", ["add", "mul", "max", "min"])
def test_binary_edges_match_torch_up_to_nan_and_zero_order(op):
    a = _edge_tensor()
    b = torch.flip(a, [1]).contiguous()
    got = _run(X.Binary(op, X.Leaf(0, B16), X.Leaf(1, B16), B16), {0: a.cuda(), 1: b.cuda()},
               a.shape)
    ref = {"add": torch.add, "mul": torch.mul, "max": torch.maximum,
           "min": torch.minimum}[op](a, b)
    if op in ("max", "min"):
        # which zero of (+0, -0) comes out is torch-path-dependent: compare values
        both_zero = (a == 0) & (b == 0)
        got = torch.where(both_zero, torch.zeros_like(got), got)
        ref = torch.where(both_zero, torch.zeros_like(ref), ref)
    _same(got, ref)
