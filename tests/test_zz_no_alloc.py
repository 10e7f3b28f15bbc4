"""ttlh_reduce_noalloc, the allocation-free variant of ttlh_reduce, on the
MI355X through the C ABI: its results must equal ttlh_reduce's (same kernels,
same summation order, so bit-identical) on two calls in a row, the second on
a smaller input (the fixed scratch array keeps the first call's partials),
for column reductions (several row splits: partials in the scratch) and
full reductions (one partial per row), sums and maxima, a fused program and a
scaler.  It allocates nothing, and a reduction whose partials exceed the
scratch array is refused before any launch."""

import pytest
import torch

from oracle import tile_ops as O
from ttlhip import _lib as L
from ttlhip import expr as X
from ttlhip import kernels as K

pytestmark = pytest.mark.gpu

SCRATCH = 4 << 20  # TTLH_REDUCE_SCRATCH_BYTES


def _prog(fused, dtype):
    leaf = X.Leaf(0, dtype)
    if not fused:
        return X.compile_expr(leaf)
    e = X.Unary("exp", X.Binary("mul", leaf, X.Const(0.25), dtype), dtype)
    return X.compile_expr(e)


def _run(x, kind, dims, out_shape, noalloc, fused=False, scaler=None):
    prog = _prog(fused, x.dtype)
    ops = [K.OperandMap(x) if s.leaf is not None else None for s in prog.steps]
    out = torch.full(out_shape, 7.0, dtype=torch.float32, device="cuda")
    K.reduce(prog, ops, kind, dims, out, (0, 0) + tuple(x.shape), scaler=scaler, scale=0.5,
             noalloc=noalloc)
    return out


@pytest.mark.parametrize("kind", ["sum", "max"])
@pytest.mark.parametrize("dims", [[0], [0, 1]])
@pytest.mark.parametrize("fused", [False, True])
def test_noalloc_equals_workspace_entry_on_two_calls(kind, dims, fused):
    sc = torch.full((1, 1), 1.5, dtype=torch.bfloat16, device="cuda")
    for i, (h, w) in enumerate([(4096, 2048), (320, 96)]):  # second call smaller
        print(f"noalloc case kind={kind} dims={dims} fused={fused} shape={(h, w)}", flush=True)
        x = O.seeded((h, w), "uniform", 100 + i, lo=-2, hi=2).cuda()
        need = int(L.load().ttlh_reduce_workspace_bytes(
            (L.REDUCE_DIM0 if 0 in dims else 0) | (L.REDUCE_DIM1 if 1 in dims else 0), h, w))
        assert 0 < need <= SCRATCH  # the case goes through the scratch array
        shape = (1, w) if dims == [0] else (1, 1)
        ref = _run(x, kind, dims, shape, False, fused, sc)
        got = _run(x, kind, dims, shape, True, fused, sc)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), ref.cpu()), f"call {i}: noalloc differs from ttlh_reduce"


def test_noalloc_row_reduce_needs_no_scratch():
    x = O.seeded((256, 512), "uniform", 7, lo=-2, hi=2).cuda()
    ref = _run(x, "sum", [1], (256, 1), False)
    got = _run(x, "sum", [1], (256, 1), True)
    assert torch.equal(got.cpu(), ref.cpu())


def test_noalloc_allocates_nothing():
    """No allocation, by torch's caching allocator or by the library itself:
    after one warm-up call (which loads the code object and with it the
    file-scope scratch array), the device's free memory (hipMemGetInfo) does
    not move across a further call whose column partials need the scratch."""
    x = O.seeded((2048, 1024), "uniform", 8, lo=-2, hi=2).cuda()
    out = torch.zeros(1, 1024, dtype=torch.float32, device="cuda")
    prog = _prog(False, x.dtype)
    need = int(L.load().ttlh_reduce_workspace_bytes(L.REDUCE_DIM0, 2048, 1024))
    assert 0 < need <= SCRATCH  # the case goes through the scratch array
    K.reduce(prog, [K.OperandMap(x)], "sum", [0], out, (0, 0, 2048, 1024), noalloc=True)
    torch.cuda.synchronize()
    n0 = torch.cuda.memory_stats().get("allocation.all.allocated", 0)
    free0, _ = torch.cuda.mem_get_info()
    out.zero_()
    torch.cuda.synchronize()
    K.reduce(prog, [K.OperandMap(x)], "sum", [0], out, (0, 0, 2048, 1024), noalloc=True)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    n1 = torch.cuda.memory_stats().get("allocation.all.allocated", 0)
    assert n1 == n0, "torch's allocator was used"
    assert free1 == free0, f"device free memory moved by {free0 - free1} bytes"
    exact = x.double().sum(0, keepdim=True).float()
    assert float((out - exact).abs().max()) <= 2048 * 2 * 2 ** -23 * 4


def test_noalloc_refuses_a_reduction_beyond_the_scratch():
    # a full reduction keeps one fp32 partial per row: 2^20 + 32 rows need
    # more than 4 MiB; refused before anything is launched
    h = (SCRATCH // 4) + 32
    x = torch.zeros(h, 1, dtype=torch.bfloat16, device="cuda")
    out = torch.full((1, 1), 7.0, dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="fixed scratch"):
        K.reduce(_prog(False, x.dtype), [K.OperandMap(x)], "sum", [0, 1], out, (0, 0, h, 1),
                 noalloc=True)
    torch.cuda.synchronize()
    assert float(out[0, 0]) == 7.0
