"""In-tile broadcast (operand masks ~31 and 0), intermediate CBs (scratch
tensors) and split store sites on the MI355X, against the oracle's eager
executor running the same kernel sources: bit-exact for + and *, within one
bf16 ulp where exp is involved.  C-ABI level at 4096 x 4096: every mask on
both axes, 8-wide and column-splat operands, against a torch gather."""

import pytest
import torch

import kernel_lib as KL
import ttl
import ttnn
from ttlhip import plan as P
from oracle import sim_exec, tile_ops as O
from ttlhip import expr as X
from ttlhip import kernels as K

pytestmark = pytest.mark.gpu


def _oracle(factory, tensors, out_index, **kw):
    k = factory(sim_exec.make_ttl(), **kw)
    args = [sim_exec.OracleTensor(t.clone()) for t in tensors]
    k(*args)
    return args[out_index].t


def _gpu(factory, tensors, out_index, **kw):
    k = factory(ttl, **kw)
    args = [ttnn.from_torch(t) for t in tensors]
    k(*args)
    return ttnn.to_torch(args[out_index]), k


def _close(got, ref, exact):
    if exact:
        assert torch.equal(got, ref)
    else:
        assert int(O.bf16_ulp_diff(got, ref).max()) <= 1


@pytest.mark.parametrize("dims", [[0], [1], [0, 1]])
@pytest.mark.parametrize("ib,expr", [((2, 2), "plain"), ((1, 1), "fma"), ((2, 1), "exp"),
                                     ((1, 2), "fma"), ((2, 2), "fma")])
def test_tile_bcast_kernel(dims, ib, expr):
    if (ib[0] == 1 and 0 not in dims) or (ib[1] == 1 and 1 not in dims):
        pytest.skip("a size-1 input block dim expands only along a broadcast dim")
    rows, cols = 8, 4
    x = O.seeded((rows * ib[0] * 32, cols * ib[1] * 32), "uniform", 11, lo=-2, hi=2)
    a = O.seeded((rows * 64, cols * 64), "uniform", 12, lo=-2, hi=2)
    out = torch.zeros(rows * 64, cols * 64, dtype=torch.bfloat16)
    kw = dict(dims=dims, ib=ib, ob=(2, 2), grid=(2, 2), expr=expr)
    got, _ = _gpu(KL.make_tile_bcast, [x, a, out], 2, **kw)
    _close(got, _oracle(KL.make_tile_bcast, [x, a, out], 2, **kw), expr != "exp")


def test_two_stage_intermediate_cb():
    x = O.seeded((512, 256), "uniform", 13, lo=-2, hi=2)
    y = O.seeded((512, 256), "uniform", 14, lo=0, hi=2)
    out = torch.zeros(512, 256, dtype=torch.bfloat16)
    got, k = _gpu(KL.make_two_stage, [x, y, out], 2)
    assert len(k.last_plan.launches) == 1  # stage 1 inlined into stage 2
    _close(got, _oracle(KL.make_two_stage, [x, y, out], 2), False)
    # a second call reuses the cached plan and its scratch tensor
    x2 = O.seeded((512, 256), "uniform", 15, lo=-2, hi=2)
    got2, _ = _gpu(KL.make_two_stage, [x2, y, out], 2)
    _close(got2, _oracle(KL.make_two_stage, [x2, y, out], 2), False)


def test_held_tile_parts():
    a = O.seeded((256, 256), "uniform", 16, lo=-2, hi=2)
    c = O.seeded((64, 64), "uniform", 17, lo=-2, hi=2)
    out = torch.zeros(256, 256, dtype=torch.bfloat16)
    got, k = _gpu(KL.make_held_tile, [a, c, out], 2)
    assert len(k.last_plan.launches) == 4
    _close(got, _oracle(KL.make_held_tile, [a, c, out], 2), True)


def _gather(t, n_out, mask, off):
    idx = torch.arange(n_out)
    return (idx & mask) + off if mask != -1 else idx + off


@pytest.mark.parametrize("rmask", [-1, ~31, 31, 0])
@pytest.mark.parametrize("cmask", [-1, ~31, 31, 0])
def test_abi_masks_4096(rmask, cmask):
    H = W = 4096
    src = O.seeded((H, W), "uniform", 18, lo=-4, hi=4).cuda()
    other = O.seeded((H, W), "uniform", 19, lo=-4, hi=4).cuda()
    roff = 64 if rmask in (31, 0) else 0
    coff = 96 if cmask in (31, 0) else 0
    prog = X.compile_expr(X.Binary("add", X.Leaf(0, torch.bfloat16), X.Leaf(1, torch.bfloat16),
                                   torch.bfloat16))
    out = torch.empty(H, W, dtype=torch.bfloat16, device="cuda")
    K.eltwise(prog, [K.OperandMap(src, rmask, cmask, roff, coff), K.OperandMap(other)], out)
    torch.cuda.synchronize()
    iy = _gather(src, H, rmask, roff).cuda()
    ix = _gather(src, W, cmask, coff).cuda()
    ref = (src[iy][:, ix].float() + other.float()).bfloat16()
    assert torch.equal(out, ref)


def test_abi_mask_region_offset_and_f32():
    # an interior region (y0, x0 not multiples of the tile) and an f32 operand
    src = O.seeded((1024, 1024), "uniform", 20, torch.float32).cuda()
    prog = X.compile_expr(X.Leaf(0, torch.float32))
    out = torch.zeros(1024, 1024, dtype=torch.float32, device="cuda")
    K.eltwise(prog, [K.OperandMap(src, ~31, 0, 0, 160)], out, region=(40, 8, 600, 512))
    torch.cuda.synchronize()
    ys = torch.arange(40, 640)
    ref = src[(ys & ~31).cuda()][:, 160:161].expand(600, 512)
    assert torch.equal(out[40:640, 8:520], ref)
    assert not out[:40].any() and not out[640:].any()


def test_long_chain_split_through_temporaries():
    a = O.seeded((512, 256), "uniform", 24, lo=-2, hi=2)
    b = O.seeded((512, 256), "uniform", 25, lo=-2, hi=2)
    c = O.seeded((512, 256), "uniform", 26, lo=-2, hi=2)
    out = torch.zeros(512, 256, dtype=torch.bfloat16)
    got, k = _gpu(KL.make_long_chain, [a, b, c, out], 3)
    assert len(k.last_plan.launches) >= 2
    # sigmoid / tanh run on the device's own math: within one bf16 ulp of the
    # oracle's torch per op, so compare the final values by ulps
    ref = _oracle(KL.make_long_chain, [a, b, c, out], 3)
    d = O.bf16_ulp_diff(got, ref)
    assert float((d > 2).float().mean()) < 1e-3 and int(d.max()) <= 64


def test_softmax_rows_through_intermediate_cbs():
    # 1024 rows of 16 tiles: reduce -> broadcast -> exp -> reduce -> scale on
    # the device: row max and row sum into scratch tensors, the exp stage
    # recomputed inside the sum and the final scale
    x = O.seeded((1024, 512), "uniform", 32, lo=-4, hi=4)
    s = torch.full((32, 32), 1.0, dtype=torch.bfloat16)
    out = torch.zeros(1024, 512, dtype=torch.bfloat16)
    got, k = _gpu(KL.make_softmax_rows, [x, s, out], 2, w=16, grid=(4, 4))
    # the exp stage is inlined into both readers; the two row reductions and
    # the scale run as one fused launch
    (l,) = k.last_plan.launches
    assert isinstance(l, P.ReduceEltwiseLaunch) and [r.kind for r in l.reds] == ["max", "sum"]
    ref = _oracle(KL.make_softmax_rows, [x, s, out], 2, w=16, grid=(4, 4))
    # the row maxima are exact; exp and the fp32 row sums (summed in another
    # order than the oracle's float64) may move a value by one bf16 ulp
    d = O.bf16_ulp_diff(got, ref)
    assert int(d.max()) <= 2 and float((d > 0).float().mean()) < 0.05
    assert float((got.float() - torch.softmax(x.float(), 1)).abs().max()) < 2e-3


@pytest.mark.parametrize("with_out", [False, True])
def test_broadcast_forms_on_full_tiles_gpu(with_out):
    # the simulator's form (no `out`: tiles added as they are) and the
    # compiler's form (with `out`: row 0 of each tile) on the device
    a = O.seeded((512, 256), "uniform", 51, lo=-2, hi=2)
    b = O.seeded((32, 256), "uniform", 52, lo=-2, hi=2)
    expect = a + (b[0:1, :].expand(512, 256) if with_out else b.repeat(16, 1))
    k = KL.make_row_bcast_forms(ttl, with_out, grid=(2, 2))
    args = [ttnn.from_torch(t) for t in (a, b, torch.zeros(512, 256, dtype=torch.bfloat16))]
    k(*args)
    assert len(k.last_plan.launches) == 1
    assert torch.equal(ttnn.to_torch(args[2]), expect)
