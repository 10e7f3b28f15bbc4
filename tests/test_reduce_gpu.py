"""ttl.math.reduce_sum / reduce_max on the MI355X (ttlh_reduce).

Kernel level: whole tt-lang kernels through the drop-in `ttl`, against the
oracle's eager executor running the same source (max: bit-exact; sum: within
1 bf16 ulp, the GPU accumulating in fp32 in its own order where the oracle
sums in float64).  C-ABI level, at 4096 x 4096: sums against float64 within
the fp32 accumulation bound (n * 2^-24 * sum |x s|, plus the output's own
rounding), maxima exact; the scalar-lane path (unaligned operand), size-1
inputs, the multi-split column path with its workspace, zero-padded result
tiles and repeatability.
"""

import pytest
import torch

import kernel_lib as KL
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from ttlhip import expr as X
from ttlhip import kernels as K

pytestmark = pytest.mark.gpu


def _scaler(v, dtype=torch.bfloat16):
    return torch.full((32, 32), v, dtype=dtype)


def _oracle(factory, tensors, out_index, **kw):
    ons = sim_exec.make_ttl()
    k = factory(ons, **kw)
    oargs = [sim_exec.OracleTensor(t.clone()) for t in tensors]
    k(*oargs)
    return oargs[out_index].t


def _gpu(factory, tensors, out_index, **kw):
    k = factory(ttl, **kw)
    args = [ttnn.from_torch(t) for t in tensors]
    k(*args)
    return ttnn.to_torch(args[out_index]), k


def _close(got, ref, kind):
    if kind == "max":
        assert torch.equal(got, ref)
    else:
        assert int(O.bf16_ulp_diff(got, ref).max()) <= 1


@pytest.mark.parametrize("kind", ["sum", "max"])
@pytest.mark.parametrize("out_w", [1, 32])
def test_row_reduce_kernel(kind, out_w):
    x = O.seeded((512, 512), "uniform", 21, lo=-2, hi=2)
    t = [x, _scaler(0.5), torch.zeros(512, out_w, dtype=torch.bfloat16)]
    got, k = _gpu(KL.make_reduce_rows, t, 2, kind=kind, gc=16)
    assert len(k.last_plan.launches) == 1
    _close(got, _oracle(KL.make_reduce_rows, t, 2, kind=kind, gc=16), kind)


@pytest.mark.parametrize("kind", ["sum", "max"])
def test_column_reduce_kernel(kind):
    x = O.seeded((512, 512), "uniform", 22, lo=-2, hi=2)
    t = [x, _scaler(-0.75), torch.zeros(32, 512, dtype=torch.bfloat16)]
    got, _ = _gpu(KL.make_reduce_cols, t, 2, kind=kind, gr=16)
    _close(got, _oracle(KL.make_reduce_cols, t, 2, kind=kind, gr=16), kind)


@pytest.mark.parametrize("kind", ["sum", "max"])
def test_full_reduce_of_fused_expression(kind):
    x = O.seeded((128, 128), "uniform", 23, lo=-1, hi=1)
    y = O.seeded((128, 128), "uniform", 24, lo=-1, hi=1)
    for ow in (1, 32):
        t = [x, y, _scaler(1.5), torch.zeros(ow, ow, dtype=torch.bfloat16)]
        got, _ = _gpu(KL.make_reduce_all, t, 3, kind=kind)
        _close(got, _oracle(KL.make_reduce_all, t, 3, kind=kind), kind)


def test_row_dot_and_accumulated_sum():
    a = O.seeded((256, 128), "uniform", 25, lo=-1, hi=1)
    b = O.seeded((256, 128), "uniform", 26, lo=-1, hi=1)
    t = [a, b, torch.zeros(256, 32, dtype=torch.bfloat16)]
    got, _ = _gpu(KL.make_row_dot, t, 2)
    _close(got, _oracle(KL.make_row_dot, t, 2), "sum")
    # several column blocks per row with store(acc=True): one fp32 sum per row
    x = O.seeded((256, 512), "uniform", 27, lo=-2, hi=2)
    got, _ = _gpu(KL.make_reduce_rows, [x, _scaler(1.0), torch.zeros(256, 1, dtype=torch.bfloat16)],
                  2, gc=2)
    exact = x.double().sum(1, keepdim=True)
    assert int(O.bf16_ulp_diff(got, exact.float().bfloat16()).max()) <= 1


# --- C ABI ---------------------------------------------------------------------


def _load_prog(dtype=torch.bfloat16):
    return X.compile_expr(X.Leaf(0, dtype))


def _reduce(x, kind, dims, out_shape, out_dtype=torch.float32, scaler=None, scale=1.0,
            out_pad=False):
    out = torch.full(out_shape, 7.0, dtype=out_dtype, device="cuda")
    K.reduce(_load_prog(x.dtype), [K.OperandMap(x)], kind, dims, out, (0, 0) + tuple(x.shape),
             out_pad=out_pad, scaler=scaler, scale=scale)
    torch.cuda.synchronize()
    return out.cpu()


def _fp32_sum_bound(xs: torch.Tensor, dim) -> torch.Tensor:
    n = xs.shape[dim] if dim is not None else xs.numel()
    a = xs.abs().sum(dim) if dim is not None else xs.abs().sum()
    return n * 2.0 ** -24 * a + 1e-30


@pytest.mark.parametrize("dims", [[1], [0], [0, 1]])
def test_abi_sum_4096(dims):
    x = O.seeded((4096, 4096), "normal", 31).cuda()
    s = torch.tensor([[0.5]], dtype=torch.float32, device="cuda")
    shape = {(1,): (4096, 1), (0,): (1, 4096), (0, 1): (1, 1)}[tuple(dims)]
    got = _reduce(x, "sum", dims, shape, scaler=s).double()
    xs = x.cpu().double() * 0.5
    d = None if dims == [0, 1] else dims[0]
    exact = xs.sum() if d is None else xs.sum(d)
    err = (got.reshape(-1) - exact.reshape(-1)).abs()
    assert bool((err <= _fp32_sum_bound(xs, d).reshape(-1)).all())


@pytest.mark.parametrize("dims", [[1], [0], [0, 1]])
def test_abi_max_4096_exact(dims):
    x = O.seeded((4096, 4096), "normal", 32).cuda()
    shape = {(1,): (4096, 1), (0,): (1, 4096), (0, 1): (1, 1)}[tuple(dims)]
    got = _reduce(x, "max", dims, shape, scale=-0.5)
    xs = x.cpu().float() * -0.5
    exact = xs.amax() if dims == [0, 1] else xs.amax(dims[0])
    assert torch.equal(got.reshape(-1), exact.reshape(-1))


def test_abi_bf16_output_rounds_once():
    x = O.seeded((1024, 2048), "uniform", 33, lo=-1, hi=1).cuda()
    got = _reduce(x, "sum", [1], (1024, 1), out_dtype=torch.bfloat16)
    exact = x.cpu().double().sum(1, keepdim=True)
    assert int(O.bf16_ulp_diff(got, exact.float().bfloat16()).max()) <= 1


def test_abi_padded_result_tiles():
    x = O.seeded((256, 256), "uniform", 34).cuda()
    rows = _reduce(x, "max", [1], (256, 32), out_pad=True)
    assert torch.equal(rows[:, 0], x.cpu().float().amax(1)) and not rows[:, 1:].any()
    cols = _reduce(x, "max", [0], (32, 256), out_pad=True)
    assert torch.equal(cols[0], x.cpu().float().amax(0)) and not cols[1:].any()
    one = _reduce(x, "max", [0, 1], (32, 32), out_pad=True)
    assert float(one[0, 0]) == float(x.max()) and torch.count_nonzero(one) == 1


def test_abi_unaligned_operand_scalar_path():
    # a row pitch that is not a multiple of 16 bytes forces one element per lane
    base = O.seeded((512, 520), "uniform", 35).cuda()
    x = base[:, :512]
    assert x.stride(0) == 520
    got = _reduce(x, "max", [1], (512, 1))
    assert torch.equal(got.reshape(-1), x.cpu().float().amax(1))
    got = _reduce(x, "max", [0], (1, 512))
    assert torch.equal(got.reshape(-1), x.cpu().float().amax(0))


def test_abi_size_one_dimensions():
    col = O.seeded((4096, 1), "uniform", 36).cuda()  # reduce a column vector over its rows
    got = _reduce(col, "max", [0], (1, 1))
    assert float(got) == float(col.max())
    row = O.seeded((1, 4096), "uniform", 37).cuda()
    got = _reduce(row, "sum", [1], (1, 1)).double()
    exact = row.cpu().double().sum()
    assert abs(float(got) - float(exact)) <= float(_fp32_sum_bound(row.cpu().double(), None))


@pytest.mark.parametrize("h", [16, 48, 4096])
def test_abi_column_splits(h):
    # h = 16: one split (no workspace); 48 and 4096: partials in the workspace
    x = O.seeded((h, 1024), "normal", 38).cuda()
    got = _reduce(x, "sum", [0], (1, 1024)).double().reshape(-1)
    xs = x.cpu().double()
    assert bool(((got - xs.sum(0)).abs() <= _fp32_sum_bound(xs, 0)).all())


def test_abi_cached_workspace_grows_and_follows_the_stream():
    # column and full reductions keep one workspace per (device, stream),
    # grown to the largest size asked for: a small call, a larger one (the
    # buffer is replaced), calls on a side stream (its own buffer) and after a
    # release all give the bits a first call on a fresh cache gives
    K.release_workspaces()
    small = O.seeded((48, 512), "normal", 41).cuda()
    large = O.seeded((4096, 2048), "normal", 42).cuda()
    want_small = _reduce(small, "sum", [0], (1, 512))
    want_large = _reduce(large, "sum", [0], (1, 2048))
    want_all = _reduce(large, "sum", [0, 1], (1, 1))
    K.release_workspaces()
    assert torch.equal(_reduce(small, "sum", [0], (1, 512)), want_small)
    assert torch.equal(_reduce(large, "sum", [0], (1, 2048)), want_large)
    assert torch.equal(_reduce(small, "sum", [0], (1, 512)), want_small)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    outs = []
    with torch.cuda.stream(side):
        for x, n in ((large, 2048), (small, 512), (large, 2048)):
            o = torch.full((1, n), 7.0, dtype=torch.float32, device="cuda")
            K.reduce(_load_prog(), [K.OperandMap(x)], "sum", [0], o, (0, 0) + tuple(x.shape),
                     stream=side)
            outs.append(o)
        a = torch.full((1, 1), 7.0, dtype=torch.float32, device="cuda")
        K.reduce(_load_prog(), [K.OperandMap(large)], "sum", [0, 1], a, (0, 0, 4096, 2048),
                 stream=side)
    side.synchronize()
    assert torch.equal(outs[0].cpu(), want_large) and torch.equal(outs[2].cpu(), want_large)
    assert torch.equal(outs[1].cpu(), want_small) and torch.equal(a.cpu(), want_all)
    K.release_workspaces()


def test_abi_repeatable_and_nan():
    x = O.seeded((2048, 2048), "normal", 39).cuda()
    a = _reduce(x, "sum", [0, 1], (1, 1))
    b = _reduce(x, "sum", [0, 1], (1, 1))
    assert torch.equal(a, b)  # fixed summation order
    x[100, 7] = float("nan")
    got = _reduce(x, "max", [1], (2048, 1)).reshape(-1)
    assert torch.isnan(got[100]) and not torch.isnan(torch.cat([got[:100], got[101:]])).any()


def test_abi_rejects_bad_arguments():
    x = torch.zeros(64, 64, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros(64, 1, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="kind"):
        K.reduce(_load_prog(), [K.OperandMap(x)], "mean", [1], out, (0, 0, 64, 64))
    with pytest.raises(ValueError, match="outside output"):
        K.reduce(_load_prog(), [K.OperandMap(x)], "sum", [0], out, (0, 0, 64, 64))
    with pytest.raises(ValueError, match="out of range"):
        K.reduce(_load_prog(), [K.OperandMap(x)], "sum", [1], out, (0, 32, 64, 64))


@pytest.mark.parametrize("at", [(3, 5), (0, 4), (31, 31)])
def test_abi_bf16_scaler_either_half_of_its_dword(at):
    # the scaler element is read through the aligned 32-bit word holding it:
    # odd columns sit in the upper half, even ones in the lower
    x = O.seeded((256, 4096), "uniform", 40, lo=-1, hi=1).cuda()
    tile = torch.zeros(32, 32, dtype=torch.bfloat16)
    tile[at] = -0.375
    tile[at[0], at[1] ^ 1] = 8.0  # the other half of the word
    sc = tile.cuda()[at[0]:at[0] + 1, at[1]:at[1] + 1]
    got = _reduce(x, "sum", [1], (256, 1), scaler=sc).double().reshape(-1)
    xs = x.cpu().double() * -0.375
    assert bool(((got - xs.sum(1)).abs() <= _fp32_sum_bound(xs, 1)).all())
    got = _reduce(x, "max", [1], (256, 1), scaler=sc).reshape(-1)
    assert torch.equal(got, (x.cpu().float() * -0.375).amax(1))


def test_abi_wide_rows_of_a_broadcast_operand():
    # every iteration row reads row 0 of the operand (row mask 0): cached
    # loads, and every result equals row 0's sum
    x = O.seeded((1, 4096), "normal", 41).cuda()
    out = torch.full((64, 1), 7.0, dtype=torch.float32, device="cuda")
    K.reduce(_load_prog(), [K.OperandMap(x, row_mask=0)], "sum", [1], out, (0, 0, 64, 4096))
    torch.cuda.synchronize()
    xs = x.cpu().double()
    exact = xs.sum()
    bound = float(_fp32_sum_bound(xs, None))
    assert bool(((out.cpu().double().reshape(-1) - exact).abs() <= bound).all())
    assert bool((out == out[0]).all())
