"""ttlh_reduce_rows_eltwise on the MI355X: row reductions and the elementwise
program reading their results in one launch must leave every output (the
program's and each reduction's result tiles) bit for bit as the separate
ttlh_reduce and ttlh_eltwise calls leave them, which tests/test_reduce_gpu.py
and tests/test_eltwise_gpu.py check against the oracle.  Forms: softmax
(reduce_max, reduce_sum of exp(x - m), exp(x - m) / sum; python/sim-style
per-op bf16 rounding), row centring with a scaled sum, and an RMS-style
normalisation with a row-vector operand read from memory.  Widths cover both
launch layouts (a wave per row below 2048 columns, a workgroup per row from
2048), ragged chunk and row counts and f32 operands and results (read from
memory at each use); refusals must leave nothing launched.
"""

import pytest
import torch

from oracle import tile_ops as O
from ttlhip import expr as X
from ttlhip import kernels as Kn

pytestmark = pytest.mark.gpu

B16 = torch.bfloat16


def _leaf(m):
    return X.Leaf(m, m.tensor.dtype)


def _ops(prog):
    return [s.leaf.ref if s.leaf is not None else None for s in prog.steps]


def _row_result(t):  # a reduction's result read as its row's value (column 0)
    return Kn.OperandMap(t, col_mask=0)


def _case(form, h, w, seed):
    x = O.seeded((h, w), "uniform", seed, lo=-4, hi=4).cuda()
    xm = Kn.OperandMap(x)
    t1 = torch.full((h, 32), 5.0, dtype=B16, device="cuda")
    t2 = torch.full((h, 32), 5.0, dtype=B16, device="cuda")
    scaler = torch.full((1, 1), 1.0, dtype=B16, device="cuda")
    if form == "softmax":
        p1 = X.compile_expr(_leaf(xm))
        e = X.Unary("exp", X.Binary("sub", _leaf(xm), _leaf(_row_result(t1)), B16), B16)
        p2 = X.compile_expr(e)
        e2 = X.Unary("exp", X.Binary("sub", _leaf(xm), _leaf(_row_result(t1)), B16), B16)
        fin = X.compile_expr(X.Binary("mul", e2, X.Unary("recip", _leaf(_row_result(t2)), B16),
                                      B16))
        reds = [Kn.RowReduce(p1, _ops(p1), "max", t1, (0, 0), True, scaler),
                Kn.RowReduce(p2, _ops(p2), "sum", t2, (0, 0), True, scaler)]
    elif form == "center":
        p1 = X.compile_expr(_leaf(xm))
        fin = X.compile_expr(X.Binary("sub", _leaf(xm),
                                      X.Binary("mul", _leaf(_row_result(t1)), X.Const(1.0 / w),
                                               B16), B16))
        reds = [Kn.RowReduce(p1, _ops(p1), "sum", t1, (0, 0), True, None, 0.5)]
    elif form == "rms":  # x * rsqrt(mean(x * x) + eps) * g, g a row vector read from memory
        g = O.seeded((1, w), "uniform", seed + 1, lo=0.5, hi=1.5).cuda()
        p1 = X.compile_expr(X.Binary("mul", _leaf(xm), _leaf(xm), B16))
        ms = X.Binary("add", _leaf(_row_result(t1)), X.Const(1e-3), B16)
        fin = X.compile_expr(X.Binary("mul", X.Binary("mul", _leaf(xm), X.Unary("rsqrt", ms, B16),
                                                      B16), _leaf(Kn.OperandMap(g)), B16))
        reds = [Kn.RowReduce(p1, _ops(p1), "sum", t1, (0, 0), True, None, 1.0 / w)]
    else:  # rms_plain: x * rsqrt(mean(x * x) + eps), an f32 result tile
        t1 = torch.full((h, 32), 5.0, dtype=torch.float32, device="cuda")
        p1 = X.compile_expr(X.Binary("mul", _leaf(xm), _leaf(xm), B16))
        ms = X.Binary("add", _leaf(_row_result(t1)), X.Const(1e-5), torch.float32)
        fin = X.compile_expr(X.Binary("mul", _leaf(xm), X.Unary("rsqrt", ms, torch.float32),
                                      torch.float32))
        reds = [Kn.RowReduce(p1, _ops(p1), "sum", t1, (0, 0), True, scaler, 1.0 / w)]
    out = torch.full((h, w), 7.0, dtype=B16, device="cuda")
    return reds, fin, out, [r.out for r in reds]


def _separate(reds, fin, out):
    h, w = out.shape
    for r in reds:
        Kn.reduce(r.prog, r.operands, r.kind, [1], r.out, (0, 0, h, w), r.out_origin, r.out_pad,
                  r.scaler, r.scale)
    Kn.eltwise(fin, _ops(fin), out, region=(0, 0, h, w))


def _bits(t):
    return t.view(torch.int16).cpu()


@pytest.mark.parametrize("form", ["softmax", "center", "rms", "rms_plain"])
@pytest.mark.parametrize("w", [128, 1056, 2048, 4096, 6144, 8192])
def test_one_launch_equals_separate_calls(form, w):
    print(f"reduce_rows_eltwise {form} w={w}", flush=True)
    h = 96
    reds, fin, out, temps = _case(form, h, w, seed=w + len(form))
    assert Kn.reduce_rows_eltwise(reds, fin, _ops(fin), out, (0, 0, h, w))
    torch.cuda.synchronize()
    fused = [_bits(out)] + [_bits(t) for t in temps]
    reds2, fin2, out2, temps2 = _case(form, h, w, seed=w + len(form))
    _separate(reds2, fin2, out2)
    torch.cuda.synchronize()
    sep = [_bits(out2)] + [_bits(t) for t in temps2]
    for a, b in zip(fused, sep):
        assert torch.equal(a, b), int((a != b).sum())
    if form == "softmax":  # and it is a softmax of x
        x = O.seeded((h, w), "uniform", w + len(form), lo=-4, hi=4).double()
        ex = torch.softmax(x, 1)
        got = out.double().cpu()
        assert float((got - ex).abs().max()) <= 2 ** -6 * float(ex.max())


@pytest.mark.parametrize("kind", ["sum", "max"])
@pytest.mark.parametrize("h,w", [(96, 2048), (33, 4096), (7, 6152), (64, 8192)])
@pytest.mark.parametrize("out_dtype", [B16, torch.float32])
def test_row_dot_alone_equals_fused(kind, h, w, out_dtype):
    # a row reduction of a * b (two bf16 operands) alone takes the bf16 row
    # kernel's product variant; inside one launch with a program it takes the
    # fused row kernel: the results must be the same bits, with a scale, a
    # scaler, NaN and infinite products included
    print(f"row dot {kind} {h}x{w} {out_dtype}", flush=True)
    a = O.seeded((h, w), "uniform", w + h, lo=-3, hi=3)
    b = O.seeded((h, w), "uniform", w + h + 1, lo=-3, hi=3)
    a[1, 5] = float("nan")
    b[2, 9] = float("inf")
    a, b = a.cuda(), b.cuda()
    am, bm = Kn.OperandMap(a), Kn.OperandMap(b)
    prog = X.compile_expr(X.Binary("mul", _leaf(am), _leaf(bm), B16))
    assert len(prog.steps) == 2
    scaler = torch.full((1, 1), 0.75, dtype=B16, device="cuda")

    def red(out):
        return Kn.RowReduce(prog, _ops(prog), kind, out, (0, 0), True, scaler, 0.5)

    t_alone = torch.full((h, 32), 5.0, dtype=out_dtype, device="cuda")
    r = red(t_alone)
    Kn.reduce(r.prog, r.operands, r.kind, [1], r.out, (0, 0, h, w), r.out_origin, r.out_pad,
              r.scaler, r.scale)
    t_fused = torch.full((h, 32), 5.0, dtype=out_dtype, device="cuda")
    fin = X.compile_expr(X.Binary("sub", _leaf(am), _leaf(_row_result(t_fused)), B16))
    out = torch.full((h, w), 7.0, dtype=B16, device="cuda")
    assert Kn.reduce_rows_eltwise([red(t_fused)], fin, _ops(fin), out, (0, 0, h, w))
    torch.cuda.synchronize()
    va, vf = t_alone.cpu(), t_fused.cpu()
    assert torch.equal(va.view(torch.int32 if out_dtype == torch.float32 else torch.int16),
                       vf.view(torch.int32 if out_dtype == torch.float32 else torch.int16))
    # and the values are the reduction of the bf16-rounded products
    prod = (a.cpu().float() * b.cpu().float()).bfloat16().double() * 0.375
    ref = prod.sum(1) if kind == "sum" else prod.amax(1)
    got = va[:, 0].double()
    fin_rows = torch.isfinite(ref)
    assert bool(torch.isnan(got[1])) and bool(torch.isnan(ref[1]))  # a NaN product
    same = (got == ref) | (torch.isnan(got) & torch.isnan(ref))
    assert bool(same[~fin_rows].all())  # infinite / NaN rows: the same value
    prod = torch.nan_to_num(prod, nan=0.0, posinf=0.0, neginf=0.0)
    tol = 2 ** -7 * prod.abs().sum(1) + 1e-6 if kind == "sum" else 2 ** -8 * ref.abs()
    if out_dtype == torch.float32 and kind == "sum":
        tol = w * 2.0 ** -24 * prod.abs().sum(1) + 1e-6
    assert bool(((got - ref).abs()[fin_rows] <= tol[fin_rows]).all())
    assert not bool(va[:, 1:].any())  # zero-padded result tiles


def test_region_offset_and_in_place_output():
    print("reduce_rows_eltwise region offset, in place", flush=True)
    big = O.seeded((160, 4096 + 64), "uniform", 3, lo=-3, hi=3).cuda()
    ref = big.clone()
    y0, x0, h, w = 32, 64, 96, 4096
    xm = Kn.OperandMap(big)
    t = torch.zeros(200, 64, dtype=B16, device="cuda")
    p1 = X.compile_expr(_leaf(xm))
    rm = Kn.OperandMap(t, col_mask=0, row_off=-y0 + 8, col_off=16)  # result rows from (8, 16)
    fin = X.compile_expr(X.Binary("sub", _leaf(xm), _leaf(rm), B16))
    red = Kn.RowReduce(p1, _ops(p1), "max", t, (8, 16), False, None, 1.0)
    assert Kn.reduce_rows_eltwise([red], fin, _ops(fin), big, (y0, x0, h, w))  # in place
    torch.cuda.synchronize()
    t2 = torch.zeros(200, 64, dtype=B16, device="cuda")
    rm2 = Kn.OperandMap(t2, col_mask=0, row_off=-y0 + 8, col_off=16)
    xm2 = Kn.OperandMap(ref)
    p1b = X.compile_expr(_leaf(xm2))
    fin2 = X.compile_expr(X.Binary("sub", _leaf(xm2), _leaf(rm2), B16))
    Kn.reduce(p1b, _ops(p1b), "max", [1], t2, (y0, x0, h, w), (8, 16), False, None, 1.0)
    Kn.eltwise(fin2, _ops(fin2), ref, region=(y0, x0, h, w))
    torch.cuda.synchronize()
    assert torch.equal(_bits(big), _bits(ref))
    assert torch.equal(_bits(t), _bits(t2))


def test_refusals_launch_nothing():
    print("reduce_rows_eltwise refusals", flush=True)
    h, w = 64, 4096
    reds, fin, out, temps = _case("softmax", h, w, seed=9)
    before = _bits(out)
    # a row wider than the fused kernel holds
    wide = torch.zeros(h, 16384, dtype=B16, device="cuda")
    wm = Kn.OperandMap(wide)
    p = X.compile_expr(_leaf(wm))
    r = Kn.RowReduce(p, _ops(p), "sum", temps[0], (0, 0), True, None)
    fw = X.compile_expr(X.Binary("add", _leaf(wm), _leaf(_row_result(temps[0])), B16))
    assert not Kn.reduce_rows_eltwise([r], fw, _ops(fw), wide, (0, 0, h, 16384))
    # a later stage reading a reduction's result other than as its row's value
    xm = reds[0].operands[0]
    bad = X.compile_expr(X.Binary("add", _leaf(xm), _leaf(Kn.OperandMap(temps[0], col_mask=31)),
                                  B16))
    assert not Kn.reduce_rows_eltwise(reds[:1], bad, _ops(bad), out, (0, 0, h, w))
    # an op outside the fused set
    lg = X.compile_expr(X.Unary("log", _leaf(xm), B16))
    assert not Kn.reduce_rows_eltwise(reds[:1], lg, _ops(lg), out, (0, 0, h, w))
    torch.cuda.synchronize()
    assert torch.equal(_bits(out), before)


@pytest.mark.parametrize("h,w", [(37, 512), (5, 2048), (33, 3000)])
def test_ragged_rows_and_fp32_operands(h, w):
    # f32 x (read from memory at each use, not held in registers), an f32
    # result for the maximum, a bf16 one for the sum; h not a multiple of the
    # four rows a workgroup takes below 2048 columns; 3000 columns leave the
    # last chunk of some lanes past the row's end
    print(f"reduce_rows_eltwise ragged h={h} w={w}", flush=True)
    if w % 8:
        pytest.skip("chunks of 8 columns")

    def case():
        x = O.seeded((h, w), "uniform", h + w, lo=-3, hi=3).float().cuda()
        g = O.seeded((1, w), "uniform", h + w + 1, lo=0.5, hi=1.5).cuda()
        xm, gm = Kn.OperandMap(x), Kn.OperandMap(g)
        t1 = torch.full((h, 32), 5.0, dtype=torch.float32, device="cuda")
        t2 = torch.full((h, 32), 5.0, dtype=B16, device="cuda")
        p1 = X.compile_expr(X.Binary("mul", _leaf(xm), _leaf(gm), torch.float32))
        p2 = X.compile_expr(X.Unary("exp", X.Binary("sub", _leaf(xm), _leaf(_row_result(t1)),
                                                    torch.float32), B16))
        fin = X.compile_expr(X.Binary("div", X.Binary("sub", _leaf(xm), _leaf(_row_result(t1)),
                                                      B16), _leaf(_row_result(t2)), B16))
        reds = [Kn.RowReduce(p1, _ops(p1), "max", t1, (0, 0), True, None, 0.5),
                Kn.RowReduce(p2, _ops(p2), "sum", t2, (0, 0), True)]
        return reds, fin, torch.full((h, w), 7.0, dtype=B16, device="cuda"), [t1, t2]

    reds, fin, out, temps = case()
    if w > 8192 or not Kn.reduce_rows_eltwise(reds, fin, _ops(fin), out, (0, 0, h, w)):
        pytest.fail("the fused launch refused a chain program")
    torch.cuda.synchronize()
    reds2, fin2, out2, temps2 = case()
    _separate(reds2, fin2, out2)
    torch.cuda.synchronize()
    for a, b in zip([out] + temps, [out2] + temps2):
        ai = a.view(torch.int16 if a.dtype == B16 else torch.int32).cpu()
        bi = b.view(torch.int16 if b.dtype == B16 else torch.int32).cpu()
        assert torch.equal(ai, bi), int((ai != bi).sum())


@pytest.mark.parametrize("form", ["recip", "div"])
@pytest.mark.parametrize("w", [512, 4096])
def test_softmax_flags_f32_results_scalers_and_specials(form, w):
    # the row softmax's dedicated kernel with f32 reduction results, scalers
    # other than 1, the e / l form as well as e * recip(l), and rows holding
    # NaN, +inf and -inf: bit for bit as the separate calls
    print(f"reduce_rows_eltwise softmax flags {form} w={w}", flush=True)
    h = 64

    def case():
        x = O.seeded((h, w), "uniform", w + 3, lo=-4, hi=4)
        x[3, 5] = float("nan")
        x[7, 9] = float("inf")
        x[11, :] = -float("inf")
        x = x.cuda()
        xm = Kn.OperandMap(x)
        t1 = torch.full((h, 32), 5.0, dtype=torch.float32, device="cuda")
        t2 = torch.full((h, 32), 5.0, dtype=torch.float32, device="cuda")
        s0 = torch.full((1, 1), 0.5, dtype=B16, device="cuda")
        p1 = X.compile_expr(_leaf(xm))
        p2 = X.compile_expr(X.Unary("exp", X.Binary("sub", _leaf(xm), _leaf(_row_result(t1)),
                                                    torch.float32), B16))
        e2 = X.Unary("exp", X.Binary("sub", _leaf(xm), _leaf(_row_result(t1)), torch.float32),
                     B16)
        if form == "recip":
            fin = X.compile_expr(X.Binary("mul", e2, X.Unary("recip", _leaf(_row_result(t2)),
                                                             torch.float32), B16))
        else:
            fin = X.compile_expr(X.Binary("div", e2, _leaf(_row_result(t2)), B16))
        reds = [Kn.RowReduce(p1, _ops(p1), "max", t1, (0, 0), True, s0, 2.0),
                Kn.RowReduce(p2, _ops(p2), "sum", t2, (0, 0), True, None, 0.25)]
        return reds, fin, torch.full((h, w), 7.0, dtype=B16, device="cuda"), [t1, t2]

    reds, fin, out, temps = case()
    assert Kn.reduce_rows_eltwise(reds, fin, _ops(fin), out, (0, 0, h, w))
    torch.cuda.synchronize()
    reds2, fin2, out2, temps2 = case()
    _separate(reds2, fin2, out2)
    torch.cuda.synchronize()
    for a, b in zip([out] + temps, [out2] + temps2):
        ai = a.view(torch.int16 if a.dtype == B16 else torch.int32).cpu()
        bi = b.view(torch.int16 if b.dtype == B16 else torch.int32).cpu()
        assert torch.equal(ai, bi), int((ai != bi).sum())
