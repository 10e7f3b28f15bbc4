"""The expression forms of tests/test_expr_forms.py on the MI355X through the
drop-in `ttl`: reductions inside one store (softmax and row centring, the
reductions planned into plan-owned tensors ahead of the elementwise launch)
and block matmuls of computed operands (the operand materialised in bf16
first).  Bars: within 2 bf16 ulps of the oracle's eager executor for the
reductions (fp32 sums in the kernel's order against the oracle's float64
sums, each then rounded to bf16) and within 2^-6 of exact softmax; matmuls
within 2^-7 max |exact| of the float64 evaluation (as the oracle is), and per
element within one bf16 rounding of the product and one of the result plus
the fp32 accumulation error (the oracle's block matmul also accumulates in
fp32, so its error here is below one rounding and is not the bar)."""

import pytest
import torch

import kernel_lib as KL
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from test_expr_forms import _mm_exact
from ttlhip import plan as P

pytestmark = pytest.mark.gpu


def _gpu_and_oracle(make, tensors, out_index, **kw):
    k = make(ttl, **kw)
    args = [ttnn.from_torch(t) for t in tensors]
    k(*args)
    got = ttnn.to_torch(args[out_index])
    ok = make(sim_exec.make_ttl(), **kw)
    oargs = [sim_exec.OracleTensor(t.clone()) for t in tensors]
    ok(*oargs)
    return got, oargs[out_index].t, k.last_plan


@pytest.mark.parametrize("form", ["softmax", "center", "rms"])
def test_reductions_inside_one_store_on_gpu(form):
    print(f"expr forms gpu: {form}", flush=True)
    x = O.seeded((512, 512), "uniform", 7, lo=-4, hi=4)
    t = [x, torch.ones(32, 32, dtype=torch.bfloat16), torch.zeros(512, 512, dtype=torch.bfloat16)]
    got, orc, plan = _gpu_and_oracle(KL.make_softmax_one_store, t, 2, gc=16, form=form)
    assert isinstance(plan.launches[0], P.ReduceEltwiseLaunch)
    ulp = O.bf16_ulp_diff(got, orc)
    assert int(ulp.max()) <= 2, int(ulp.max())
    if form == "softmax":
        ex = torch.softmax(x.double(), 1)
        assert float((got.double() - ex).abs().max()) <= 2 ** -6 * float(ex.max())


@pytest.mark.parametrize("form", ["scale", "relu_b", "both"])
def test_matmul_of_computed_operands_on_gpu(form):
    print(f"expr forms gpu: matmul {form}", flush=True)
    bm, bk, bn = 2, 4, 2
    M, K, N = bm * 32 * 4, bk * 32, bn * 32 * 4
    a, b, c = (O.seeded(s, "normal", 60 + i) for i, s in enumerate([(M, K), (K, N), (M, N)]))
    tensors = [a, b, c, torch.zeros(M, N, dtype=torch.bfloat16)]
    got, orc, plan = _gpu_and_oracle(KL.make_matmul_computed_operand, tensors, 3, bm=bm, bk=bk,
                                     bn=bn, form=form)
    ex = _mm_exact(a, b, c, form)
    top = float(ex.abs().max())
    e_gpu = float((got.double() - ex).abs().max())
    e_orc = float((orc.double() - ex).abs().max())
    assert e_gpu <= 2 ** -7 * top and e_orc <= 2 ** -7 * top, (e_gpu, e_orc)
    # per element: one bf16 rounding of the fp32-accumulated product (which
    # may fall on the other side of a rounding boundary than the float64 one)
    # and one of the result, plus the fp32 accumulation error
    r = lambda v: v.to(torch.bfloat16).double()
    A, B = a.double(), b.double()
    prod = {"scale": r(A * 0.25) @ B, "relu_b": A @ r(torch.relu(B)),
            "both": r(A + A) @ r(B * 2.0)}[form]
    bound = 2 ** -8 * (prod.abs() + ex.abs()) + 1e-6 * K ** 0.5 * float(prod.abs().max())
    err = (got.double() - ex).abs()
    assert bool((err <= bound).all()), float((err - bound).max())
