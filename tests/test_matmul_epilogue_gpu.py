"""A tile or block matmul inside a larger store expression on the MI355X:
the plan's product launch (ttlh_matmul into a plan-owned tensor) and its
elementwise launch, against a float64 evaluation of the same program and
against the oracle's execution of the same kernel.

Bar (as for the CPU plan in test_matmul_epilogue.py): within 2^-7 max |exact|
of the float64 evaluation (product rounded to bf16 once, the other ops exact)
and no worse than the oracle's error plus 2^-9 max |exact|.
"""

import pytest
import torch

import kernel_lib as KL
import ttl
import ttnn
from oracle import tile_ops as O
from ttlhip import plan as P
from test_matmul_epilogue import (CASES, _two_products_kernel, exact, inputs, run_oracle,
                                  two_products_case)

pytestmark = pytest.mark.gpu


def _gpu(case, tensors, kern=None):
    bm, bk, bn, _, _, epi = case
    kern = kern or KL.make_matmul_epilogue(ttl, bm, bk, bn, epi)
    args = [ttnn.from_torch(t) for t in tensors]
    kern(*args)
    torch.cuda.synchronize()
    return ttnn.to_torch(args[3]), kern


def _check(case, seed=1, kern=None):
    a, b, c, out = inputs(*case, seed=seed)
    got, kern = _gpu(case, (a, b, c, out), kern)
    ex = exact(a, b, c, case[5])
    top = float(ex.abs().max())
    e_gpu = float((got.double() - ex).abs().max())
    e_orc = float((run_oracle(case, (a, b, c, out)).double() - ex).abs().max())
    assert e_gpu <= 2 ** -7 * top, e_gpu
    assert e_gpu <= e_orc + 2 ** -9 * top, (e_gpu, e_orc)
    return kern


@pytest.mark.parametrize("case", CASES + [(2, 8, 2, 8, 8, "relu_bias")])
def test_matmul_epilogue_on_gpu(case):
    kern = _check(case)
    (fl,) = kern.last_plan.launches
    assert isinstance(fl, P.FusedMatmulLaunch)


# Problems the fused entry point takes (>= 192 output blocks of 256 x 256):
# the executor runs one ttlh_matmul_eltwise launch for short programs
# (relu_bias, row_bias), the two launches otherwise (scale_exp).
# Either way the fused launch is bit-identical to the two launches (the same
# product rounding to bf16, the same program semantics), never stores the
# product (its plan-owned tensor is never allocated when it runs) and is
# within the bounds above against float64.
@pytest.mark.parametrize("epi,fused", [("relu_bias", True), ("row_bias", True),
                                       ("scale_exp", False)])
def test_fused_epilogue_equals_two_launches(epi, fused):
    from ttlhip import kernels as Kn
    print(f"fused epilogue {epi}", flush=True)
    bm, bk, bn = 4, 8, 4
    M, K, N = 4096, 256, 3072  # 16 x 12 = 192 blocks of 256 x 256
    a = O.seeded((M, K), "normal", 91)
    b = O.seeded((K, N), "normal", 92)
    c = O.seeded((1, N) if epi == "row_bias" else (M, N), "normal", 93)
    args = [ttnn.from_torch(t) for t in (a, b, c, torch.zeros(M, N, dtype=torch.bfloat16))]
    kern = KL.make_matmul_epilogue(ttl, bm, bk, bn, epi)
    kern(*args)
    (fl,) = kern.last_plan.launches
    assert isinstance(fl, P.FusedMatmulLaunch)
    assert Kn.matmul_eltwise_preferred(fl.ew.prog) == fused
    assert (fl.mm.c.obj._t is None) == fused, "the executor took the other form"
    got = ttnn.to_torch(args[3])
    forced = dict(enumerate(args[:3] + [ttnn.from_torch(torch.zeros(M, N, dtype=torch.bfloat16))]))
    assert P._execute_fused(fl, forced, None, Kn, force=True)
    two = dict(enumerate(args[:3] + [ttnn.from_torch(torch.zeros(M, N, dtype=torch.bfloat16))]))
    P._execute_one(fl.mm, two, None, Kn)
    P._execute_one(fl.ew, two, None, Kn)
    torch.cuda.synchronize()
    ref = ttnn.to_torch(two[3])
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(ttnn.to_torch(forced[3]).view(torch.int16), ref.view(torch.int16))
    ex = exact(a, b, c, epi)
    assert float((got.double() - ex).abs().max()) <= 2 ** -7 * float(ex.abs().max())


def test_matmul_epilogue_plan_reused_with_new_inputs():
    case = CASES[2]
    kern = _check(case, seed=5)
    _check(case, seed=9, kern=kern)
    assert len(kern._cache) == 1


def test_two_products_and_an_offset_product_on_gpu():
    tensors, ex = two_products_case()
    args = [ttnn.from_torch(t) for t in tensors]
    _two_products_kernel(ttl)(*args)
    torch.cuda.synchronize()
    got = ttnn.to_torch(args[2]).double()
    assert float((got - ex).abs().max()) <= 2 ** -7 * float(ex.abs().max())
