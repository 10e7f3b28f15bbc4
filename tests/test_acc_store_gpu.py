"""store(expr, acc=True) on the MI355X (the CPU twin, tests/test_acc_store.py,
states the semantics: round 0 stores expr, round r > 0 stores block + expr,
each rounded to the block's dtype, python/sim/block.py:850-864).

Inputs are small integers, so every product is exact in fp32 and the whole
computation has one correct bf16 result: the GPU must match the oracle's
execution of the same kernel bit for bit at test sizes, and the sequential
closed form (torch, float64 products, bf16 rounding after every op) at a
size where the first round runs on the fused GEMM epilogue.
"""

import pytest
import torch

import kernel_lib as KL
import ttl
import ttnn
from ttlhip import plan as P
from test_acc_store import CASES, int_inputs, run_oracle

pytestmark = pytest.mark.gpu


def _gpu(form, bm, bk, bn, tensors):
    args = [ttnn.from_torch(t) for t in tensors]
    kern = KL.make_acc_expr(ttl, bm, bk, bn, form)
    kern(*args)
    torch.cuda.synchronize()
    return ttnn.to_torch(args[3]), kern


@pytest.mark.parametrize("case", CASES)
def test_acc_expression_on_gpu_bit_exact_with_oracle(case):
    form, bm, bk, bn, M, K, N = case
    print(f"acc store {case}", flush=True)
    a, b, c = int_inputs(bm, bk, bn, M, K, N, seed=bm + 3 * bk + 7 * bn)
    out = torch.zeros(M, N, dtype=torch.bfloat16)
    ref = run_oracle(form, bm, bk, bn, (a, b, c, out))
    got, _ = _gpu(form, bm, bk, bn, (a, b, c, out))
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_acc_expression_large_with_fused_first_round():
    bm, bk, bn = 4, 2, 4  # (4, 2) @ (2, 4): a block matmul (equal shapes pair tile-wise)
    M, K, N = 4096, 256, 3072  # 16 x 12 = 192 blocks of 256 x 256, 4 rounds
    print("acc store large", flush=True)
    a, b, c = int_inputs(bm, bk, bn, M, K, N, seed=5)
    got, kern = _gpu("mm_scale_bias", bm, bk, bn, (a, b, c, torch.zeros(M, N, dtype=torch.bfloat16)))
    kinds = [type(l) for l in kern.last_plan.launches]
    assert kinds[0] is P.FusedMatmulLaunch and len(kinds) == 4, kinds
    kw = bk * 32
    acc = None
    for k in range(K // kw):
        t = (a[:, k * kw:(k + 1) * kw].double() @ b[k * kw:(k + 1) * kw].double()).bfloat16()
        v = ((t * 0.5).bfloat16() + c).bfloat16()
        acc = v if acc is None else (acc + v).bfloat16()
    assert torch.equal(got.view(torch.int16), acc.view(torch.int16))
