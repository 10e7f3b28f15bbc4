"""ttnn.bfloat8_b in the drop-in: packed-tile tensors (from_torch / to_torch /
typecast), tile matmuls with a bfloat8_b B operand planned onto the bf16 x
bfloat8_b GEMM, and the patterns that are refused with a clear error.

CPU tests: the packer is the library's host codec, checked against the
oracle's C restatement (pinned by brute force in test_bfp8.py); matmul plans
run on the CPU plan interpreter against float64 products of the oracle's
dequantisation.
"""

import pytest
import torch

import kernel_lib as KL
import plan_interp
import ttl
import ttnn
from oracle import bfp8 as OB
from oracle import tile_ops as O
from ttlhip import plan as P


def _w(rows, cols, seed, std=0.02):
    return O.seeded((rows, cols), "normal", seed, torch.float32, std=std)


def test_from_torch_packs_like_the_oracle_and_to_torch_is_float32():
    w = _w(96, 160, 1, std=1.0)
    t = ttnn.from_torch(w, dtype=ttnn.bfloat8_b, layout=ttnn.TILE_LAYOUT)
    assert t.dtype is ttnn.bfloat8_b and t.shape == (96, 160) and t.is_block_float
    assert torch.equal(t._tensor.cpu(), OB.pack_c(w))
    back = ttnn.to_torch(t)
    assert back.dtype == torch.float32
    assert torch.equal(back, OB.unpack_c(OB.pack_c(w), 96, 160).float())
    # typecast both ways
    assert torch.equal(ttnn.typecast(t, ttnn.bfloat16).to_torch(), back.bfloat16())
    assert torch.equal(ttnn.typecast(ttnn.from_torch(back), ttnn.bfloat8_b)._tensor.cpu(),
                       t._tensor.cpu())


def test_block_float_creation_and_indexing_rules():
    z = ttnn.zeros((64, 64), dtype=ttnn.bfloat8_b)
    assert torch.equal(z.to_torch(), torch.zeros(64, 64))
    with pytest.raises(ValueError, match="whole 32x32 tiles"):
        ttnn.from_torch(torch.zeros(40, 64), dtype=ttnn.bfloat8_b)
    with pytest.raises(TypeError, match="indexed by tiles only"):
        z[0:3]


@pytest.mark.parametrize("M,K,N", [(256, 256, 320), (64, 512, 96)])
def test_matmul_kernel_with_bfloat8_b_weights_plans_the_bfp8_gemm(M, K, N):
    a = O.seeded((M, K), "normal", 2)
    w = _w(K, N, 3)
    wq = ttnn.from_torch(w, dtype=ttnn.bfloat8_b)
    c = ttnn.Tensor(torch.zeros(M, N, dtype=torch.bfloat16))
    k = KL.make_matmul_multi(ttl, ttnn)
    args = [ttnn.Tensor(a.clone()), wq, c]
    plan = k.trace(*args)
    (l,) = plan.launches
    assert isinstance(l, P.MatmulLaunch) and l.b_block
    plan_interp.run(plan, {i: x for i, x in enumerate(args)})
    exact = (a.double() @ OB.unpack_c(OB.pack_c(w), K, N).double()).bfloat16()
    assert torch.equal(c._tensor, exact)


def test_block_float_refusals():
    wq = ttnn.from_torch(_w(64, 64, 4), dtype=ttnn.bfloat8_b)
    a = ttnn.Tensor(torch.zeros(64, 64, dtype=torch.bfloat16))
    out = ttnn.Tensor(torch.zeros(64, 64, dtype=torch.bfloat16))
    # elementwise use of a bfloat8_b tensor
    with pytest.raises(P.PlanError, match="elementwise operand"):
        KL.make_eltwise_add(ttl, granularity=2, grid=(1, 1)).trace(a, wq, out)
    # bfloat8_b as the A operand
    with pytest.raises(P.PlanError, match="B operand of a tile matmul only"):
        KL.make_matmul_single(ttl).trace(wq, a, out)
