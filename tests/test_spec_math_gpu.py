"""The spec's further ttl.math functions (TTLangSpecification.md:700-750) on
the MI355X through the drop-in `ttl`, against the oracle executor (the torch
functions the spec links, per tile in bf16): within 1 bf16 ulp (device libm
vs torch's CPU libm; "parity unpinned" at the last ulp, as for exp / log).
Also the C-ABI's fused softsign opcode (one rounding) and NaN propagation
through the out-of-line functions."""

import pytest
import torch

import kernel_lib as KL
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from spec_math_cases import CASES
from ttlhip import expr as X
from ttlhip import kernels as K

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", sorted(CASES))
def test_spec_math_kernel(name):
    params, (lo, hi) = CASES[name]
    x = O.seeded((512, 512), "uniform", 91, lo=lo, hi=hi)
    k = KL.make_unary_map(ttl, name, params, g=4)
    args = [ttnn.from_torch(x), ttnn.from_torch(torch.zeros(512, 512, dtype=torch.bfloat16))]
    k(*args)
    got = ttnn.to_torch(args[1])
    ko = KL.make_unary_map(sim_exec.make_ttl(), name, params, g=4)
    oargs = [sim_exec.OracleTensor(x.clone()), sim_exec.OracleTensor(torch.zeros_like(x))]
    ko(*oargs)
    assert int(O.bf16_ulp_diff(got, oargs[1].t).max()) <= 1, name


def _unary_abi(op, x, imm=0.0, imm2=0.0):
    e = X.Unary(op, X.Leaf(0, torch.bfloat16), torch.bfloat16, imm=imm, imm2=imm2)
    out = torch.empty_like(x)
    K.eltwise(X.compile_expr(e), [K.OperandMap(x), None], out)
    torch.cuda.synchronize()
    return out.cpu()


def test_fused_softsign_rounds_once():
    x = O.seeded((256, 256), "uniform", 92, lo=-6, hi=6)
    got = _unary_abi("softsign", x.cuda())
    ref = (x.float() / (1 + x.float().abs())).bfloat16()
    assert int(O.bf16_ulp_diff(got, ref).max()) <= 1


@pytest.mark.parametrize("op,imm,imm2", [("gelu", 0, 0), ("elu", 1.5, 0), ("selu", 1.05, 1.67),
                                         ("softplus", 2.0, 5.0), ("sin", 0, 0)])
def test_nan_propagates(op, imm, imm2):
    x = torch.full((32, 32), 0.5, dtype=torch.bfloat16)
    x[3, 7] = float("nan")
    got = _unary_abi(op, x.cuda(), imm, imm2)
    assert torch.isnan(got[3, 7]) and int(torch.isnan(got).sum()) == 1
