"""The spec's further ttl.math functions (TTLangSpecification.md:700-750) on
the CPU: traced + planned by the drop-in and run by the CPU plan
interpreter, bit-exact against the oracle executor (the torch functions the
spec links, one op per tile in the tile dtype).  Neither the reference
compiler's op table nor its simulator implements these, so against the
reference they are "parity unpinned"; the oracle is the linked torch
function.  The compositions (square, rsub, relu_max / relu_min, hardtanh,
leaky_relu, prelu) are checked against those torch functions directly: they
round once, like the fused functions."""

import pytest
import torch

import kernel_lib as KL
import plan_interp
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from spec_math_cases import CASES


@pytest.mark.parametrize("name", sorted(CASES))
def test_spec_math_plan_matches_oracle(name):
    params, (lo, hi) = CASES[name]
    x = O.seeded((256, 256), "uniform", 81, lo=lo, hi=hi)
    k = KL.make_unary_map(ttl, name, params)
    args = [ttnn.Tensor(x.clone()), ttnn.Tensor(torch.zeros(256, 256, dtype=torch.bfloat16))]
    plan = k.trace(*args)
    assert len(plan.launches) == 1
    plan_interp.run(plan, dict(enumerate(args)))
    ko = KL.make_unary_map(sim_exec.make_ttl(), name, params)
    oargs = [sim_exec.OracleTensor(x.clone()), sim_exec.OracleTensor(torch.zeros_like(x))]
    ko(*oargs)
    assert torch.equal(args[1]._tensor, oargs[1].t)


def test_oracle_gelu_is_the_mathematical_value():
    # closed form at points where erfc is known: gelu(0) = 0, gelu(x) -> x
    # for large x, and the x << 0 tail (x / 2 erfc(-x / sqrt 2) via math.erfc)
    import math
    x = torch.tensor([0.0, 6.0, -3.0, -5.0, -8.0]).bfloat16()
    got = O.UNARY["gelu"](x).double()
    for xi, gi in zip(x.double().tolist(), got.tolist()):
        exact = 0.5 * xi * math.erfc(-xi / math.sqrt(2.0))
        assert abs(gi - exact) <= abs(exact) * 2 ** -8 + 1e-45


def test_compositions_equal_torch_functions():
    F = torch.nn.functional
    x = O.seeded((256, 256), "uniform", 82, lo=-4, hi=4)
    ref = {
        "square": torch.square(x), "rsub": 3 - x, "relu_max": torch.clamp(x, 0, 2),
        "relu_min": torch.relu(torch.clamp(x, min=1)), "hardtanh": F.hardtanh(x, -1, 2),
        "leaky_relu": F.leaky_relu(x, 0.125), "prelu": F.leaky_relu(x, 0.25),
    }
    for name, r in ref.items():
        params = CASES[name][0]
        k = KL.make_unary_map(ttl, name, params)
        args = [ttnn.Tensor(x.clone()), ttnn.Tensor(torch.zeros_like(x))]
        plan_interp.run(k.trace(*args), dict(enumerate(args)))
        assert torch.equal(args[1]._tensor, r), name
