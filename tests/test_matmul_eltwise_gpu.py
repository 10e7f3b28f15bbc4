"""ttlh_matmul_eltwise, the GEMM with the store's elementwise program fused
into its epilogue, against the two launches it replaces (ttlh_matmul into a
bf16 tensor, then ttlh_eltwise over it): bit for bit, over every op the
epilogue runs, both operand orders, broadcast and tile-re-use operand maps,
intermediate f32 steps, NaN / inf operands, an output region inside a larger
tensor and block counts that do not divide the problem.  The two-launch form
is itself checked against the oracle (tests/test_eltwise_gpu.py,
tests/test_matmul_gpu.py); the semantics both follow are the simulator's
(python/sim/block.py:870-920: the product materialised in bf16, then the
elementwise ops with per-op rounding).

Refusals: problems below 192 output blocks, f32 outputs, programs that use
the stack, ops outside the epilogue's set: TTLH_EUNSUPPORTED before any
launch (the executor then runs the two launches).
"""

import pytest
import torch

from ttlhip import _lib as L
from ttlhip import kernels as Kn
from ttlhip.expr import StackProgram, Step

pytestmark = pytest.mark.gpu

B16, F32 = L.TTLH_BF16, L.TTLH_F32
OP = L.OP


def _operands(M, N, seed):
    g = torch.Generator().manual_seed(seed)
    c = torch.randn(M, N, generator=g).bfloat16()
    c[::97, ::89] = float("nan")
    c[5::101, 3::83] = float("inf")
    c[7::103, 1::79] = -float("inf")
    d = (torch.rand(M, N, generator=g) + 0.5).bfloat16()
    row = torch.randn(1, N, generator=g).bfloat16()
    col = torch.randn(M, 1, generator=g).bfloat16()
    tile = torch.randn(32, 32, generator=g).bfloat16()
    return {k: v.cuda() for k, v in dict(c=c, d=d, row=row, col=col, tile=tile).items()}


def _programs(t):
    c, d = Kn.OperandMap(t["c"]), Kn.OperandMap(t["d"])
    row, col = Kn.OperandMap(t["row"]), Kn.OperandMap(t["col"])
    tile = Kn.OperandMap(t["tile"], 31, 31)
    L0 = Step(L.FORM_LOAD)
    progs = {
        "identity": ([Step(L.FORM_LOAD, rnd=B16)], [None]),
        "x*0.125": ([L0, Step(L.FORM_BIN_IMM, OP["mul"], B16, 0.125)], [None, None]),
        "3-x": ([L0, Step(L.FORM_BIN_IMM_REV, OP["sub"], B16, 3.0)], [None, None]),
        "relu(x+c)": ([L0, Step(L.FORM_BIN, OP["add"], B16), Step(L.FORM_UNARY, OP["relu"], B16)],
                      [None, c, None]),
        "c-x": ([L0, Step(L.FORM_BIN_REV, OP["sub"], B16)], [None, c]),
        "d/x": ([L0, Step(L.FORM_BIN_REV, OP["div"], B16)], [None, d]),
        "x/d": ([L0, Step(L.FORM_BIN, OP["div"], B16)], [None, d]),
        "max(x,c)": ([L0, Step(L.FORM_BIN, OP["max"], B16)], [None, c]),
        "min(c,x)": ([L0, Step(L.FORM_BIN_REV, OP["min"], B16)], [None, c]),
        "x*row+col": ([L0, Step(L.FORM_BIN, OP["mul"], B16), Step(L.FORM_BIN, OP["add"], B16)],
                      [None, row, col]),
        "x-tile": ([L0, Step(L.FORM_BIN, OP["sub"], B16)], [None, tile]),
        "exp(x*s)*c": ([L0, Step(L.FORM_BIN_IMM, OP["mul"], F32, 0.125),
                        Step(L.FORM_UNARY, OP["exp"], B16), Step(L.FORM_BIN, OP["mul"], B16)],
                       [None, None, None, c]),
        "exp(4x)": ([L0, Step(L.FORM_BIN_IMM, OP["mul"], F32, 40.0),
                     Step(L.FORM_UNARY, OP["exp"], B16)], [None, None, None]),
        "sqrt|x|": ([L0, Step(L.FORM_UNARY, OP["abs"], F32), Step(L.FORM_UNARY, OP["sqrt"], B16)],
                    [None, None, None]),
        "rsqrt(x)": ([L0, Step(L.FORM_UNARY, OP["rsqrt"], B16)], [None, None]),
        "recip(-x)": ([L0, Step(L.FORM_UNARY, OP["neg"], F32), Step(L.FORM_UNARY, OP["recip"], B16)],
                      [None, None, None]),
        "(x+c)*d-row": ([L0, Step(L.FORM_BIN, OP["add"], F32), Step(L.FORM_BIN, OP["mul"], F32),
                         Step(L.FORM_BIN, OP["sub"], B16)], [None, c, d, row]),
        "c+x (product last)": ([Step(L.FORM_LOAD), Step(L.FORM_BIN, OP["add"], B16)], [c, None]),
    }
    return progs


def _bits(t):
    return t.view(torch.int16)


def _pair(a, b, prog, ops, prod_step, out_shape, region):
    """(fused, two-launch) outputs, both starting from the same filled tensor."""
    y0, x0, M, N = region
    fill = torch.full(out_shape, 7.0, dtype=torch.bfloat16, device="cuda")
    fused, two = fill.clone(), fill.clone()
    Kn.matmul_eltwise(a, b, prog, ops, prod_step, fused, region)
    tmp = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    Kn.matmul(a, b, tmp)
    ops2 = list(ops)
    ops2[prod_step] = Kn.OperandMap(tmp, -1, -1, -y0, -x0)
    Kn.eltwise(prog, ops2, two, region)
    torch.cuda.synchronize()
    return fused, two


@pytest.mark.parametrize("M,N,K", [(4096, 3072, 256), (4160, 3104, 160)])
def test_fused_epilogue_bit_identical_to_two_launches(M, N, K):
    torch.manual_seed(M + N + K)
    a = (torch.randn(M, K) * 0.25).bfloat16().cuda()
    b = (torch.randn(K, N) * 0.25).bfloat16().cuda()
    t = _operands(M, N, 7)
    for name, (steps, ops) in _programs(t).items():
        print(f"matmul_eltwise {M}x{N}x{K} {name}", flush=True)
        prod = next(k for k, s in enumerate(steps)
                    if s.form in (L.FORM_LOAD, L.FORM_BIN, L.FORM_BIN_REV) and ops[k] is None)
        fused, two = _pair(a, b, StackProgram(steps, 1), ops, prod, (M, N), (0, 0, M, N))
        assert torch.equal(_bits(fused), _bits(two)), name


def test_fused_epilogue_into_a_region_of_a_larger_output():
    M, N, K = 4096, 3072, 128
    a = (torch.randn(M, K) * 0.25).bfloat16().cuda()
    b = (torch.randn(K, N) * 0.25).bfloat16().cuda()
    c = torch.randn(M + 64, N + 96).bfloat16().cuda()
    # c addressed at the output element: (y, x) of the region's tensor
    prog = StackProgram([Step(L.FORM_LOAD), Step(L.FORM_BIN, OP["add"], B16),
                         Step(L.FORM_UNARY, OP["relu"], B16)], 1)
    ops = [None, Kn.OperandMap(c), None]
    region = (32, 64, M, N)
    fused, two = _pair(a, b, prog, ops, 0, (M + 64, N + 96), region)
    assert torch.equal(_bits(fused), _bits(two))
    # outside the region the output is untouched
    assert bool((fused[:32] == 7.0).all()) and bool((fused[:, :64] == 7.0).all())
    assert bool((fused[32 + M:] == 7.0).all()) and bool((fused[:, 64 + N:] == 7.0).all())


def _refused(fn):
    with pytest.raises(L.TTLHError) as e:
        fn()
    assert e.value.code == L.TTLH_EUNSUPPORTED, e.value


def test_fused_epilogue_refusals():
    M, N, K = 4096, 3072, 64
    a = torch.randn(M, K).bfloat16().cuda()
    b = torch.randn(K, N).bfloat16().cuda()
    relu = StackProgram([Step(L.FORM_LOAD), Step(L.FORM_UNARY, OP["relu"], B16)], 1)
    out32 = torch.zeros(M, N, device="cuda")
    _refused(lambda: Kn.matmul_eltwise(a, b, relu, [None, None], 0, out32, (0, 0, M, N)))
    out = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
    small_a, small_b = a[:1024].contiguous(), b[:, :1024].contiguous()
    _refused(lambda: Kn.matmul_eltwise(small_a, small_b, relu, [None, None], 0, out[:1024, :1024],
                                       (0, 0, 1024, 1024)))
    tanh = StackProgram([Step(L.FORM_LOAD), Step(L.FORM_UNARY, OP["tanh"], B16)], 1)
    _refused(lambda: Kn.matmul_eltwise(a, b, tanh, [None, None], 0, out, (0, 0, M, N)))
    c = Kn.OperandMap(torch.randn(M, N).bfloat16().cuda())
    # (c * x) + (c * c): a value pushed on the stack
    stack = StackProgram([Step(L.FORM_LOAD), Step(L.FORM_BIN, OP["mul"], B16),
                          Step(L.FORM_PUSH), Step(L.FORM_BIN, OP["mul"], B16),
                          Step(L.FORM_BIN_POP, OP["add"], B16)], 2)
    _refused(lambda: Kn.matmul_eltwise(a, b, stack, [c, None, c, c, None], 1, out, (0, 0, M, N)))
    assert not Kn.matmul_eltwise_supported(M, N, K, stack)
    assert not Kn.matmul_eltwise_supported(M, N, K, tanh)
    assert Kn.matmul_eltwise_supported(M, N, K, relu)
    torch.cuda.synchronize()
    assert bool((out == 0).all()), "a refused call launched"
