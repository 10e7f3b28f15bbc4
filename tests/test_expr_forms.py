"""Block expressions the spec and the simulator accept, on the CPU: a tile or
block matmul of computed operands ((a * s) @ b, a @ relu(b) + c: the spec
types __matmul__(self, other: BlockExpr), docs/sphinx/specs/
TTLangSpecification.md:693, and python/sim/block.py:1012-1013 pairs any
blocks) and reductions inside a larger expression of one store (reduce_sum /
reduce_max are BlockExpr -> BlockExpr, TTLangSpecification.md:754-755).  The
plan materialises each such value in its dtype first, as the simulator
materialises every intermediate, and reads it back as an operand.

Bars: reductions and elementwise ops bit-exact with the oracle's eager
executor (plan interpreter on the CPU); matmuls within 2^-7 max |exact| of a
float64 evaluation of the same program (operands rounded to bf16 once, the
product rounded once) and no worse than the oracle's error plus 2^-9.  The
oracle is pinned to exact softmax / row centring / products by those float64
evaluations, which a dropped term or a wrong reduction axis misses by far.
"""

import pytest
import torch

import kernel_lib as KL
import plan_interp
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from ttlhip import plan as P


def _both(make, tensors, out_index, **kw):
    k = make(ttl, **kw)
    args = [ttnn.Tensor(t.clone()) for t in tensors]
    plan = k.trace(*args)
    plan_interp.run(plan, dict(enumerate(args)))
    ok = make(sim_exec.make_ttl(), **kw)
    oargs = [sim_exec.OracleTensor(t.clone()) for t in tensors]
    ok(*oargs)
    return args[out_index]._tensor, oargs[out_index].t, plan


def softmax_case(seed=5, rows=128, cols=128):
    x = O.seeded((rows, cols), "uniform", seed, lo=-4, hi=4)
    return [x, torch.ones(32, 32, dtype=torch.bfloat16), torch.zeros(rows, cols, dtype=torch.bfloat16)]


def test_softmax_in_one_store_plans_reductions_first_and_matches_oracle():
    t = softmax_case()
    got, orc, plan = _both(KL.make_softmax_one_store, t, 2)
    (l,) = plan.launches  # the two reductions and the program: one fused launch
    assert isinstance(l, P.ReduceEltwiseLaunch) and [r.kind for r in l.reds] == ["max", "sum"]
    assert torch.equal(got, orc)
    # the oracle against exact softmax: within a few bf16 roundings
    ex = torch.softmax(t[0].double(), 1)
    assert float((orc.double() - ex).abs().max()) <= 2 ** -6 * float(ex.max())
    # a softmax without the recip of the row sum is far off
    assert float((torch.exp(t[0].double() - t[0].double().amax(1, keepdim=True)) - ex).abs().max()) > 0.5


def test_row_centring_in_one_store_matches_oracle():
    t = softmax_case(seed=6)
    got, orc, plan = _both(KL.make_softmax_one_store, t, 2, form="center")
    (l,) = plan.launches
    assert isinstance(l, P.ReduceEltwiseLaunch) and [r.kind for r in l.reds] == ["sum"]
    assert torch.equal(got, orc)
    x = t[0].double()
    ex = x - x.mean(1, keepdim=True)
    assert float((orc.double() - ex).abs().max()) <= 2 ** -6 * float(x.abs().max())


def test_rms_normalisation_in_one_store_matches_oracle():
    t = softmax_case(seed=8)
    got, orc, plan = _both(KL.make_softmax_one_store, t, 2, form="rms")
    (l,) = plan.launches
    assert isinstance(l, P.ReduceEltwiseLaunch) and [r.kind for r in l.reds] == ["sum"]
    assert torch.equal(got, orc)
    x = t[0].double()
    ex = x * torch.rsqrt((x * x).mean(1, keepdim=True) + 1e-5)
    assert float((orc.double() - ex).abs().max()) <= 2 ** -6 * float(ex.abs().max())


def _mm_exact(a, b, c, form):
    r = lambda v: v.to(torch.bfloat16).double()  # one bf16 rounding
    A, B = a.double(), b.double()
    if form == "scale":
        return r(r(A * 0.25) @ B)
    if form == "relu_b":
        return r(r(A @ r(torch.relu(B))) + c.double())
    return r(r(A + A) @ r(B * 2.0))


@pytest.mark.parametrize("form", ["scale", "relu_b", "both"])
def test_matmul_of_computed_operands(form):
    bm, bk, bn = 2, 3, 2
    M, K, N = bm * 32 * 2, bk * 32, bn * 32 * 2
    a, b, c = (O.seeded(s, "normal", 40 + i) for i, s in enumerate([(M, K), (K, N), (M, N)]))
    tensors = [a, b, c, torch.zeros(M, N, dtype=torch.bfloat16)]
    got, orc, plan = _both(KL.make_matmul_computed_operand, tensors, 3, bm=bm, bk=bk, bn=bn,
                           form=form)
    kinds = [type(l).__name__ for l in plan.launches]
    mm = "FusedMatmulLaunch" if form == "relu_b" else "MatmulLaunch"
    assert kinds.count(mm) == 1 and kinds.index(mm) > 0, kinds
    ex = _mm_exact(a, b, c, form)
    top = float(ex.abs().max())
    e_plan = float((got.double() - ex).abs().max())
    e_orc = float((orc.double() - ex).abs().max())
    assert e_orc <= 2 ** -7 * top, e_orc
    assert e_plan <= 2 ** -7 * top and e_plan <= e_orc + 2 ** -9 * top, (e_plan, e_orc)


def test_matmul_of_computed_operand_exact_reference_catches_a_dropped_scale():
    a, b = O.seeded((128, 96), "normal", 50), O.seeded((96, 128), "normal", 51)
    ex = _mm_exact(a, b, None, "scale")
    wrong = (a.double() @ b.double()).to(torch.bfloat16).double()
    assert float((wrong - ex).abs().max()) > 2 ** -3 * float(ex.abs().max())


def test_operand_reused_with_different_values_is_refused():
    # the same a tile scaled by two different factors in two stores of one
    # site would need two values in one tile of the operand's tensor
    @ttl.kernel(grid=(1, 1))
    def k(a, b, s, out):
        a_cb = ttl.make_circular_buffer_like(a, shape=(2, 3), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(3, 1), buffer_factor=2)
        s_cb = ttl.make_circular_buffer_like(s, shape=(1, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(2, 1), buffer_factor=2)

        @ttl.compute()
        def comp():
            for _ in range(2):
                with a_cb.wait() as ab, b_cb.wait() as bb, s_cb.wait() as sb, \
                        o_cb.reserve() as ob:
                    ob.store((ab * ttl.math.broadcast(sb, ab, dims=[0, 1])) @ bb)

        @ttl.datamovement()
        def rd():
            for j in range(2):
                with a_cb.reserve() as ab, b_cb.reserve() as bb, s_cb.reserve() as sb:
                    ttl.copy(a[0:2, 0:3], ab).wait()
                    ttl.copy(b[0:3, j:j + 1], bb).wait()
                    ttl.copy(s[0, j], sb).wait()

        @ttl.datamovement()
        def wr():
            for j in range(2):
                with o_cb.wait() as ob:
                    ttl.copy(ob, out[0:2, j:j + 1]).wait()

    args = [ttnn.Tensor(t) for t in (torch.ones(64, 96), torch.ones(96, 64), torch.ones(32, 64),
                                     torch.zeros(64, 64))]
    with pytest.raises(P.PlanError, match="more than once"):
        k.trace(*args)
