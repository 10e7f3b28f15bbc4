"""store(expr, acc=True) of an expression that is not a lone tile product:
the simulator assigns on a block's first acc store and adds on the later
ones, block = block + expr rounded to the block's dtype
(python/sim/block.py:850-864).  The planner splits the stores into rounds
(round r = the r-th acc store into its block) and plans each round after the
one before: round 0 stores expr, round r > 0 stores out + expr, with a tile
matmul inside expr planned into its own product tensor per round.

Pinned by the simulator's known answer (test/sim/test_cb.py:801-833: two
acc stores of 5 / 10 / 15 and 3 / 6 / 9 give 8 / 16 / 24) and, for the loop
forms, bit for bit against the oracle's execution of the same kernel on
inputs whose products are exact in fp32 (small integers: no summation-order
freedom, so a wrong round, a dropped term or a swapped operand shows).
"""

import pytest
import torch

import kernel_lib as KL
import plan_interp
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from ttlhip import plan as P


def _known_answer_kernel(ns):
    @ns.kernel(grid=(1, 1))
    def k(a, b, out):
        acb = ns.make_circular_buffer_like(a, shape=(3, 1))
        bcb = ns.make_circular_buffer_like(b, shape=(3, 1))
        ocb = ns.make_circular_buffer_like(out, shape=(3, 1))

        @ns.compute()
        def c():
            with ocb.reserve() as o:
                with acb.wait() as x:
                    o.store(x, acc=True)
                with bcb.wait() as y:
                    o.store(y, acc=True)

        @ns.datamovement()
        def r():
            with acb.reserve() as blk:
                ns.copy(a[0:3, 0:1], blk).wait()
            with bcb.reserve() as blk:
                ns.copy(b[0:3, 0:1], blk).wait()

        @ns.datamovement()
        def w():
            with ocb.wait() as o:
                ns.copy(o, out[0:3, 0:1]).wait()

    return k


def test_acc_store_known_answer():
    a = torch.cat([torch.full((32, 32), v) for v in (5.0, 10.0, 15.0)]).bfloat16()
    b = torch.cat([torch.full((32, 32), v) for v in (3.0, 6.0, 9.0)]).bfloat16()
    args = [ttnn.Tensor(a), ttnn.Tensor(b), ttnn.Tensor(torch.zeros(96, 32, dtype=torch.bfloat16))]
    plan = _known_answer_kernel(ttl).trace(*args)
    assert [type(l) for l in plan.launches] == [P.EltwiseLaunch, P.EltwiseLaunch]
    plan_interp.run(plan, dict(enumerate(args)))
    got = args[2]._tensor.float()
    for i, v in enumerate((8.0, 16.0, 24.0)):
        assert bool((got[32 * i:32 * (i + 1)] == v).all())


def int_inputs(bm, bk, bn, M, K, N, seed):
    g = torch.Generator().manual_seed(seed)
    a = torch.randint(-3, 4, (M, K), generator=g).bfloat16()
    b = torch.randint(-3, 4, (K, N), generator=g).bfloat16()
    c = torch.randint(-8, 9, (M, N), generator=g).bfloat16()
    return a, b, c


def run_oracle(form, bm, bk, bn, tensors, grid=(2, 2)):
    oargs = [sim_exec.OracleTensor(t.clone()) for t in tensors]
    KL.make_acc_expr(sim_exec.make_ttl(), bm, bk, bn, form, grid)(*oargs)
    return oargs[3].t


CASES = [("mm_scale_bias", 2, 2, 3, 128, 256, 192), ("relu_mm", 1, 1, 2, 128, 128, 128),
         ("eltwise", 2, 1, 1, 128, 128, 64), ("mm_scale_bias", 1, 3, 2, 64, 192, 128)]


@pytest.mark.parametrize("case", CASES)
def test_acc_expression_rounds_bit_exact_with_oracle(case):
    form, bm, bk, bn, M, K, N = case
    a, b, c = int_inputs(bm, bk, bn, M, K, N, seed=bm + 3 * bk + 7 * bn)
    out = torch.zeros(M, N, dtype=torch.bfloat16)
    ref = run_oracle(form, bm, bk, bn, (a, b, c, out))
    args = [ttnn.Tensor(t.clone()) for t in (a, b, c, out)]
    kern = KL.make_acc_expr(ttl, bm, bk, bn, form)
    plan = kern.trace(*args)
    kt = K // (bk * 32)
    # one store group per round; a product inside each round's expression
    n_mm = sum(isinstance(l, (P.MatmulLaunch, P.FusedMatmulLaunch)) for l in plan.launches)
    assert n_mm == (0 if form == "eltwise" else kt)
    plan_interp.run(plan, dict(enumerate(args)))
    assert torch.equal(args[3]._tensor.view(torch.int16), ref.view(torch.int16))


def test_acc_rounds_order_and_dropped_round_caught():
    # the oracle's value differs from one round less and from the rounds
    # added in a different rounding order: the bit-exact check above is
    # sensitive to both
    form, bm, bk, bn, M, K, N = CASES[0]
    a, b, c = int_inputs(bm, bk, bn, M, K, N, seed=bm + 3 * bk + 7 * bn)
    ref = run_oracle(form, bm, bk, bn, (a, b, c, torch.zeros(M, N, dtype=torch.bfloat16)))
    kt = K // (bk * 32)
    terms = [(a[:, k * bk * 32:(k + 1) * bk * 32].float() @ b[k * bk * 32:(k + 1) * bk * 32].float())
             .bfloat16() for k in range(kt)]
    vals = [((t * 0.5).bfloat16() + c).bfloat16() for t in terms]
    acc = vals[0]
    for v in vals[1:]:
        acc = (acc + v).bfloat16()
    assert torch.equal(acc.view(torch.int16), ref.view(torch.int16))
    assert not torch.equal(vals[0].view(torch.int16), ref.view(torch.int16))


def test_acc_store_of_expression_with_reduction_after_a_first_store_refused():
    @ttl.kernel(grid=(1, 1))
    def k(a, out):
        acb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        ocb = ttl.make_circular_buffer_like(out, shape=(1, 1), buffer_factor=2)

        @ttl.compute()
        def c():
            with ocb.reserve() as o:
                for _ in range(2):
                    with acb.wait() as x:
                        o.store(x - ttl.math.reduce_max(x, 1.0, dims=[1]), acc=True)

        @ttl.datamovement()
        def r():
            for i in range(2):
                with acb.reserve() as blk:
                    ttl.copy(a[0:1, i:i + 1], blk).wait()

        @ttl.datamovement()
        def w():
            with ocb.wait() as o:
                ttl.copy(o, out[0:1, 0:1]).wait()

    args = [ttnn.Tensor(torch.zeros(32, 64, dtype=torch.bfloat16)),
            ttnn.Tensor(torch.zeros(32, 32, dtype=torch.bfloat16))]
    with pytest.raises(NotImplementedError, match="reduction inside"):
        k.trace(*args)
