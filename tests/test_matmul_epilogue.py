"""A tile or block matmul inside a larger store expression, e.g.
`store(relu(a @ b + c))` (the spec's block ops compose freely:
docs/sphinx/specs/TTLangSpecification.md:693-761).  The simulator
materialises the product block in its operands' promoted dtype (bf16 here)
before the other ops read it (python/sim/block.py:870-920); the drop-in
plans the same thing as two launches: the product into a plan-owned tensor
laid out like the output, then the elementwise program reading it.

Bar: the oracle (oracle/sim_exec.py) and the plan, run by the CPU plan
interpreter, are each within 2^-7 max |exact| of a float64 evaluation of
the same program (product rounded to bf16 once, the other ops exact); the
plan's error is no larger than the oracle's plus 2^-9 max |exact|.  Dropping
the bias, the relu or the scale, or pairing the wrong tiles, moves the
result by far more than that.
"""

import pytest
import torch

import kernel_lib as KL
import plan_interp
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from ttlhip import plan as P

# (bm, bk, bn, R, C, epilogue): block matmuls (bk > 1, shapes the simulator
# cannot pair tile-wise) and tile-wise products with K = 32 (bk = 1);
# R x C output blocks dealt over a 2 x 2 grid
CASES = [(2, 3, 1, 2, 2, "relu_bias"), (1, 1, 2, 4, 2, "row_bias"),
         (1, 2, 3, 2, 2, "scale_exp"), (1, 1, 1, 4, 4, "relu_bias")]


def inputs(bm, bk, bn, R, C, epi, seed=1):
    M, K, N = bm * 32 * R, bk * 32, bn * 32 * C
    a = O.seeded((M, K), "normal", seed)
    b = O.seeded((K, N), "normal", seed + 1)
    c = O.seeded((1, N) if epi == "row_bias" else (M, N), "normal", seed + 2)
    return a, b, c, torch.zeros(M, N, dtype=torch.bfloat16)


def exact(a, b, c, epi):
    p = (a.double() @ b.double()).to(torch.bfloat16).double()
    if epi == "relu_bias":
        return torch.relu(p + c.double())
    if epi == "row_bias":
        return p + c.double()
    return torch.exp(p * 0.125) * c.double()


def run_oracle(case, tensors):
    bm, bk, bn, _, _, epi = case
    args = [sim_exec.OracleTensor(t.clone()) for t in tensors]
    KL.make_matmul_epilogue(sim_exec.make_ttl(), bm, bk, bn, epi)(*args)
    return args[3].t


@pytest.mark.parametrize("case", CASES)
def test_oracle_pinned_to_exact(case):
    a, b, c, out = inputs(*case)
    ex = exact(a, b, c, case[5])
    err = float((run_oracle(case, (a, b, c, out)).double() - ex).abs().max())
    assert err <= 2 ** -7 * float(ex.abs().max()), err


def test_exact_reference_catches_a_dropped_bias():
    # the bar above is far below what a planted mistake in the oracle moves
    a, b, c, _ = inputs(*CASES[0])
    ex = exact(a, b, c, "relu_bias")
    wrong = torch.relu((a.double() @ b.double()).to(torch.bfloat16).double())
    assert float((wrong - ex).abs().max()) > 2 ** -5 * float(ex.abs().max())


@pytest.mark.parametrize("case", CASES)
def test_plan_is_a_matmul_with_its_program_fused_and_matches(case):
    bm, bk, bn, R, C, epi = case
    a, b, c, out = inputs(*case)
    orc = run_oracle(case, (a, b, c, out))
    args = [ttnn.Tensor(t.clone()) for t in (a, b, c, out)]
    plan = KL.make_matmul_epilogue(ttl, bm, bk, bn, epi).trace(*args)
    (fl,) = plan.launches
    assert isinstance(fl, P.FusedMatmulLaunch)
    mm, ew = fl.mm, fl.ew
    assert isinstance(mm, P.MatmulLaunch) and isinstance(ew, P.EltwiseLaunch)
    assert ew.operands[fl.prod_step].ref.obj is mm.c.obj
    assert mm.k == bk * 32
    plan_interp.run(plan, dict(enumerate(args)))
    ex = exact(a, b, c, epi)
    top = float(ex.abs().max())
    e_plan = float((args[3]._tensor.double() - ex).abs().max())
    e_orc = float((orc.double() - ex).abs().max())
    assert e_plan <= 2 ** -7 * top, e_plan
    assert e_plan <= e_orc + 2 ** -9 * top, (e_plan, e_orc)


def _one_block_kernel(body):
    @ttl.kernel(grid=(1, 1))
    def k(a, b, c, out):
        a_cb = ttl.make_circular_buffer_like(a, shape=(1, 2), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(2, 3), buffer_factor=2)
        c_cb = ttl.make_circular_buffer_like(c, shape=(1, 3), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, 3), buffer_factor=2)

        @ttl.compute()
        def comp():
            with a_cb.wait() as ab, b_cb.wait() as bb, c_cb.wait() as cc, o_cb.reserve() as ob:
                body(ob, ab, bb, cc)

        @ttl.datamovement()
        def rd():
            with a_cb.reserve() as ab, b_cb.reserve() as bb, c_cb.reserve() as cc:
                ttl.copy(a[0:1, 0:2], ab).wait()
                ttl.copy(b[0:2, 0:3], bb).wait()
                ttl.copy(c[0:1, 0:3], cc).wait()

        @ttl.datamovement()
        def wr():
            with o_cb.wait() as ob:
                ttl.copy(ob, out[0:1, 0:3]).wait()

    return k


def _trace(body):
    a, b, c = (O.seeded(s, "normal", i) for i, s in enumerate([(32, 64), (64, 96), (32, 96)]))
    args = [ttnn.Tensor(t) for t in (a, b, c, torch.zeros(32, 96, dtype=torch.bfloat16))]
    return _one_block_kernel(body).trace(*args)


def test_one_block_product_plus_bias_plans():
    plan = _trace(lambda ob, ab, bb, cc: ob.store(ab @ bb + cc))
    assert [type(l) for l in plan.launches] == [P.FusedMatmulLaunch]


def _two_products_kernel(ns):
    @ns.kernel(grid=(1, 1))
    def k(a, b, out):
        a0_cb = ns.make_circular_buffer_like(a, shape=(1, 2), buffer_factor=2)
        a1_cb = ns.make_circular_buffer_like(a, shape=(1, 2), buffer_factor=2)
        b_cb = ns.make_circular_buffer_like(b, shape=(2, 3), buffer_factor=2)
        o_cb = ns.make_circular_buffer_like(out, shape=(1, 3), buffer_factor=2)

        @ns.compute()
        def comp():
            with a0_cb.wait() as a0, a1_cb.wait() as a1, b_cb.wait() as bb, \
                    o_cb.reserve() as ob:
                ob.store(a0 @ bb + a1 @ bb)
            with a0_cb.wait() as a0, b_cb.wait() as bb, o_cb.reserve() as ob:
                ob.store(a0 @ bb * (a0 @ bb))
            with a1_cb.wait() as a1, b_cb.wait() as bb, o_cb.reserve() as ob:
                ob.store(a1 @ bb)

        @ns.datamovement()
        def rd():
            with a0_cb.reserve() as x, a1_cb.reserve() as y, b_cb.reserve() as z:
                ns.copy(a[0:1, 0:2], x).wait()
                ns.copy(a[1:2, 0:2], y).wait()
                ns.copy(b[0:2, 0:3], z).wait()
            with a0_cb.reserve() as x, b_cb.reserve() as z:
                ns.copy(a[0:1, 0:2], x).wait()
                ns.copy(b[0:2, 0:3], z).wait()
            with a1_cb.reserve() as y, b_cb.reserve() as z:
                ns.copy(a[1:2, 0:2], y).wait()
                ns.copy(b[0:2, 0:3], z).wait()

        @ns.datamovement()
        def wr():
            for r in range(3):
                with o_cb.wait() as ob:
                    ns.copy(ob, out[r:r + 1, 0:3]).wait()

    return k


def two_products_case():
    a = O.seeded((64, 64), "normal", 3)
    b = O.seeded((64, 96), "normal", 4)
    p0 = (a[:32].double() @ b.double()).to(torch.bfloat16).double()
    p1 = (a[32:].double() @ b.double()).to(torch.bfloat16).double()
    return (a, b, torch.zeros(96, 96, dtype=torch.bfloat16)), torch.cat([p0 + p1, p0 * p0, p1])


def test_two_products_in_one_expression_and_an_offset_product():
    # two products of blocks of the same tensors (a's tile rows 0 and 1, the
    # same b) each get their own tensor: a0 @ b + a1 @ b, a0 @ b twice; and
    # a1 @ b stored into output tile row 2 (A read at a fixed row offset)
    tensors, ex = two_products_case()
    args = [ttnn.Tensor(t.clone()) for t in tensors]
    plan = _two_products_kernel(ttl).trace(*args)
    mms = [l for l in plan.launches if isinstance(l, P.MatmulLaunch)]
    fused = [l for l in plan.launches if isinstance(l, P.FusedMatmulLaunch)]
    # a0 @ b + a1 @ b: two products read by one program (not fused); a0 @ b
    # twice in one product: two products; a1 @ b stored on its own
    assert len(mms) + len(fused) == 5
    plan_interp.run(plan, dict(enumerate(args)))
    oargs = [sim_exec.OracleTensor(t.clone()) for t in tensors]
    _two_products_kernel(sim_exec.make_ttl())(*oargs)
    top = float(ex.abs().max())
    e_plan = float((args[2]._tensor.double() - ex).abs().max())
    e_orc = float((oargs[2].t.double() - ex).abs().max())
    assert e_orc <= 2 ** -7 * top, e_orc
    assert e_plan <= 2 ** -7 * top and e_plan <= e_orc + 2 ** -9 * top, (e_plan, e_orc)


def test_single_acc_store_of_an_expression_is_a_plain_store():
    # the first store(acc=True) into a block assigns (python/sim/block.py:
    # 850-864): one acc store per block plans like store() (the loop forms:
    # tests/test_acc_store.py)
    plan = _trace(lambda ob, ab, bb, cc: ob.store(ab @ bb + cc, acc=True))
    assert [type(l) for l in plan.launches] == [P.FusedMatmulLaunch]


def test_computed_operand_plans_the_operand_first():
    # (a * 2) @ b + c: the operand is materialised in bf16 first (an
    # elementwise launch into a tensor laid out like a), then the product,
    # then the epilogue (tests/test_expr_forms.py checks the values)
    plan = _trace(lambda ob, ab, bb, cc: ob.store((ab * 2.0) @ bb + cc))
    assert [type(l) for l in plan.launches] == [P.EltwiseLaunch, P.FusedMatmulLaunch]


@pytest.mark.parametrize("epi,fused", [("relu_bias", True), ("row_bias", True),
                                       ("scale_exp", False)])
def test_fused_form_chosen_by_program_length(epi, fused):
    # the executor's choice between ttlh_matmul_eltwise and the two launches
    # (kernels.matmul_eltwise_preferred); both are supported at this size
    from ttlhip import kernels as Kn
    bm, bk, bn = 4, 8, 4
    M, K, N = 4096, 256, 3072
    tensors = [torch.zeros(M, K, dtype=torch.bfloat16), torch.zeros(K, N, dtype=torch.bfloat16),
               torch.zeros((1, N) if epi == "row_bias" else (M, N), dtype=torch.bfloat16),
               torch.zeros(M, N, dtype=torch.bfloat16)]
    plan = KL.make_matmul_epilogue(ttl, bm, bk, bn, epi).trace(*[ttnn.Tensor(t) for t in tensors])
    (fl,) = plan.launches
    assert isinstance(fl, P.FusedMatmulLaunch)
    assert Kn.matmul_eltwise_supported(M, N, K, fl.ew.prog)
    assert Kn.matmul_eltwise_preferred(fl.ew.prog) == fused
