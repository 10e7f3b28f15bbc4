"""The spec's block matmul `a @ b` of an (M, K) block by a (K, N) block
(docs/sphinx/specs/TTLangSpecification.md:693): output tile (i, j) = sum
over k of a(i, k) @ b(k, j), in fp32, rounded once.  The simulator pairs
blocks tile by tile (python/sim/block.py:870-920) and raises for these
shapes; where its pairing applies it wins.

Oracle (oracle/sim_exec.py `_Tiles.__matmul__`) pinned against float64
products: every element within one bf16 ulp of the exactly rounded value.
Drop-in: the store site plans onto one tile-matmul launch accumulating
over K; run by the CPU plan interpreter it matches the oracle to one ulp.
"""

import pytest
import torch

import kernel_lib as KL
import plan_interp
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from ttlhip import dsl
from ttlhip import plan as P


def _ulps(got, exact):
    return O.bf16_ulp_diff(got, exact.to(torch.bfloat16)).abs().max()


@pytest.mark.parametrize("sa,sb,block", [((1, 3), (3, 4), True), ((2, 3), (3, 2), True),
                                        ((4, 2), (2, 1), True), ((2, 2), (2, 2), False),
                                        ((1, 1), (1, 1), False), ((3, 1), (1, 3), False),
                                        ((2, 4), (2, 4), False), ((1, 2), (2, 1), False)])
def test_which_shapes_are_block_matmuls(sa, sb, block):
    # equal or broadcast-compatible shapes ((1, 2) @ (2, 1) pairs into (2, 2))
    # and size-1 inner dims keep the simulator's tile pairing
    assert dsl._is_block_matmul(sa, sb) == block


@pytest.mark.parametrize("bm,bk,bn,R,C", [(1, 3, 4, 2, 1), (2, 3, 2, 1, 3), (3, 2, 1, 2, 2)])
def test_block_matmul_oracle_and_drop_in(bm, bk, bn, R, C):
    a = O.seeded((bm * 32 * R, bk * 32), "normal", bm + 10 * bk)
    b = O.seeded((bk * 32, bn * 32 * C), "normal", bn + 10 * R)
    exact = a.double() @ b.double()
    oargs = [sim_exec.OracleTensor(t.clone()) for t in
             (a, b, torch.zeros(a.shape[0], b.shape[1], dtype=torch.bfloat16))]
    KL.make_block_matmul(sim_exec.make_ttl(), bm, bk, bn)(*oargs)
    orc = oargs[2].t
    assert int(_ulps(orc, exact)) <= 1
    kern = KL.make_block_matmul(ttl, bm, bk, bn)
    args = [ttnn.Tensor(a.clone()), ttnn.Tensor(b.clone()),
            ttnn.Tensor(torch.zeros(a.shape[0], b.shape[1], dtype=torch.bfloat16))]
    plan = kern.trace(*args)
    (l,) = plan.launches
    assert isinstance(l, P.MatmulLaunch) and l.k == bk * 32
    plan_interp.run(plan, dict(enumerate(args)))
    got = args[2]._tensor
    assert int(_ulps(got, exact)) <= 1
    assert int(O.bf16_ulp_diff(got, orc).abs().max()) <= 1


def test_block_matmul_of_a_computed_block_matches_oracle():
    # (a * 2) @ b: the operand is materialised in bf16 first, as the
    # simulator does; exact here (a * 2 is exact in bf16, one product rounding)
    @ttl.kernel(grid=(1, 1))
    def bad(a, b, out):
        a_cb = ttl.make_circular_buffer_like(a, shape=(1, 3), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(3, 2), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, 2), buffer_factor=2)

        @ttl.compute()
        def comp():
            with a_cb.wait() as ab, b_cb.wait() as bb, o_cb.reserve() as ob:
                ob.store((ab * 2.0) @ bb)

        @ttl.datamovement()
        def rd():
            with a_cb.reserve() as ab, b_cb.reserve() as bb:
                ttl.copy(a[0:1, 0:3], ab).wait()
                ttl.copy(b[0:3, 0:2], bb).wait()

        @ttl.datamovement()
        def wr():
            with o_cb.wait() as ob:
                ttl.copy(ob, out[0:1, 0:2]).wait()

    a = O.seeded((32, 96), "normal", 81)
    b = O.seeded((96, 64), "normal", 82)
    args = [ttnn.Tensor(a), ttnn.Tensor(b), ttnn.Tensor(torch.zeros(32, 64, dtype=torch.bfloat16))]
    plan = bad.trace(*args)
    plan_interp.run(plan, dict(enumerate(args)))
    exact = ((a.double() * 2.0) @ b.double()).to(torch.bfloat16)
    assert torch.equal(args[2]._tensor, exact)
