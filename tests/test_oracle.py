"""Pins of the CPU oracle (oracle/) against what the reference's own tests and
the mathematics fix, so that a wrong oracle fails here rather than passing
wrong kernels.

  - store(acc=True) known answer 5+3=8, 10+6=16, 15+9=24
    (test/sim/test_cb.py:801-833), in sim_exec and tile_ops.store_acc;
  - tile copy order: tile (h, w) of a slice lands in slot h*width + w and a
    round trip tensor -> block -> tensor is the identity
    (test/sim/test_copy.py:340-500 equality tests);
  - the reference examples' own goldens: eltwise add == a + b
    (examples/eltwise_add.py:131-132), matmul == a @ b within rtol = atol =
    1e-4 (singlecore_matmul.py:84-88), broadcast y = a*b + c
    (broadcast.py:126-143);
  - closed forms: bf16 add / mul == one RNE rounding of the exact fp32
    result; tile_matmul_sim equals an independent per-tile loop and stays
    within bf16 accumulation bounds of float64; sdpa_ref rows sum to one and
    match the textbook softmax formula.
"""

import math

import numpy as np
import pytest
import torch

from oracle import sim_exec, tile_ops as O

TILE = 32


def _copy_kernel(ttl, shape):
    @ttl.kernel(grid=(1, 1))
    def k(src, dst):
        cb = ttl.make_circular_buffer_like(src, shape=shape, buffer_factor=2)
        ocb = ttl.make_circular_buffer_like(dst, shape=shape, buffer_factor=2)

        @ttl.compute()
        def c():
            with cb.wait() as x, ocb.reserve() as o:
                o.store(x)

        @ttl.datamovement()
        def r():
            with cb.reserve() as blk:
                ttl.copy(src[0:shape[0], 0:shape[1]], blk).wait()

        @ttl.datamovement()
        def w():
            with ocb.wait() as o:
                ttl.copy(o, dst[0:shape[0], 0:shape[1]]).wait()
    return k


def test_store_acc_known_answer_sim_exec():
    ns = sim_exec.make_ttl()

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

    a = torch.cat([torch.full((32, 32), v) for v in (5.0, 10.0, 15.0)])
    b = torch.cat([torch.full((32, 32), v) for v in (3.0, 6.0, 9.0)])
    out = sim_exec.OracleTensor(torch.zeros(96, 32))
    k(sim_exec.OracleTensor(a), sim_exec.OracleTensor(b), out)
    assert [out.t[32 * i, 0].item() for i in range(3)] == [8.0, 16.0, 24.0]
    assert O.store_acc([torch.tensor(5.0), torch.tensor(3.0)]).item() == 8.0


@pytest.mark.parametrize("shape", [(1, 1), (2, 3), (3, 1)])
def test_tile_copy_round_trip_and_order(shape):
    ns = sim_exec.make_ttl()
    src = torch.arange(shape[0] * 32 * shape[1] * 32, dtype=torch.float32).reshape(
        shape[0] * 32, shape[1] * 32)
    dst = sim_exec.OracleTensor(torch.zeros_like(src))
    _copy_kernel(ns, shape)(sim_exec.OracleTensor(src), dst)
    assert torch.equal(dst.t, src)
    # slot order: the block's slot h*width + w is the tile at (h, w)
    cb = sim_exec._CB(src, shape, 1)
    blk = cb.reserve()
    sim_exec._copy(sim_exec.OracleTensor(src)[0:shape[0], 0:shape[1]], blk)
    for h in range(shape[0]):
        for w in range(shape[1]):
            tile = cb.slots[blk.idx[h * shape[1] + w]]
            assert torch.equal(tile, src[h * 32:(h + 1) * 32, w * 32:(w + 1) * 32])


def test_degenerate_column_tiles():
    ns = sim_exec.make_ttl()
    c = torch.arange(64, dtype=torch.float32).reshape(64, 1)
    blkcb = sim_exec._CB(c, (2, 1), 1)
    blk = blkcb.reserve()
    sim_exec._copy(sim_exec.OracleTensor(c)[0:2, 0], blk)
    assert blkcb.slots[blk.idx[1]].shape == (32, 1)
    assert torch.equal(blkcb.slots[blk.idx[1]][:, 0], c[32:, 0])


def test_examples_goldens_through_sim_exec():
    import kernel_lib as KL
    import ttnn
    ns = sim_exec.make_ttl()
    a, b = torch.rand(128, 128), torch.rand(128, 128)
    out = sim_exec.OracleTensor(torch.zeros(128, 128))
    KL.make_eltwise_add(ns)(sim_exec.OracleTensor(a), sim_exec.OracleTensor(b), out)
    torch.testing.assert_close(out.t, a + b, rtol=1e-5, atol=1e-8)  # eltwise_add.py:131-132
    a, b = torch.rand(128, 256), torch.rand(256, 64)
    out = sim_exec.OracleTensor(torch.zeros(128, 64))
    KL.make_matmul_multi(ns, ttnn)(sim_exec.OracleTensor(a), sim_exec.OracleTensor(b), out)
    torch.testing.assert_close(out.t, a @ b, rtol=1e-4, atol=1e-4)  # singlecore_matmul.py:84-88
    a, b = torch.rand(256, 256).bfloat16(), torch.rand(256, 256).bfloat16()
    c = torch.rand(256, 1).bfloat16()
    y = sim_exec.OracleTensor(torch.zeros(256, 256, dtype=torch.bfloat16))
    KL.make_bcast_fma(ns, g=2, grid=(2, 2))(sim_exec.OracleTensor(a), sim_exec.OracleTensor(b),
                                            sim_exec.OracleTensor(c), y)
    assert torch.allclose(y.t.float(), (a * b + c).float(), rtol=1e-2, atol=1e-2)  # broadcast.py


def test_bf16_elementwise_is_one_rounding_of_exact_fp32():
    g = torch.Generator().manual_seed(0)
    a = (torch.rand(4096, generator=g) * 8 - 4).bfloat16()
    b = (torch.rand(4096, generator=g) * 8 - 4).bfloat16()
    for op in ("add", "mul", "sub"):
        got = O.eval_expr((op, ("leaf", "a"), ("leaf", "b")), {"a": a, "b": b})
        exact = O.BINARY[op](a.double(), b.double())  # exact in double
        assert torch.equal(got, exact.float().bfloat16())  # exact in fp32 too, then RNE


def test_tile_matmul_sim_independent_loop_and_bounds():
    g = torch.Generator().manual_seed(1)
    a = torch.randn(64, 96, generator=g).bfloat16()
    b = torch.randn(96, 64, generator=g).bfloat16()
    sim = O.tile_matmul_sim(a, b)
    # independent restatement: explicit per-tile loop with the acc rule
    ref = torch.zeros(64, 64, dtype=torch.bfloat16)
    for m in range(2):
        for n in range(2):
            acc = None
            for k in range(3):
                p = a[m * 32:(m + 1) * 32, k * 32:(k + 1) * 32] @ b[k * 32:(k + 1) * 32, n * 32:(n + 1) * 32]
                acc = p if acc is None else acc + p
            ref[m * 32:(m + 1) * 32, n * 32:(n + 1) * 32] = acc
    assert torch.equal(sim, ref)
    exact = a.double() @ b.double()
    # 3 bf16 roundings of partial sums: |err| <= 3 * 2^-8 * sum |partial| (loose)
    bound = 3 * 2.0 ** -8 * (a.double().abs() @ b.double().abs())
    assert bool(((sim.double() - exact).abs() <= bound).all())


def test_sdpa_ref_invariants():
    g = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(1, 1, 64, 32, generator=g) for _ in range(3))
    out = O.sdpa_ref(q, k, v, 0.25)
    s = (q[0, 0].double() @ k[0, 0].double().T) * 0.25
    p = torch.exp(s) / torch.exp(s).sum(-1, keepdim=True)  # textbook form
    assert torch.allclose(out[0, 0], p @ v[0, 0].double(), atol=1e-12)
    ones = O.sdpa_ref(q, k, torch.ones_like(v), 0.25)
    assert torch.allclose(ones, torch.ones_like(ones, dtype=torch.float64), atol=1e-12)
    causal = O.sdpa_ref(q, k, v, 0.25, causal=True)
    assert torch.allclose(causal[0, 0, 0], v[0, 0, 0].double())  # row 0 attends to itself only
