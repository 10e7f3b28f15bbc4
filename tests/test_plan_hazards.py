"""Planner hazards on the CPU: the plan must give the oracle's answer when an
argument is passed twice, when a store overwrites a tensor an inlined
intermediate stage reads, and when an intermediate CB is a reduction's scaler.
Each kernel runs through tracer + planner + CPU plan interpreter and through
the oracle's eager executor (the simulator's semantics), bit-exact."""

import pytest
import torch

import plan_interp
import ttl
import ttnn
import kernel_lib as KL
from oracle import sim_exec, tile_ops as O
from ttlhip import plan as P
from ttlhip import runner


def _both(make, tensors):
    """(plan result tensors, oracle result tensors, plan)."""
    k = make(ttl)
    args = [ttnn.Tensor(t.clone()) for t in tensors]
    plan = k.trace(*args)
    plan_interp.run(plan, {i: a for i, a in enumerate(args)})
    ok = make(sim_exec.make_ttl())
    oargs = [sim_exec.OracleTensor(t.clone()) for t in tensors]
    ok(*oargs)
    return [a._tensor for a in args], [a.t for a in oargs], plan


def test_cached_plan_respects_argument_aliasing(monkeypatch):
    # a plan traced for k(a, a, out) binds both leaves to argument 0; a later
    # k(a, b, out) must not reuse it
    monkeypatch.setattr(runner.P, "execute", lambda plan, amap, **kw: plan_interp.run(plan, amap))
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    k = KL.make_eltwise_add(ttl)
    a = ttnn.Tensor(torch.full((64, 64), 1.0))
    b = ttnn.Tensor(torch.full((64, 64), 5.0))
    out = ttnn.Tensor(torch.zeros(64, 64))
    k(a, a, out)
    assert torch.equal(out._tensor, torch.full((64, 64), 2.0))
    k(a, b, out)
    assert torch.equal(out._tensor, torch.full((64, 64), 6.0))
    k(b, b, out)
    assert torch.equal(out._tensor, torch.full((64, 64), 10.0))
    assert len(k._cache) == 2


def _make_overwrite(ttl):
    """S = a * 2 into an intermediate CB; a + 100 is stored back into `a`;
    then out = S + 1 (S must still be 2a of the old a)."""
    @ttl.kernel(grid=(1, 1))
    def overwrite(a, out):
        a_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        s_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        w_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, 1), buffer_factor=2)

        @ttl.compute()
        def comp():
            with a_cb.wait() as ab:
                with s_cb.reserve() as sb:
                    sb.store(ab * 2)
                with w_cb.reserve() as wb:
                    wb.store(ab + 100)
            with s_cb.wait() as sb, o_cb.reserve() as ob:
                ob.store(sb + 1)

        @ttl.datamovement()
        def rd():
            with a_cb.reserve() as ab:
                ttl.copy(a[0, 0], ab).wait()

        @ttl.datamovement()
        def wr():
            with w_cb.wait() as wb:
                ttl.copy(wb, a[0, 0]).wait()
            with o_cb.wait() as ob:
                ttl.copy(ob, out[0, 0]).wait()

    return overwrite


def test_inlined_stage_not_moved_past_an_overwrite_of_its_operand():
    a = torch.full((32, 32), 1.0, dtype=torch.bfloat16)
    out = torch.zeros(32, 32, dtype=torch.bfloat16)
    (pa, po), (oa, oo), plan = _both(_make_overwrite, [a, out])
    assert torch.equal(oo, torch.full((32, 32), 3.0, dtype=torch.bfloat16))
    assert torch.equal(oa, torch.full((32, 32), 101.0, dtype=torch.bfloat16))
    assert torch.equal(po, oo) and torch.equal(pa, oa)
    # the S stage keeps its launch: it has to run before a is overwritten
    assert len(plan.launches) == 3


def _make_self_overwrite(ttl):
    """S = a[0, 0] * 2 into an intermediate CB, then a[0, 0:2] = S + z (S
    re-used over the tile grid).  Inlined, the second store would read
    a[0, 0] in the same launch that overwrites it: on the GPU other lanes'
    writes race with those reads."""
    @ttl.kernel(grid=(1, 1))
    def self_overwrite(a, z):
        a_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        z_cb = ttl.make_circular_buffer_like(z, shape=(1, 2), buffer_factor=2)
        s_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(a, shape=(1, 2), buffer_factor=2)

        @ttl.compute()
        def comp():
            with a_cb.wait() as ab, s_cb.reserve() as sb:
                sb.store(ab * 2)
            with s_cb.wait() as sb, z_cb.wait() as zb, o_cb.reserve() as ob:
                ob.store(sb + zb)

        @ttl.datamovement()
        def rd():
            with a_cb.reserve() as ab:
                ttl.copy(a[0, 0], ab).wait()
            with z_cb.reserve() as zb:
                ttl.copy(z[0:1, 0:2], zb).wait()

        @ttl.datamovement()
        def wr():
            with o_cb.wait() as ob:
                ttl.copy(ob, a[0:1, 0:2]).wait()

    return self_overwrite


def _make_scaler_stage(ttl):
    """S = ones * 2 into an intermediate CB, read both as reduce_sum's scaler
    and as an elementwise operand (x + S)."""
    @ttl.kernel(grid=(1, 1))
    def scaler_stage(ones, x, r, y):
        one_cb = ttl.make_circular_buffer_like(ones, shape=(1, 1), buffer_factor=2)
        x_cb = ttl.make_circular_buffer_like(x, shape=(1, 1), buffer_factor=2)
        s_cb = ttl.make_circular_buffer_like(ones, shape=(1, 1), buffer_factor=2)
        r_cb = ttl.make_circular_buffer_like(r, shape=(1, 1), buffer_factor=2)
        y_cb = ttl.make_circular_buffer_like(y, shape=(1, 1), buffer_factor=2)

        @ttl.compute()
        def comp():
            with one_cb.wait() as ob, s_cb.reserve() as sb:
                sb.store(ob * 2)
            with s_cb.wait() as sb, x_cb.wait() as xb:
                with r_cb.reserve() as rb:
                    rb.store(ttl.math.reduce_sum(xb, sb, dims=[1]))
                with y_cb.reserve() as yb:
                    yb.store(xb + sb)

        @ttl.datamovement()
        def rd():
            with one_cb.reserve() as ob:
                ttl.copy(ones[0, 0], ob).wait()
            with x_cb.reserve() as xb:
                ttl.copy(x[0, 0], xb).wait()

        @ttl.datamovement()
        def wr():
            with r_cb.wait() as rb:
                ttl.copy(rb, r[0, 0]).wait()
            with y_cb.wait() as yb:
                ttl.copy(yb, y[0, 0]).wait()

    return scaler_stage


def test_scratch_scaler_keeps_its_writer():
    ones = torch.ones(32, 32, dtype=torch.bfloat16)
    x = torch.ones(32, 32, dtype=torch.bfloat16)
    r = torch.zeros(32, 32, dtype=torch.bfloat16)
    y = torch.zeros(32, 32, dtype=torch.bfloat16)
    (_, _, pr, py), (_, _, orr, oy), plan = _both(_make_scaler_stage, [ones, x, r, y])
    assert float(orr[0, 0]) == 64.0 and float(oy[0, 0]) == 3.0
    assert torch.equal(pr, orr) and torch.equal(py, oy)
    assert any(isinstance(l.out.obj, P._Scratch) for l in plan.launches)


def test_inlined_stage_not_read_by_a_launch_that_overwrites_its_operand():
    a = torch.tensor([[1.0] * 32 + [10.0] * 32] * 32, dtype=torch.bfloat16)
    z = O.seeded((32, 64), "uniform", 3, lo=-1, hi=1)
    (pa, _), (oa, _), plan = _both(_make_self_overwrite, [a, z])
    assert torch.equal(pa, oa)
    # both tiles: 2 * a[0, 0] (= 2) + z, one bf16 rounding
    assert torch.equal(oa, torch.full((32, 64), 2.0, dtype=torch.bfloat16) + z)
    # the stage keeps its own launch; the second store reads the scratch
    assert len(plan.launches) == 2
    assert isinstance(plan.launches[0].out.obj, P._Scratch)


@pytest.mark.parametrize("aliased", [False, True])
def test_cache_key_distinguishes_aliasing(aliased):
    a = ttnn.Tensor(torch.zeros(32, 32))
    b = ttnn.Tensor(torch.zeros(32, 32))
    o = ttnn.Tensor(torch.zeros(32, 32))
    k1 = runner.KernelRunner._cache_key(runner.KernelRunner, (a, a if aliased else b, o), {})
    k2 = runner.KernelRunner._cache_key(runner.KernelRunner, (b, b if aliased else a, o), {})
    k3 = runner.KernelRunner._cache_key(runner.KernelRunner, (a, b if aliased else a, o), {})
    assert k1 == k2 and k1 != k3


def _make_repeat_with_overwrite(ttl):
    """Two iterations of { out[0, 0] = x[0, 0] + 1; x[0, 0] = y[0, 0] * 2 }:
    the two instances of the first store read the same tiles but different
    values of x.  One data-movement thread both writes x and reads it again,
    so the second read follows the first write in program order."""
    @ttl.kernel(grid=(1, 1))
    def repeat_overwrite(x, y, out):
        x_cb = ttl.make_circular_buffer_like(x, shape=(1, 1), buffer_factor=2)
        y_cb = ttl.make_circular_buffer_like(y, shape=(1, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, 1), buffer_factor=2)
        w_cb = ttl.make_circular_buffer_like(x, shape=(1, 1), buffer_factor=2)

        @ttl.compute()
        def comp():
            for _ in range(2):
                with x_cb.wait() as xb, o_cb.reserve() as ob:
                    ob.store(xb + 1)
                with y_cb.wait() as yb, w_cb.reserve() as wb:
                    wb.store(yb * 2)

        @ttl.datamovement()
        def dm_x():
            for _ in range(2):
                with x_cb.reserve() as xb:
                    ttl.copy(x[0, 0], xb).wait()
                with w_cb.wait() as wb:
                    ttl.copy(wb, x[0, 0]).wait()

        @ttl.datamovement()
        def dm_y():
            for _ in range(2):
                with y_cb.reserve() as yb:
                    ttl.copy(y[0, 0], yb).wait()
                with o_cb.wait() as ob:
                    ttl.copy(ob, out[0, 0]).wait()

    return repeat_overwrite


def test_repeated_store_not_merged_across_an_overwrite_of_its_operand():
    # merging the two `out = x + 1` instances into one launch would compute
    # out from the first value of x only; the simulator's second instance
    # reads x after `x = y * 2` wrote it
    x = torch.ones(32, 32, dtype=torch.bfloat16)
    y = torch.ones(32, 32, dtype=torch.bfloat16)
    out = torch.zeros(32, 32, dtype=torch.bfloat16)
    ok = _make_repeat_with_overwrite(sim_exec.make_ttl())
    oargs = [sim_exec.OracleTensor(t.clone()) for t in (x, y, out)]
    ok(*oargs)
    assert torch.equal(oargs[2].t, torch.full((32, 32), 3.0, dtype=torch.bfloat16))
    k = _make_repeat_with_overwrite(ttl)
    args = [ttnn.Tensor(t.clone()) for t in (x, y, out)]
    with pytest.raises(P.PlanError, match="written more than once"):
        k.trace(*args)


def test_repeated_store_still_merged_when_nothing_else_touches_it():
    # every core of the grid running the same loop (broadcast_demo.py style)
    # writes the same tile from the same operands: planned once
    a = O.seeded((64, 64), "uniform", 11, lo=-1, hi=1)
    b = O.seeded((64, 64), "uniform", 12, lo=-1, hi=1)
    (_, _, po), (_, _, oo), plan = _both(_make_same_tile_all_cores,
                                         [a, b, torch.zeros(64, 64, dtype=torch.bfloat16)])
    assert torch.equal(po, oo)
    assert len(plan.launches) == 1 and plan.launches[0].tiles == 1


def _make_same_tile_all_cores(ttl):
    @ttl.kernel(grid=(2, 2))
    def same_tile(a, b, out):
        a_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        b_cb = ttl.make_circular_buffer_like(b, shape=(1, 1), buffer_factor=2)
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, 1), buffer_factor=2)

        @ttl.compute()
        def comp():
            with a_cb.wait() as ab, b_cb.wait() as bb, o_cb.reserve() as ob:
                ob.store(ab + bb)

        @ttl.datamovement()
        def rd():
            with a_cb.reserve() as ab:
                ttl.copy(a[0, 0], ab).wait()
            with b_cb.reserve() as bb:
                ttl.copy(b[0, 0], bb).wait()

        @ttl.datamovement()
        def wr():
            with o_cb.wait() as ob:
                ttl.copy(ob, out[0, 0]).wait()

    return same_tile
