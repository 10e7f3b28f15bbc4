"""Pipes (core-to-core block transfers, python/sim/pipe.py) and tensors a
kernel body creates, on the CPU: traced, planned (a received block takes the
tile origin of the matching sent block) and run by the plan interpreter;
the reference's pipe examples run unmodified (skipped without
/root/reference)."""

import os
import sys

import pytest
import torch

import kernel_lib as KL
import plan_interp
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from ttlhip import plan as P

REF = "/root/reference/examples"
needs_ref = pytest.mark.skipif(not os.path.isdir(REF), reason="reference examples not present")


def _interp(kernel, tensors):
    args = [ttnn.Tensor(t) for t in tensors]
    plan = kernel.trace(*args)
    plan_interp.run(plan, {i: a for i, a in enumerate(args)})
    return plan


def test_row_bias_multicast_plan_and_result():
    a = O.seeded((512, 256), "uniform", 1)
    bias = O.seeded((1, 256), "uniform", 2)
    y = torch.zeros(512, 256, dtype=torch.bfloat16)
    plan = _interp(KL.make_row_bias_multicast(ttl), [a, bias, y])
    assert len(plan.launches) == 1
    assert torch.equal(y, a + bias)


def test_pipe_receive_without_send_is_a_deadlock():
    @ttl.kernel(grid=(1, 2))
    def k(a, out):
        cb = ttl.make_circular_buffer_like(a, shape=(1, 1))
        ocb = ttl.make_circular_buffer_like(out, shape=(1, 1))
        pipe = ttl.Pipe((0, 0), (0, 1))
        net = ttl.PipeNet([pipe])

        @ttl.compute()
        def c():
            with cb.wait() as b, ocb.reserve() as o:
                o.store(b)

        @ttl.datamovement()
        def r():
            with cb.reserve() as b:
                def recv(p):
                    ttl.copy(p, b).wait()
                net.if_dst(recv)
                if ttl.core(dims=1) == 0:
                    ttl.copy(a[0, 0], b).wait()

        @ttl.datamovement()
        def w():
            with ocb.wait() as o:
                ttl.copy(o, out[0, ttl.core(dims=1)]).wait()

    with pytest.raises(RuntimeError, match="Deadlock: core 1 receives more blocks"):
        k.trace(ttnn.Tensor(torch.zeros(32, 64)), ttnn.Tensor(torch.zeros(32, 64)))


def test_pipe_membership_and_ranges():
    seen = {}

    @ttl.kernel(grid=(2, 4))
    def k(a, out):
        cb = ttl.make_circular_buffer_like(a, shape=(1, 1))
        p = ttl.Pipe((1, 3), (slice(0, 2), slice(1, 3)))

        @ttl.compute()
        def c():
            seen[ttl.core(dims=1)] = (p.has_current_core(), p._dsts())

        @ttl.datamovement()
        def r():
            pass

        @ttl.datamovement()
        def w():
            pass

    plan = k.trace(ttnn.Tensor(torch.zeros(32, 32)), ttnn.Tensor(torch.zeros(32, 32)))
    assert plan.launches == []
    # cores (0,1) (0,2) (1,1) (1,2) = 1, 2, 5, 6 receive; (1,3) = 7 sends
    assert seen[0][1] == [1, 2, 5, 6]
    assert [c for c, (m, _) in sorted(seen.items()) if m] == [1, 2, 5, 6, 7]


def test_body_created_tensor_is_rebound_on_cache_hit():
    k = KL.make_scalar_expand_add(ttl, ttnn)
    a = O.seeded((64, 128), "uniform", 3)
    y = ttnn.Tensor(torch.zeros(64, 128, dtype=torch.bfloat16))
    c1 = ttnn.Tensor(torch.full((1, 1), 1.5, dtype=torch.bfloat16))
    plan = k.trace(ttnn.Tensor(a), c1, y)
    assert plan.uses_created and len(plan.created) >= 1
    c2 = ttnn.Tensor(torch.full((1, 1), -2.0, dtype=torch.bfloat16))
    again = k._created_tensors(ttnn.Tensor(a), c2, y)
    assert len(again) == len(plan.created)
    args = {0: ttnn.Tensor(a), 1: c2, 2: y}
    args.update({("created", i): t for i, t in enumerate(again)})
    plan_interp.run(plan, args)
    assert torch.equal(y._tensor, a + torch.tensor(-2.0, dtype=torch.bfloat16))


@needs_ref
@pytest.mark.parametrize("name", ["eltwise_pipe.py", "eltwise_pipe_core3.py"])
def test_reference_pipe_examples_run_unmodified(name, monkeypatch):
    from ttlhip import runner

    def call(self, *args):
        plan_interp.run(self.trace(*args), {i: x for i, x in enumerate(args)})
    monkeypatch.setattr(runner.KernelRunner, "__call__", call)
    assert not any(p.startswith("/root/reference") for p in sys.path)
    g = {"__name__": "example"}
    exec(compile(open(os.path.join(REF, name)).read(), os.path.join(REF, name), "exec"), g)
    g["main"]()  # the example's own golden check (assert_pcc)
    for m in list(sys.modules.values()):
        f = getattr(m, "__file__", None) or ""
        assert not f.startswith("/root/reference"), f"reference module imported: {f}"


def _chain_case():
    a = O.seeded((32, 64), "uniform", 11)
    b = O.seeded((64, 96), "uniform", 12)
    return [a, b, torch.zeros(64, 96, dtype=torch.bfloat16)]


def test_forwarded_pipe_block_matches_closed_form():
    # core 1 sends on a second pipe the block it received on the first: the
    # plan gives core 2's reads the tile origin core 0 copied it from.  The
    # oracle executor has no pipes; the result is pinned by its closed form
    # (one bf16 add of known tiles, exact in fp32 then rounded once, which is
    # torch's bf16 add)
    tensors = _chain_case()
    args = [ttnn.Tensor(t.clone()) for t in tensors]
    plan = KL.make_pipe_chain(ttl).trace(*args)
    plan_interp.run(plan, dict(enumerate(args)))
    a, b, _ = tensors
    want = torch.cat([torch.cat([a[:, 32 * j:32 * (j + 1)] + b[32 * j:32 * (j + 1),
                                                               32 * c:32 * (c + 1)]
                                 for c in range(3)], 1) for j in range(2)], 0)
    assert torch.equal(args[2]._tensor, want)
    # x_j = a tile (0, j) feeds output tile row j: one launch per row
    assert len(plan.launches) == 2


def test_pipes_forwarding_in_a_cycle_are_refused():
    @ttl.kernel(grid=(1, 2))
    def k(a, y):
        x_cb = ttl.make_circular_buffer_like(a, shape=(1, 1), buffer_factor=2)
        y_cb = ttl.make_circular_buffer_like(y, shape=(1, 1), buffer_factor=2)
        n01 = ttl.PipeNet([ttl.Pipe((0, 0), (0, 1))])
        n10 = ttl.PipeNet([ttl.Pipe((0, 1), (0, 0))])

        @ttl.compute()
        def comp():
            with x_cb.wait() as xb, y_cb.reserve() as yb:
                yb.store(xb)

        @ttl.datamovement()
        def reader():
            with x_cb.reserve() as xb:
                def recv(p):
                    ttl.copy(p, xb).wait()

                def send(p):
                    ttl.copy(xb, p).wait()
                n01.if_dst(recv)
                n10.if_dst(recv)
                n01.if_src(send)
                n10.if_src(send)

        @ttl.datamovement()
        def writer():
            with y_cb.wait() as yb:
                ttl.copy(yb, y[0, ttl.core(dims=1)]).wait()

    with pytest.raises((P.PlanError, RuntimeError), match="cycle|Deadlock"):
        k.trace(ttnn.Tensor(torch.zeros(32, 64)), ttnn.Tensor(torch.zeros(32, 64)))
