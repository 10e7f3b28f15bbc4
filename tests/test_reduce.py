"""ttl.math.reduce_sum / reduce_max on the CPU: the oracle pinned by closed
forms, the tracer + planner checked end to end against it (through the CPU
plan interpreter), and the DSL / planner error paths.

The reference specifies only the signature of the reductions
(docs/sphinx/specs/TTLangSpecification.md:754-755) and implements neither, so
there is no reference output to compare with ("parity unpinned" against the
reference).  What pins the oracle instead: sums of constant blocks, maxima of
integer patterns (exact in bf16), the sign rule of a negative scaler, NaN
propagation, and the equivalence of a row reduction with the transposed
column reduction.
"""

import pytest
import torch

import kernel_lib as KL
import plan_interp
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from ttlhip import plan as P


def _oracle(factory, tensors, out_index, **kw):
    ons = sim_exec.make_ttl()
    k = factory(ons, **kw)
    oargs = [sim_exec.OracleTensor(t.clone()) for t in tensors]
    k(*oargs)
    return oargs[out_index].t


def _run_both(factory, tensors, out_index, **kw):
    k = factory(ttl, **kw)
    args = [ttnn.Tensor(t.clone()) for t in tensors]
    plan = k.trace(*args)
    plan_interp.run(plan, {i: a for i, a in enumerate(args)})
    return args[out_index]._tensor, _oracle(factory, tensors, out_index, **kw), plan


def _scaler(v, dtype=torch.bfloat16):
    return torch.full((32, 32), v, dtype=dtype)


# --- the oracle against closed forms ----------------------------------------


def test_oracle_row_sum_of_ones():
    x = torch.ones(256, 256, dtype=torch.bfloat16)
    out = torch.zeros(256, 1, dtype=torch.bfloat16)
    got = _oracle(KL.make_reduce_rows, [x, _scaler(0.5), out], 2, gc=8)
    assert torch.equal(got, torch.full((256, 1), 128.0, dtype=torch.bfloat16))


def test_oracle_row_max_integer_pattern_and_negative_scaler():
    j = torch.arange(256) % 64 - 32  # -32 .. 31 in every row
    x = j.repeat(256, 1).to(torch.bfloat16)
    for s, expect in ((0.5, 15.5), (-0.5, 16.0)):  # max(x * s): 31 * 0.5, -32 * -0.5
        out = torch.zeros(256, 32, dtype=torch.bfloat16)
        got = _oracle(KL.make_reduce_rows, [x, _scaler(s), out], 2, kind="max", gc=8)
        assert torch.equal(got[:, 0], torch.full((256,), expect, dtype=torch.bfloat16))
        assert torch.count_nonzero(got[:, 1:]) == 0  # the rest of each result tile is zero


def test_oracle_column_sum_closed_form():
    i = torch.arange(256) % 8  # column sums: 32 * (0 + ... + 7) = 896
    x = i.view(-1, 1).repeat(1, 256).to(torch.bfloat16)
    out = torch.zeros(1, 256, dtype=torch.bfloat16)
    got = _oracle(KL.make_reduce_cols, [x, _scaler(1.0), out], 2, gr=8, gc=2)
    assert torch.equal(got, torch.full((1, 256), 896.0, dtype=torch.bfloat16))


def test_oracle_nan_propagates_per_row():
    x = torch.ones(256, 256, dtype=torch.bfloat16)
    x[5, 77] = float("nan")
    for kind in ("sum", "max"):
        out = torch.zeros(256, 1, dtype=torch.bfloat16)
        got = _oracle(KL.make_reduce_rows, [x, _scaler(1.0), out], 2, kind=kind, gc=8)
        assert torch.isnan(got[5, 0]) and not torch.isnan(got[torch.arange(256) != 5]).any()


def test_oracle_row_reduce_equals_transposed_column_reduce():
    x = O.seeded((256, 256), "uniform", 11, lo=-3, hi=3)
    rows = _oracle(KL.make_reduce_rows, [x, _scaler(0.25), torch.zeros(256, 1, dtype=torch.bfloat16)],
                   2, kind="max", gc=8)
    cols = _oracle(KL.make_reduce_cols, [x.T.contiguous(), _scaler(0.25),
                                         torch.zeros(1, 256, dtype=torch.bfloat16)],
                   2, kind="max", gr=8, gc=2)
    assert torch.equal(rows.view(-1), cols.view(-1))


def test_oracle_full_max_closed_form():
    x = torch.zeros(128, 128, dtype=torch.bfloat16)  # exp(0) = 1, so the max is max(y) * s
    y = O.seeded((128, 128), "uniform", 12, lo=-1, hi=1)
    got = _oracle(KL.make_reduce_all, [x, y, _scaler(2.0), torch.zeros(1, 1, dtype=torch.bfloat16)], 3)
    assert float(got) == float(y.max()) * 2.0


# --- tracer + planner against the oracle --------------------------------------


@pytest.mark.parametrize("kind", ["sum", "max"])
@pytest.mark.parametrize("out_w", [1, 32])
def test_row_reduce_plan_and_parity(kind, out_w):
    x = O.seeded((256, 256), "uniform", 1, lo=-2, hi=2)
    out = torch.zeros(256, out_w, dtype=torch.bfloat16)
    got, ref, plan = _run_both(KL.make_reduce_rows, [x, _scaler(0.5), out], 2, kind=kind, gc=8)
    (l,) = plan.launches
    assert isinstance(l, P.ReduceLaunch) and l.dims == (1,) and l.kind == kind
    assert l.region == (0, 0, 256, 256) and l.out_pad == (out_w == 32)
    assert l.scaler is not None and l.scaler_at == (0, 0)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("kind", ["sum", "max"])
def test_column_reduce_plan_and_parity(kind):
    x = O.seeded((256, 256), "uniform", 2, lo=-2, hi=2)
    out = torch.zeros(1, 256, dtype=torch.bfloat16)
    got, ref, plan = _run_both(KL.make_reduce_cols, [x, _scaler(-0.75), out], 2, kind=kind, gr=8)
    (l,) = plan.launches
    assert l.dims == (0,) and l.region == (0, 0, 256, 256) and not l.out_pad
    assert torch.equal(got, ref)


def test_full_reduce_of_fused_expression():
    x = O.seeded((128, 128), "uniform", 3, lo=-1, hi=1)
    y = O.seeded((128, 128), "uniform", 4, lo=-1, hi=1)
    for ow in (1, 32):
        got, ref, plan = _run_both(KL.make_reduce_all, [x, y, _scaler(1.5),
                                                        torch.zeros(ow, ow, dtype=torch.bfloat16)], 3)
        (l,) = plan.launches
        assert l.dims == (0, 1) and len(l.prog.steps) == 3  # exp(x) * y
        assert torch.equal(got, ref)


def test_row_dot_constant_scaler():
    a = O.seeded((256, 128), "uniform", 5, lo=-1, hi=1)
    b = O.seeded((256, 128), "uniform", 6, lo=-1, hi=1)
    got, ref, plan = _run_both(KL.make_row_dot, [a, b, torch.zeros(256, 32, dtype=torch.bfloat16)], 2)
    (l,) = plan.launches
    assert l.scaler is None and l.scale == 1.0
    assert torch.equal(got, ref)


def test_accumulated_row_sum_over_blocks():
    # several column blocks per row stored with acc=True: the planner sums the
    # whole row in fp32 and rounds once; the simulator adds bf16-rounded
    # partial sums, so the two agree to within the partials' rounding
    x = O.seeded((256, 256), "uniform", 7, lo=-2, hi=2)
    got, ref, plan = _run_both(KL.make_reduce_rows, [x, _scaler(1.0),
                                                     torch.zeros(256, 1, dtype=torch.bfloat16)],
                               2, gc=2)
    (l,) = plan.launches
    assert l.region == (0, 0, 256, 256)
    exact = x.double().sum(1, keepdim=True)
    assert float((got.double() - exact).abs().max()) <= float(exact.abs().max()) * 2 ** -8
    assert float((got.double() - ref.double()).abs().max()) <= float(exact.abs().max()) * 2 ** -5


# --- errors ---------------------------------------------------------------------


def _one_block_kernel(body):
    @ttl.kernel(grid=(1, 1))
    def k(x, s, out):
        x_cb = ttl.make_circular_buffer_like(x, shape=(2, 2), buffer_factor=1)
        s_cb = ttl.make_circular_buffer_like(s, shape=(1, 1), buffer_factor=1)
        o_cb = ttl.make_circular_buffer_like(out, shape=(2, 1), buffer_factor=1)

        @ttl.compute()
        def comp():
            with x_cb.wait() as xb, s_cb.wait() as sb, o_cb.reserve() as ob:
                body(ob, xb, sb)

        @ttl.datamovement()
        def reader():
            with x_cb.reserve() as xb, s_cb.reserve() as sb:
                tx = ttl.copy(x[0:2, 0:2], xb)
                ts = ttl.copy(s[0, 0], sb)
                tx.wait()
                ts.wait()

        @ttl.datamovement()
        def writer():
            with o_cb.wait() as ob:
                ttl.copy(ob, out[0:2, 0]).wait()

    x = ttnn.Tensor(torch.ones(64, 64, dtype=torch.bfloat16))
    s = ttnn.Tensor(_scaler(1.0))
    out = ttnn.Tensor(torch.zeros(64, 1, dtype=torch.bfloat16))
    return k.trace(x, s, out)


@pytest.mark.parametrize("body,exc,msg", [
    (lambda ob, xb, sb: ob.store(ttl.math.reduce_sum(xb, sb)), ValueError, "dims parameter"),
    (lambda ob, xb, sb: ob.store(ttl.math.reduce_sum(xb, sb, dims=[2])), ValueError, "dims must"),
    (lambda ob, xb, sb: ob.store(ttl.math.reduce_sum(xb, xb, dims=[1])), ValueError,
     "scaler must be a \\(1, 1\\) block"),
    (lambda ob, xb, sb: ob.store(ttl.math.reduce_max(xb, sb, dims=[0])), ValueError,
     "must have the reduced shape"),
])
def test_reduce_validation(body, exc, msg):
    with pytest.raises(exc, match=msg):
        _one_block_kernel(body)


def test_reduction_inside_a_larger_expression_plans_it_first():
    # reduce_sum(...) * 2: the reduction into a plan-owned tensor, then the
    # scale reading it (tests/test_expr_forms.py checks values end to end)
    plan = _one_block_kernel(lambda ob, xb, sb: ob.store(ttl.math.reduce_sum(xb, sb, dims=[1]) * 2.0))
    # (the scale runs over the result tile, not the reduced rows: two launches)
    assert [type(l) for l in plan.launches] == [P.ReduceLaunch, P.EltwiseLaunch]


def test_reduce_max_accumulated_over_stores_is_rejected():
    x = O.seeded((64, 256), "uniform", 8)
    k = KL.make_reduce_rows(ttl, kind="max", gr=2, gc=2, grid=(1, 1))
    with pytest.raises(P.PlanError, match="reduce_max partial results"):
        k.trace(ttnn.Tensor(x), ttnn.Tensor(_scaler(1.0)),
                ttnn.Tensor(torch.zeros(64, 1, dtype=torch.bfloat16)))
