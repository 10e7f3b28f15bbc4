"""The compiler's in-tile broadcast, intermediate CBs and split store sites
on the CPU: the oracle pinned by the reference's own known answers
(test/python/test_bcast_ops.py: a tile's row 0 / column 0 / [0, 0] filling
the tile, per tile of a 2x2 block, and shape expansion (1, 1) / (2, 1) /
(1, 2) -> (2, 2)), then tracer + planner + CPU plan interpreter against the
oracle, bit-exact."""

import pytest
import torch

import kernel_lib as KL
import plan_interp
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from ttlhip import plan as P


def _oracle(factory, tensors, out_index, **kw):
    k = factory(sim_exec.make_ttl(), **kw)
    args = [sim_exec.OracleTensor(t.clone()) for t in tensors]
    k(*args)
    return args[out_index].t


def _plan_run(factory, tensors, out_index, **kw):
    k = factory(ttl, **kw)
    args = [ttnn.Tensor(t.clone()) for t in tensors]
    plan = k.trace(*args)
    plan_interp.run(plan, {i: a for i, a in enumerate(args)})
    return args[out_index]._tensor, plan


def _known_input(kind, ib, values):
    """Per input tile only row 0 / column 0 / [0, 0] set (the reference's
    create_*_bcast_input helpers); values[t] for tile t in row-major order."""
    R, C = ib
    x = torch.zeros(R * 32, C * 32, dtype=torch.bfloat16)
    for t, v in enumerate(values):
        r, c = divmod(t, C)
        if kind == "row":
            x[r * 32, c * 32:(c + 1) * 32] = v
        elif kind == "col":
            x[r * 32:(r + 1) * 32, c * 32] = v
        else:
            x[r * 32, c * 32] = v
    return x


DIMS = {"row": [0], "col": [1], "scalar": [0, 1]}


@pytest.mark.parametrize("kind", ["row", "col", "scalar"])
def test_oracle_known_answer_per_tile(kind):
    vals = [1.0, 2.0, -2.5, 0.125]
    x = _known_input(kind, (2, 2), vals)
    a = torch.zeros(64, 64, dtype=torch.bfloat16)
    got = _oracle(KL.make_tile_bcast, [x, a, torch.zeros(64, 64, dtype=torch.bfloat16)], 2,
                  dims=DIMS[kind], grid=(1, 1))
    expect = torch.zeros(64, 64, dtype=torch.bfloat16)
    for t, v in enumerate(vals):
        r, c = divmod(t, 2)
        expect[r * 32:(r + 1) * 32, c * 32:(c + 1) * 32] = v
    assert torch.equal(got, expect)


@pytest.mark.parametrize("kind,ib", [("col", (2, 1)), ("row", (1, 2)), ("scalar", (1, 1))])
def test_oracle_known_answer_shape_expansion(kind, ib):
    vals = [3.0, -1.0][:ib[0] * ib[1]]
    x = _known_input(kind, ib, vals)
    a = torch.zeros(64, 64, dtype=torch.bfloat16)
    got = _oracle(KL.make_tile_bcast, [x, a, torch.zeros(64, 64, dtype=torch.bfloat16)], 2,
                  dims=DIMS[kind], ib=ib, ob=(2, 2), grid=(1, 1))
    expect = torch.zeros(64, 64, dtype=torch.bfloat16)
    for r in range(2):
        for c in range(2):
            t = (r if ib[0] > 1 else 0) * ib[1] + (c if ib[1] > 1 else 0)
            expect[r * 32:(r + 1) * 32, c * 32:(c + 1) * 32] = vals[t]
    assert torch.equal(got, expect)


def test_oracle_general_tile_is_replicated_not_kept():
    # a full random tile: dims [0] keeps row 0 only (a plausible mistake,
    # returning the tile unchanged as the simulator's validate-only broadcast
    # does, fails here)
    x = O.seeded((32, 32), "uniform", 3)
    got = _oracle(KL.make_tile_bcast, [x, torch.zeros_like(x), torch.zeros_like(x)], 2,
                  dims=[0], ib=(1, 1), ob=(1, 1), grid=(1, 1))
    assert torch.equal(got, x[:1].expand(32, 32))
    got = _oracle(KL.make_tile_bcast, [x, torch.zeros_like(x), torch.zeros_like(x)], 2,
                  dims=[1], ib=(1, 1), ob=(1, 1), grid=(1, 1))
    assert torch.equal(got, x[:, :1].expand(32, 32))


@pytest.mark.parametrize("dims", [[0], [1], [0, 1]])
@pytest.mark.parametrize("ib,expr", [((2, 2), "plain"), ((1, 1), "fma"), ((2, 1), "exp"),
                                     ((1, 2), "fma")])
def test_plan_parity(dims, ib, expr):
    if (ib[0] == 1 and 0 not in dims) or (ib[1] == 1 and 1 not in dims):
        pytest.skip("a size-1 input block dim expands only along a broadcast dim")
    rows, cols = 4, 2  # block grid
    x = O.seeded((rows * ib[0] * 32, cols * ib[1] * 32), "uniform", 5, lo=-2, hi=2)
    a = O.seeded((rows * 64, cols * 64), "uniform", 6, lo=-2, hi=2)
    out = torch.zeros(rows * 64, cols * 64, dtype=torch.bfloat16)
    kw = dict(dims=dims, ib=ib, ob=(2, 2), grid=(2, 2), expr=expr)
    got, plan = _plan_run(KL.make_tile_bcast, [x, a, out], 2, **kw)
    # an expanded block dim makes the input tile the output tile / 2: one
    # launch per input tile row / column along such a dim
    assert len(plan.launches) == (rows if ib[0] == 1 else 1) * (cols if ib[1] == 1 else 1)
    assert torch.equal(got, _oracle(KL.make_tile_bcast, [x, a, out], 2, **kw))


def test_two_stage_intermediate_cb():
    x = O.seeded((256, 128), "uniform", 7, lo=-2, hi=2)
    y = O.seeded((256, 128), "uniform", 8, lo=-2, hi=2)
    out = torch.zeros(256, 128, dtype=torch.bfloat16)
    got, plan = _plan_run(KL.make_two_stage, [x, y, out], 2)
    # stage 1 (elementwise, bf16 into a bf16 CB) is inlined into stage 2: one
    # launch reading x and y, no scratch round trip
    (l,) = plan.launches
    assert not any(isinstance(s.ref.obj, P._Temp) for s in l.operands if s is not None)
    assert torch.equal(got, _oracle(KL.make_two_stage, [x, y, out], 2))


def test_compose_axis_matches_brute_force():
    # ((c & mb) + ob) & ma) + oa == (c & m) + o for every mask pair
    masks = [-1, 31, 0, ~31]
    c = torch.arange(0, 512)
    for mb in masks:
        for ma in masks:
            for ob in (0, 64):
                for oa in (0, 96):
                    m, o = P._compose_axis(mb, ob, ma, oa)
                    s = (c & mb) + ob
                    assert torch.equal((s & ma) + oa, (c & m) + o), (mb, ob, ma, oa)


def test_intermediate_stage_kept_when_read_by_matmul_or_reduced():
    # softmax: the reduce stages still go through scratch tensors, the
    # elementwise exp stage is inlined into both of its readers
    x = O.seeded((128, 128), "uniform", 33, lo=-3, hi=3)
    s = torch.full((32, 32), 1.0, dtype=torch.bfloat16)
    _, plan = _plan_run(KL.make_softmax_rows, [x, s, torch.zeros(128, 128, dtype=torch.bfloat16)],
                        2)
    (l,) = plan.launches  # reduce_max, reduce_sum, the normalising program: one launch
    assert isinstance(l, P.ReduceEltwiseLaunch) and [r.kind for r in l.reds] == ["max", "sum"]
    assert isinstance(l.reds[0].out.obj, P._Scratch)


def test_held_tile_split_into_parts():
    a = O.seeded((256, 256), "uniform", 9, lo=-2, hi=2)
    c = O.seeded((64, 64), "uniform", 10, lo=-2, hi=2)
    out = torch.zeros(256, 256, dtype=torch.bfloat16)
    got, plan = _plan_run(KL.make_held_tile, [a, c, out], 2)
    assert len(plan.launches) == 4  # one per held tile (2x2 grid of 4x4-tile regions)
    assert torch.equal(got, _oracle(KL.make_held_tile, [a, c, out], 2))


def test_broadcast_validation():
    @ttl.kernel(grid=(1, 1))
    def k(x, out):
        x_cb = ttl.make_circular_buffer_like(x, shape=(2, 2), buffer_factor=1)
        o_cb = ttl.make_circular_buffer_like(out, shape=(2, 2), buffer_factor=1)

        @ttl.compute()
        def comp():
            with x_cb.wait() as xb, o_cb.reserve() as ob:
                ob.store(ttl.math.broadcast(xb, dims=[0]))  # no `out`: dims must be size 1

        @ttl.datamovement()
        def rd():
            with x_cb.reserve() as xb:
                ttl.copy(x[0:2, 0:2], xb).wait()

        @ttl.datamovement()
        def wr():
            with o_cb.wait() as ob:
                ttl.copy(ob, out[0:2, 0:2]).wait()

    t = ttnn.Tensor(torch.zeros(64, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="dimension must have size 1, but has size 2"):
        k.trace(t, ttnn.Tensor(torch.zeros(64, 64, dtype=torch.bfloat16)))


def test_long_chain_split_through_temporaries():
    a = O.seeded((256, 128), "uniform", 21, lo=-2, hi=2)
    b = O.seeded((256, 128), "uniform", 22, lo=-2, hi=2)
    c = O.seeded((256, 128), "uniform", 23, lo=-2, hi=2)
    out = torch.zeros(256, 128, dtype=torch.bfloat16)
    got, plan = _plan_run(KL.make_long_chain, [a, b, c, out], 3)
    assert len(plan.launches) >= 2
    assert all(len(l.prog.steps) <= 12 for l in plan.launches)
    assert isinstance(plan.launches[0].out.obj, P._Temp)
    assert torch.equal(got, _oracle(KL.make_long_chain, [a, b, c, out], 3))


def test_softmax_rows_through_intermediate_cbs():
    x = O.seeded((256, 128), "uniform", 31, lo=-3, hi=3)
    s = torch.full((32, 32), 1.0, dtype=torch.bfloat16)
    out = torch.zeros(256, 128, dtype=torch.bfloat16)
    got, plan = _plan_run(KL.make_softmax_rows, [x, s, out], 2)
    (l,) = plan.launches
    assert isinstance(l, P.ReduceEltwiseLaunch) and [r.kind for r in l.reds] == ["max", "sum"]
    assert torch.equal(got, _oracle(KL.make_softmax_rows, [x, s, out], 2))
    # and it is a softmax: rows sum to 1, close to torch's
    assert float((got.float() - torch.softmax(x.float(), 1)).abs().max()) < 2e-3


def test_inliner_keeps_stage_read_by_split_store():
    # a scratch read by a store site that has to be split into parts keeps its
    # writer's launch (the parts read the scratch itself)
    sc = P._Scratch.__new__(P._Scratch)
    inl = P._Inliner([])
    inl.exprs[id(sc)] = (None, {}, object())
    inl.note_read(sc, True)
    inl.note_read(sc, False)
    plan = P.Plan()
    writer = inl.exprs[id(sc)][2]
    plan.launches = [writer]
    inl.finish(plan)
    assert plan.launches == [writer]


@pytest.mark.parametrize("with_out", [False, True])
def test_broadcast_forms_differ_on_full_tiles(with_out):
    # b holds full 32-row tiles whose rows differ: the simulator's form (no
    # `out`, python/sim/math.py:20-106) adds the tiles as they are, the
    # compiler's form (with `out`, python/ttl/operators.py:333-360) adds row
    # 0 of each tile; closed forms with one bf16 rounding per element
    a = O.seeded((128, 128), "uniform", 41, lo=-2, hi=2)
    b = O.seeded((32, 128), "uniform", 42, lo=-2, hi=2)
    out = torch.zeros(128, 128, dtype=torch.bfloat16)
    if with_out:
        expect = a + b[0:1, :].expand(128, 128)
    else:
        expect = a + b.repeat(4, 1)
    ref = _oracle(KL.make_row_bcast_forms, [a, b, out], 2, with_out=with_out)
    got, plan = _plan_run(KL.make_row_bcast_forms, [a, b, out], 2, with_out=with_out)
    assert torch.equal(ref, expect) and torch.equal(got, expect)
    assert len(plan.launches) == 1
    other = a + (b.repeat(4, 1) if with_out else b[0:1, :].expand(128, 128))
    assert not torch.equal(expect, other)  # the two forms really differ here

