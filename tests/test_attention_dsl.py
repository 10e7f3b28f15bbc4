"""Attention written tile by tile with the spec's block ops
(tests/kernel_lib.py make_attention: @, reduce_max, exp, broadcast,
reduce_sum, recip; docs/sphinx/specs/TTLangSpecification.md:693-761) and
planned by the drop-in onto one fused ttlh_sdpa_fwd launch.

CPU side: which programs fuse (both ways of writing the softmax numerator,
both ways of normalising) and which do not (keys of another head, a scaled
row sum, a maximum taken at another scale: the checks on every tile
position and constant, not just the op sequence); the fused plan run by the
CPU plan interpreter (float32 attention per head) against the oracle's
execution of the same program (bf16 CBs, python/sim semantics) and against
float64 softmax(Q K^T s) V.  Bar: max |plan - exact| <= 1e-2 max |exact| and
no worse than the oracle's own error (itself <= 2e-2 max |exact|: its S CB
holds bf16 scores); max |plan - oracle| within the sum of the two errors.
"""

import math

import pytest
import torch

import kernel_lib as KL
import plan_interp
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from ttlhip import plan as P


def _qkv(BH, S, D, seed):
    return [O.seeded((BH * S, D), "normal", seed + i) for i in range(3)]


def _exact(q, k, v, BH, S, D, scale):
    shape = (BH, S, D)
    return O.sdpa_ref(q.view(shape), k.view(shape), v.view(shape), scale).reshape(BH * S, D)


def _oracle(q, k, v, S, scale, **kw):
    kern = KL.make_attention(sim_exec.make_ttl(), S, scale, grid=(2, 2), **kw)
    args = [sim_exec.OracleTensor(x.clone()) for x in
            (q, k.t().contiguous(), v, torch.zeros_like(q))]
    kern(*args)
    return args[3].t


def _plan(q, k, v, S, scale, **kw):
    kern = KL.make_attention(ttl, S, scale, grid=(2, 2), **kw)
    args = [ttnn.Tensor(q.clone()), ttnn.Tensor(k.clone().t()), ttnn.Tensor(v.clone()),
            ttnn.Tensor(torch.zeros_like(q))]
    plan = kern.trace(*args)
    return plan, args


@pytest.mark.parametrize("exp_form", ["scaled_max", "scaled_diff"])
@pytest.mark.parametrize("norm", ["recip", "div"])
def test_attention_program_plans_to_one_fused_launch(exp_form, norm):
    BH, S, D = 3, 128, 64
    scale = 1.0 / math.sqrt(D)
    plan, _ = _plan(*_qkv(BH, S, D, 1), S, scale, exp_form=exp_form, norm=norm)
    assert len(plan.launches) == 1
    l = plan.launches[0]
    assert isinstance(l, P.SdpaLaunch)
    assert (l.heads, l.seq, l.scale) == (BH, S, scale)
    assert (l.q.arg, l.kt.arg, l.v.arg, l.out.arg) == (0, 1, 2, 3)


@pytest.mark.parametrize("kw", [dict(own_head=False), dict(sum_scale=2.0),
                                dict(max_scale=1.0)],
                         ids=["keys-of-head-0", "scaled-row-sum", "max-at-another-scale"])
def test_programs_that_are_not_attention_do_not_fuse(kw):
    # every query reading head 0's keys, L = 2 * row sum, or exp(S*s - max(S))
    # are other functions; the generic planner then refuses the tile matmul
    # into a score row placed at other columns than K^T's
    BH, S, D = 2, 128, 64
    with pytest.raises(P.PlanError):
        _plan(*_qkv(BH, S, D, 2), S, 1.0 / math.sqrt(D), **kw)


def test_one_sequence_per_tensor_fuses_as_one_head():
    plan, _ = _plan(*_qkv(1, 256, 128, 3), 256, 0.1)
    (l,) = plan.launches
    assert isinstance(l, P.SdpaLaunch) and (l.heads, l.seq) == (1, 256)


@pytest.mark.parametrize("BH,S,D", [(2, 128, 64), (2, 256, 128), (1, 512, 128)])
@pytest.mark.parametrize("exp_form,norm", [("scaled_max", "recip"), ("scaled_diff", "div")])
def test_fused_plan_matches_the_oracle_program(BH, S, D, exp_form, norm):
    q, k, v = _qkv(BH, S, D, 10 * S + D)
    scale = 1.0 / math.sqrt(D)
    exact = _exact(q, k, v, BH, S, D, scale)
    orc = _oracle(q, k, v, S, scale, exp_form=exp_form, norm=norm)
    plan, args = _plan(q, k, v, S, scale, exp_form=exp_form, norm=norm)
    plan_interp.run(plan, {i: a for i, a in enumerate(args)})
    got = args[3]._tensor
    e_plan = float((got.double() - exact).abs().max())
    e_orc = float((orc.double() - exact).abs().max())
    top = float(exact.abs().max())
    # the oracle computes attention up to its bf16 CBs: S (|S| ~ 4 sqrt(D))
    # rounded to bf16 before scaling moves a logit by up to ~1e-2
    assert e_orc <= 2e-2 * top
    assert e_plan <= 1e-2 * top and e_plan <= e_orc
    assert float((got.double() - orc.double()).abs().max()) <= e_orc + e_plan


def test_plan_rebinds_to_other_arguments():
    # a cached plan refers to argument positions: traced on one set of
    # tensors, it runs on others of the same shapes
    BH, S, D = 2, 128, 64
    kern = KL.make_attention(ttl, S, 0.125, grid=(2, 2))
    plan = None
    for seed in (5, 6):
        q, k, v = _qkv(BH, S, D, seed)
        args = [ttnn.Tensor(q), ttnn.Tensor(k.t()), ttnn.Tensor(v), ttnn.Tensor(torch.zeros_like(q))]
        plan = plan or kern.trace(*args)
        plan_interp.run(plan, {i: a for i, a in enumerate(args)})
        err = (args[3]._tensor.double() - _exact(q, k, v, BH, S, D, 0.125)).abs().max()
        assert float(err) <= 1e-2
