"""Attention tile programs (tests/kernel_lib.py make_attention) run through
the drop-in on the MI355X: the plan is one ttlh_sdpa_fwd launch, checked
against float64 softmax(Q K^T s) V and against the oracle's execution of
the same program.

Bar (north star: bf16 within a stated tolerance of an exact reference and
no worse than the simulator's own error): max |Y - exact| <= 1e-2 max |exact|
and <= the oracle's max error on the same inputs.  The full config-5 shape
runs through the drop-in too: sampled heads against float64 and the whole
output bit-identical to a direct ttlh_sdpa_fwd call on the same tensors.
A K^T stored as such (not a transposed view of K rows) goes through
ttlh_transpose_bf16 first; its output is bit-identical to the view's.
"""

import math

import pytest
import torch

import kernel_lib as KL
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from ttlhip import kernels as K
from ttlhip import plan as P

pytestmark = pytest.mark.gpu


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


def _gpu(q, k, v, S, scale, kt_view=True, kern=None, **kw):
    kern = kern or KL.make_attention(ttl, S, scale, grid=(8, 8), **kw)
    kt = ttnn.Tensor(k.cuda().t()) if kt_view else ttnn.from_torch(k.t())
    args = [ttnn.from_torch(q), kt, ttnn.from_torch(v), ttnn.from_torch(torch.zeros_like(q))]
    kern(*args)
    torch.cuda.synchronize()
    return ttnn.to_torch(args[3]), kern


@pytest.mark.parametrize("BH,S,D", [(2, 256, 128), (3, 128, 64), (1, 512, 128), (2, 384, 128),
                                    (2, 96, 128), (3, 160, 64)])
@pytest.mark.parametrize("exp_form,norm", [("scaled_max", "recip"), ("scaled_diff", "div")])
def test_attention_program_on_gpu_matches_exact_and_oracle(BH, S, D, exp_form, norm):
    q, k, v = _qkv(BH, S, D, 7 * S + D)
    scale = 1.0 / math.sqrt(D)
    got, kern = _gpu(q, k, v, S, scale, exp_form=exp_form, norm=norm)
    (l,) = kern.last_plan.launches
    assert isinstance(l, P.SdpaLaunch) and (l.heads, l.seq) == (BH, S)
    assert l.kbuf._t is None  # K^T was a view of K rows: nothing staged
    exact = _exact(q, k, v, BH, S, D, scale)
    e_gpu = float((got.double() - exact).abs().max())
    e_orc = float((_oracle(q, k, v, S, scale, exp_form=exp_form, norm=norm).double()
                   - exact).abs().max())
    assert e_gpu <= 1e-2 * float(exact.abs().max()), e_gpu
    assert e_gpu <= e_orc, (e_gpu, e_orc)


@pytest.mark.parametrize("BH,S,D", [(2, 256, 128), (3, 128, 64)])
def test_stored_kt_is_transposed_first(BH, S, D):
    q, k, v = _qkv(BH, S, D, 90)
    scale = 1.0 / math.sqrt(D)
    ref, _ = _gpu(q, k, v, S, scale, kt_view=True)
    kern = KL.make_attention(ttl, S, scale, grid=(8, 8))
    got, _ = _gpu(q, k, v, S, scale, kt_view=False, kern=kern)
    (l,) = kern.last_plan.launches
    assert l.kbuf._t is not None and torch.equal(l.kbuf._t.cpu(), k)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("rows,cols", [(128, 4096), (96, 136), (8, 8), (520, 64)])
def test_transpose_kernel_bitexact(rows, cols):
    x = O.seeded((rows, cols), "normal", rows + cols).cuda()
    y = torch.full((cols, rows), 7.0, dtype=torch.bfloat16, device="cuda")
    K.transpose(x, y)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), x.cpu().t())


def test_transpose_kernel_strided_rows():
    # row strides above the widths: only [rows, cols] / [cols, rows] touched
    base = O.seeded((64, 200), "normal", 3).cuda()
    x = base[:, :136]
    out = torch.full((136, 96), 5.0, dtype=torch.bfloat16, device="cuda")
    y = out[:, :64]
    K.transpose(x, y)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), x.cpu().t())
    assert bool((out[:, 64:].cpu() == 5.0).all())


def test_plan_cached_across_calls_on_gpu():
    BH, S, D = 2, 256, 128
    kern = KL.make_attention(ttl, S, 0.1, grid=(8, 8))
    for seed in (11, 12):
        q, k, v = _qkv(BH, S, D, seed)
        got, _ = _gpu(q, k, v, S, 0.1, kern=kern)
        exact = _exact(q, k, v, BH, S, D, 0.1)
        assert float((got.double() - exact).abs().max()) <= 1e-2 * float(exact.abs().max())
    assert len(kern._cache) == 1


def test_attention_program_config5_through_the_drop_in():
    # B 4, H 32, S 4096, D 128, N(0, 1), scale 1/sqrt(128)
    B, H, S, D = 4, 32, 4096, 128
    scale = 1.0 / math.sqrt(D)
    q, k, v = _qkv(B * H, S, D, 21)
    got, kern = _gpu(q, k, v, S, scale)
    (l,) = kern.last_plan.launches
    assert isinstance(l, P.SdpaLaunch) and (l.heads, l.seq, l.scale) == (B * H, S, scale)
    direct = torch.empty(B, H, S, D, dtype=torch.bfloat16, device="cuda")
    K.sdpa_fwd(*(x.cuda().view(B, H, S, D) for x in (q, k, v)), direct, scale)
    torch.cuda.synchronize()
    assert torch.equal(got, direct.cpu().view(B * H * S, D))
    for h in (0, 77, 127):
        rows = slice(h * S, (h + 1) * S)
        ref = _exact(q[rows], k[rows], v[rows], 1, S, D, scale)
        err = float((got[rows].double() - ref).abs().max())
        assert err <= 1e-2 * float(ref.abs().max()), (h, err)
