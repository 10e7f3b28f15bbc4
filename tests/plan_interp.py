"""CPU interpreter of a front-end Plan (test infrastructure).

Executes the launches a traced kernel produced with torch on the CPU, using
the launch's own operand maps (mask / offset / size-1 broadcast) and stack
program, so the CPU test suite can check the tracer + planner end to end
against the oracle's eager executor without a GPU.
"""

import torch

from oracle import tile_ops as O
from ttlhip import _lib as L
from ttlhip.plan import (EltwiseLaunch, FusedMatmulLaunch, MatmulLaunch, ReduceEltwiseLaunch,
                         ReduceLaunch, SdpaLaunch)

_TORCH_BIN = {
    L.OP["add"]: torch.add, L.OP["sub"]: torch.sub, L.OP["mul"]: torch.mul,
    L.OP["div"]: torch.true_divide, L.OP["max"]: torch.maximum, L.OP["min"]: torch.minimum,
    L.OP["pow"]: torch.pow, L.OP["floordiv"]: torch.floor_divide, L.OP["mod"]: torch.remainder,
}
_TORCH_UN = {
    L.OP["exp"]: torch.exp, L.OP["log"]: torch.log, L.OP["sqrt"]: torch.sqrt,
    L.OP["rsqrt"]: torch.rsqrt, L.OP["tanh"]: torch.tanh, L.OP["abs"]: torch.abs,
    L.OP["neg"]: torch.neg, L.OP["relu"]: torch.relu, L.OP["sigmoid"]: torch.sigmoid,
    L.OP["recip"]: torch.reciprocal,
}
for _name, _fn in O.UNARY.items():  # the spec's further functions
    _TORCH_UN.setdefault(L.OP[_name], _fn)
_PARAM_UN = {L.OP[k]: f for k, f in O.PARAM_UNARY.items()}


def _operand(t: torch.Tensor, spec, y0, x0, h, w) -> torch.Tensor:
    ys = torch.arange(y0, y0 + h)
    xs = torch.arange(x0, x0 + w)
    iy = (ys & spec.row_mask) + spec.row_off if spec.row_mask != -1 else ys + spec.row_off
    ix = (xs & spec.col_mask) + spec.col_off if spec.col_mask != -1 else xs + spec.col_off
    if t.shape[0] == 1:
        iy = torch.zeros_like(iy)
    if t.shape[1] == 1:
        ix = torch.zeros_like(ix)
    return t[iy][:, ix].float()


def _rnd(x, r):
    return x.to(torch.bfloat16).float() if r == L.TTLH_BF16 else x


def _values(l, args):
    """The launch's stack program over its region, with per-step rounding."""
    y0, x0, h, w = l.region
    acc, stack = None, []
    for s, spec in zip(l.prog.steps, l.operands):
        v = None
        if spec is not None:
            v = _operand(spec.ref.resolve(args).cpu(), spec, y0, x0, h, w)
        if s.form in (L.FORM_LOAD, L.FORM_PUSH):
            if s.form == L.FORM_PUSH:
                stack.append(acc)
            acc = v
        elif s.form in (L.FORM_CONST, L.FORM_PUSH_CONST):
            if s.form == L.FORM_PUSH_CONST:
                stack.append(acc)
            acc = torch.full((h, w), s.imm)
        elif s.form == L.FORM_UNARY:
            if s.op == L.OP["powi"]:
                acc = acc ** s.imm
            elif s.op in _PARAM_UN:
                acc = _PARAM_UN[s.op](acc, s.imm, s.imm2)
            else:
                acc = _TORCH_UN[s.op](acc)
        elif s.form == L.FORM_BIN:
            acc = _TORCH_BIN[s.op](acc, v)
        elif s.form == L.FORM_BIN_REV:
            acc = _TORCH_BIN[s.op](v, acc)
        elif s.form == L.FORM_BIN_IMM:
            acc = _TORCH_BIN[s.op](acc, torch.tensor(s.imm))
        elif s.form == L.FORM_BIN_IMM_REV:
            acc = _TORCH_BIN[s.op](torch.tensor(s.imm), acc)
        else:
            acc = _TORCH_BIN[s.op](stack.pop(), acc)
        acc = _rnd(acc, s.rnd)
    return acc


def run_eltwise(l: EltwiseLaunch, args):
    y0, x0, h, w = l.region
    acc = _values(l, args)
    out = l.out.resolve(args)
    out[y0:y0 + h, x0:x0 + w] = acc.to(out.dtype).to(out.device)


def run_reduce(l: ReduceLaunch, args):
    v = _values(l, args).double()
    s = l.scale
    if l.scaler is not None:
        r, c = l.scaler_at
        s *= float(l.scaler.resolve(args)[r, c])
    v = v * s
    dims = tuple(l.dims)
    fn = (lambda t, d: t.sum(d)) if l.kind == "sum" else (lambda t, d: t.amax(d))
    out = l.out.resolve(args)
    oy, ox = l.out_origin
    if dims == (0, 1):
        res = fn(v.reshape(-1), 0).reshape(1, 1)
    elif dims == (1,):
        res = fn(v, 1).reshape(-1, 1)
    else:
        res = fn(v, 0).reshape(1, -1)
    res = res.to(torch.float32).to(out.dtype)
    rh, rw = res.shape
    if l.out_pad:  # whole 32-wide result tiles, zeros beside the values
        ph = 32 if 0 in dims else rh
        pw = 32 if 1 in dims else rw
        out[oy:oy + ph, ox:ox + pw] = 0
    out[oy:oy + rh, ox:ox + rw] = res.to(out.device)


def run_matmul(l: MatmulLaunch, args):
    a, b, c = l.a.resolve(args), l.b.resolve(args), l.c.resolve(args)
    r0, r1 = l.rows
    c0, c1 = l.cols
    (ar0, ar1), (bc0, bc1) = l.operand_ranges()
    if l.b_block:  # packed block-float tiles: the oracle's integer decoders
        from oracle import bfp8 as OB
        fmt = l.b.resolve_obj(args).dtype.codec
        b = (OB.unpack_c if fmt == "bfp8" else OB.unpack4_c)(b.cpu(), a.shape[1], c.shape[1])
    ks = l.k_slice()
    c[r0:r1, c0:c1] = (a[ar0:ar1, ks].double() @ b[ks, bc0:bc1].double()).to(c.dtype)


def run_sdpa(l: SdpaLaunch, args):
    """Fused attention: the oracle's softmax(Q K^T s) V in float32 per head
    (the fused kernel keeps S, P and the row statistics in fp32), rounded
    once to the output dtype."""
    q, kt, v, y = (r.resolve(args) for r in (l.q, l.kt, l.v, l.out))
    D = q.shape[1]
    shape = (l.heads, l.seq, D)
    res = O.sdpa_ref(q.reshape(shape), kt.t().reshape(shape), v.reshape(shape), l.scale,
                     dtype=torch.float32)
    y.copy_(res.reshape(y.shape).to(y.dtype))


class _MapRef:
    def __init__(self, t):
        self.t = t

    def resolve(self, args):
        return self.t


class _MapSpec:
    """An OperandMap (kernels.OperandMap) in a launch operand's shape."""

    def __init__(self, m):
        self.ref = _MapRef(m.tensor)
        self.row_mask, self.col_mask = m.row_mask, m.col_mask
        self.row_off, self.col_off = m.row_off, m.col_off


def eltwise_cpu(prog, operands, out, region=None, stream=None):
    """CPU stand-in for ttlhip.kernels.eltwise (same arguments): the ttnn
    elementwise ops of the drop-in on the CPU test path."""
    region = region if region is not None else (0, 0, out.shape[0], out.shape[1])
    l = EltwiseLaunch(prog, [None if m is None else _MapSpec(m) for m in operands],
                      _MapRef(out), tuple(region))
    run_eltwise(l, {})


def run(plan, args):
    for l in plan.launches:
        if isinstance(l, ReduceLaunch):
            run_reduce(l, args)
        elif isinstance(l, EltwiseLaunch):
            run_eltwise(l, args)
        elif isinstance(l, SdpaLaunch):
            run_sdpa(l, args)
        elif isinstance(l, FusedMatmulLaunch):  # the product materialised, then the program
            run_matmul(l.mm, args)
            run_eltwise(l.ew, args)
        elif isinstance(l, ReduceEltwiseLaunch):  # the reductions, then the program
            for r in l.reds:
                run_reduce(r, args)
            run_eltwise(l.ew, args)
        else:
            run_matmul(l, args)
