"""Op-level CPU restatement of the simulator's tile arithmetic (test oracle).

Everything here runs torch on the CPU exactly the way tt-lang's simulator
does: one torch op per operator, every intermediate materialised in the
dtype torch promotion gives it (python/sim/block.py:870-1010 ->
python/sim/ttnnsim.py:384-452), broadcasting by torch rules over the tile
grid and inside degenerate tiles (block.py:886-920, ttnnsim.py:67-109).
Elementwise ops commute with tiling, so evaluating them on whole tensors is
element-for-element the same as the simulator's per-tile loop; the
tile-by-tile executor in sim_exec.py is the literal restatement.
"""

from __future__ import annotations

import math
from typing import Dict, Tuple

import torch

TILE = 32  # python/sim/constants.py:42-44

# Block operators (python/sim/block.py:963-1010) and the TTL elementwise op
# table (include/ttlang/Dialect/TTL/TTLElementwiseOps.def:61-82; spec
# docs/sphinx/specs/TTLangSpecification.md:683-761).
BINARY = {
    "add": torch.add,
    "sub": torch.sub,
    "mul": torch.mul,
    "div": torch.true_divide,
    "max": torch.maximum,
    "min": torch.minimum,
    "pow": torch.pow,
    "floordiv": torch.floor_divide,
    "mod": torch.remainder,
}
UNARY = {
    "exp": torch.exp,
    "log": torch.log,
    "sqrt": torch.sqrt,
    "rsqrt": torch.rsqrt,
    "tanh": torch.tanh,
    "abs": torch.abs,
    "neg": torch.neg,
    "relu": torch.relu,
    "sigmoid": torch.sigmoid,
    "recip": torch.reciprocal,
    # the spec's further math functions (TTLangSpecification.md:700-750),
    # the torch functions the spec links
    "exp2": torch.exp2,
    "expm1": torch.expm1,
    "logp1": torch.log1p,
    "sin": torch.sin,
    "cos": torch.cos,
    "tan": torch.tan,
    "asin": torch.asin,
    "acos": torch.acos,
    "atan": torch.atan,
    "asinh": torch.asinh,
    "acosh": torch.acosh,
    "atanh": torch.atanh,
    "gelu": lambda t: gelu_exact(t),
    "silu": torch.nn.functional.silu,
    "softsign": torch.nn.functional.softsign,
    "hardsigmoid": torch.nn.functional.hardsigmoid,
}


def gelu_exact(x: torch.Tensor) -> torch.Tensor:
    """GELU x / 2 (1 + erf(x / sqrt 2)) evaluated as x / 2 erfc(-x / sqrt 2) in
    float64 and rounded (via fp32) to x's dtype.  torch's CPU kernel (the
    function the spec links) cancels in 1 + erf for x << 0 and is up to 32
    bf16 ulp off at x = -5, so the oracle takes the mathematical value."""
    d = x.double()
    return (0.5 * d * torch.erfc(-d / math.sqrt(2.0))).to(torch.float32).to(x.dtype)


def selu_p(x: torch.Tensor, scale: float, alpha: float) -> torch.Tensor:
    """scale (max(x, 0) + min(alpha (exp(x) - 1), 0)) in fp32, rounded once
    (torch.nn.SELU with the spec's explicit parameters)."""
    f = x.float()
    r = scale * (torch.clamp(f, min=0) + torch.clamp(alpha * torch.expm1(f), max=0))
    return r.to(x.dtype)


# parameterised unary functions: name -> f(x, p0, p1)
PARAM_UNARY = {
    "elu": lambda x, a, _b: torch.nn.functional.elu(x, alpha=a),
    "celu": lambda x, a, _b: torch.nn.functional.celu(x, alpha=a),
    "selu": selu_p,
    "softplus": lambda x, beta, thr: torch.nn.functional.softplus(x, beta=beta, threshold=thr),
}


def eval_expr(e, env: Dict[str, torch.Tensor]) -> torch.Tensor:
    """Evaluates a nested-tuple expression with the simulator's semantics.

    e is ("leaf", name) | ("const", value) | ("powi", x, n) | (unary, x) |
    (binary, x, y).  Leaves are CPU tensors (whole operands, already shaped
    so torch broadcasting reproduces the block broadcast), constants are
    Python scalars (torch keeps the tensor dtype for tensor-op-scalar).
    """
    tag = e[0]
    if tag == "leaf":
        return env[e[1]]
    if tag == "const":
        return e[1]
    if tag == "powi":
        return eval_expr(e[1], env) ** int(e[2])
    if tag in UNARY:
        return UNARY[tag](eval_expr(e[1], env))
    if tag in BINARY:
        a, b = eval_expr(e[1], env), eval_expr(e[2], env)
        if not isinstance(a, torch.Tensor):
            a = torch.tensor(a, dtype=b.dtype)
        return BINARY[tag](a, b)
    raise ValueError(f"unknown op {tag!r}")


def store_acc(slot_values):
    """store(acc=True) sequence on one reserved block slot
    (python/sim/block.py:850-864): the first store assigns, later ones add in
    the dtype of the stored tensors."""
    acc = None
    for v in slot_values:
        acc = v if acc is None else acc + v
    return acc


def tile_matmul_sim(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """C = A @ B the way the simulator runs singlecore/multicore_matmul.py:
    for every output tile, the K tile products A(m,k) @ B(k,n) are torch
    matmuls of 32x32 tiles in the inputs' dtype (block.py:1012-1013 ->
    ttnnsim.py:454-459), summed by store(acc=True) in that dtype, first
    store assigning (block.py:850-864), k in ascending order."""
    M, K = a.shape
    K2, N = b.shape
    assert K == K2 and M % TILE == 0 and N % TILE == 0 and K % TILE == 0
    mt, kt, nt = M // TILE, K // TILE, N // TILE
    at = a.reshape(mt, TILE, kt, TILE).permute(0, 2, 1, 3).contiguous()  # [mt, kt, 32, 32]
    bt = b.reshape(kt, TILE, nt, TILE).permute(0, 2, 1, 3).contiguous()  # [kt, nt, 32, 32]
    acc = None
    for k in range(kt):
        # [mt, 1, 32, 32] @ [1, nt, 32, 32] -> [mt, nt, 32, 32]: one tile matmul per pair
        p = torch.matmul(at[:, k].unsqueeze(1).expand(mt, nt, TILE, TILE).reshape(-1, TILE, TILE),
                         bt[k].unsqueeze(0).expand(mt, nt, TILE, TILE).reshape(-1, TILE, TILE))
        p = p.reshape(mt, nt, TILE, TILE)
        acc = p if acc is None else acc + p
    return acc.permute(0, 2, 1, 3).reshape(M, N)


def matmul_fp64(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Exact-as-possible reference product (float64 on the CPU)."""
    return a.double() @ b.double()


def sdpa_ref(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
             causal: bool = False, dtype=torch.float64) -> torch.Tensor:
    """softmax(Q K^T * scale) V on the CPU in `dtype` (default float64).

    Attention is not in the reference; this composes the spec's ops
    (@, exp, reduce_max, reduce_sum, recip, broadcast:
    docs/sphinx/specs/TTLangSpecification.md:693-761) in the standard
    max-subtracted form."""
    qd, kd, vd = q.to(dtype), k.to(dtype), v.to(dtype)
    s = torch.matmul(qd, kd.transpose(-1, -2).contiguous()) * scale
    if causal:
        S = s.shape[-1]
        mask = torch.ones(S, S, dtype=torch.bool).triu(1)
        s = s.masked_fill(mask, float("-inf"))
    m = s.amax(dim=-1, keepdim=True)
    p = torch.exp(s - m)
    l = p.sum(dim=-1, keepdim=True)
    return torch.matmul(p / l, vd)


# ---- tilized element order ------------------------------------------------
# The storage order of a TILE_LAYOUT tensor (which the reference's compiled
# path requires, python/ttl/ttl_api.py:489-506; the tilize itself is in
# un-vendored tt-metal): 32x32 tiles row-major over the tile grid, each tile
# four 16x16 faces (rows 0-15 / cols 0-15, rows 0-15 / cols 16-31, rows 16-31 /
# cols 0-15, rows 16-31 / cols 16-31), each face row-major - the face split of
# the bfloat8_b tiles (oracle/bfp8_ref.c).

def tilize_ref(x: torch.Tensor) -> torch.Tensor:
    """[R, C] (multiples of 32) -> 1-D tensor in tilized order."""
    r, c = x.shape
    t = x.reshape(r // TILE, 2, 16, c // TILE, 2, 16)  # (tr, fr, i, tc, fc, j)
    return t.permute(0, 3, 1, 4, 2, 5).reshape(-1)


def untilize_ref(d: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    t = d.reshape(rows // TILE, cols // TILE, 2, 2, 16, 16)  # (tr, tc, fr, fc, i, j)
    return t.permute(0, 2, 4, 1, 3, 5).reshape(rows, cols)


# ---- seeded inputs shared by the CPU oracle and the GPU path --------------

def seeded(shape: Tuple[int, ...], dist: str, seed: int, dtype=torch.bfloat16,
           lo: float = -1.0, hi: float = 1.0, std: float = 1.0) -> torch.Tensor:
    """Inputs of the benchmark configs, generated on the CPU from a seed so
    both sides see bit-identical values: "uniform" = U[lo, hi), "normal" =
    N(0, std^2); rounded (RNE) to `dtype`."""
    g = torch.Generator().manual_seed(seed)
    if dist == "uniform":
        x = torch.rand(shape, generator=g, dtype=torch.float32) * (hi - lo) + lo
    elif dist == "normal":
        x = torch.randn(shape, generator=g, dtype=torch.float32) * std
    else:
        raise ValueError(dist)
    return x.to(dtype)


def bf16_ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """|ulp distance| between two bf16 tensors (ordered-integer metric)."""
    def ordered(t):
        i = t.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -32768 - i, i)
    return (ordered(a) - ordered(b)).abs()
