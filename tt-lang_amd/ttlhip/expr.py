"""Elementwise tile-expression IR and its compiler to the libttlhip stack program.

An expression is the per-element function a compute thread stores into an
output block, e.g. ``exp(a + b_row) * c``.  Leaves are input operands (tiles
streamed from a tensor), constants, and inner nodes are the TTL elementwise
ops (include/ttlang/Dialect/TTL/TTLElementwiseOps.def:61-82, plus the
simulator's Block operators ``+ - * / // % **``, python/sim/block.py:963-1010).

Every node carries the torch dtype the simulator would materialise it in
(torch type promotion; the simulator rounds every intermediate tile to that
dtype, python/sim/ttnnsim.py:384-452).  The compiler emits one stack-machine
step per node and rounds after each step whose node dtype is bfloat16, which
reproduces that rounding exactly for + - * / (one fp32 op, one RNE rounding).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Tuple

import torch

from . import _lib as L


class Expr:
    dtype: torch.dtype

    # structural key: equal keys <=> same program (leaf identity by slot id)
    def key(self) -> Tuple:
        raise NotImplementedError

    def leaves(self) -> List["Leaf"]:
        out: List[Leaf] = []
        self._collect(out)
        return out

    def _collect(self, out: List["Leaf"]) -> None:
        pass


@dataclass(eq=False)
class Leaf(Expr):
    """An input operand; `ref` is whatever the caller uses to address it."""

    ref: Any
    dtype: torch.dtype

    def key(self) -> Tuple:
        return ("leaf", id(self), str(self.dtype))

    def _collect(self, out: List["Leaf"]) -> None:
        out.append(self)


@dataclass(eq=False)
class Const(Expr):
    value: float
    dtype: torch.dtype = torch.float32

    def key(self) -> Tuple:
        return ("const", float(self.value))


@dataclass(eq=False)
class Unary(Expr):
    op: str
    x: Expr
    dtype: torch.dtype
    imm: float = 0.0
    imm2: float = 0.0

    def key(self) -> Tuple:
        return ("un", self.op, self.imm, self.imm2, str(self.dtype), self.x.key())

    def _collect(self, out: List["Leaf"]) -> None:
        self.x._collect(out)


@dataclass(eq=False)
class Binary(Expr):
    op: str
    a: Expr
    b: Expr
    dtype: torch.dtype

    def key(self) -> Tuple:
        return ("bin", self.op, str(self.dtype), self.a.key(), self.b.key())

    def _collect(self, out: List["Leaf"]) -> None:
        self.a._collect(out)
        self.b._collect(out)


def promote(a: torch.dtype, b: torch.dtype) -> torch.dtype:
    return torch.promote_types(a, b)


def _rnd(dt: torch.dtype) -> int:
    return L.TTLH_BF16 if dt == torch.bfloat16 else L.TTLH_F32


@dataclass
class Step:
    form: int
    op: int = 0
    rnd: int = L.TTLH_F32
    imm: float = 0.0
    leaf: Optional[Leaf] = None  # operand owned by this step
    imm2: float = 0.0


@dataclass
class StackProgram:
    steps: List[Step] = field(default_factory=list)
    max_depth: int = 0

    def leaves(self) -> List[Optional[Leaf]]:
        return [s.leaf for s in self.steps]


def compile_expr(e: Expr) -> StackProgram:
    """Compiles an expression tree into libttlhip's stack-machine program.

    Leaf operands are fused into the consuming binary step (forms BIN /
    BIN_REV) so a chain such as exp(a + b) * c needs no stack traffic; only a
    node whose two children are both computed values pushes.
    """
    prog = StackProgram()
    depth = 0

    def emit(step: Step, delta: int) -> None:
        nonlocal depth
        depth += delta
        prog.max_depth = max(prog.max_depth, depth)
        prog.steps.append(step)

    def simple(n: Expr) -> bool:
        return isinstance(n, (Leaf, Const))

    def gen(n: Expr) -> None:
        if isinstance(n, Leaf):
            # a bare leaf keeps its value; round only if promotion narrows
            if depth == 0:
                emit(Step(L.FORM_LOAD, leaf=n, rnd=L.TTLH_F32), 1)
            else:
                emit(Step(L.FORM_PUSH, leaf=n, rnd=L.TTLH_F32), 1)
        elif isinstance(n, Const):
            form = L.FORM_CONST if depth == 0 else L.FORM_PUSH_CONST
            emit(Step(form, imm=float(n.value), rnd=_rnd(n.dtype)), 1)
        elif isinstance(n, Unary):
            if n.op not in L.UNARY_OPS:
                raise NotImplementedError(f"unsupported unary tile op {n.op!r}")
            gen(n.x)
            emit(Step(L.FORM_UNARY, op=L.OP[n.op], imm=n.imm, imm2=n.imm2, rnd=_rnd(n.dtype)), 0)
        elif isinstance(n, Binary):
            if n.op not in L.BINARY_OPS:
                raise NotImplementedError(f"unsupported binary tile op {n.op!r}")
            op = L.OP[n.op]
            r = _rnd(n.dtype)
            if isinstance(n.b, Leaf):
                gen(n.a)
                emit(Step(L.FORM_BIN, op=op, leaf=n.b, rnd=r), 0)
            elif isinstance(n.b, Const):
                gen(n.a)
                emit(Step(L.FORM_BIN_IMM, op=op, imm=float(n.b.value), rnd=r), 0)
            elif isinstance(n.a, Leaf):
                gen(n.b)
                emit(Step(L.FORM_BIN_REV, op=op, leaf=n.a, rnd=r), 0)
            elif isinstance(n.a, Const):
                gen(n.b)
                emit(Step(L.FORM_BIN_IMM_REV, op=op, imm=float(n.a.value), rnd=r), 0)
            else:
                gen(n.a)
                gen(n.b)
                emit(Step(L.FORM_BIN_POP, op=op, rnd=r), -1)
        else:
            raise TypeError(f"not an expression node: {n!r}")

    gen(e)
    if len(prog.steps) > L.TTLH_MAX_INSTR:
        raise NotImplementedError(
            f"fused tile expression needs {len(prog.steps)} steps; the kernel takes at most "
            f"{L.TTLH_MAX_INSTR}"
        )
    if prog.max_depth > L.TTLH_MAX_STACK:
        raise NotImplementedError(
            f"fused tile expression needs a stack of {prog.max_depth}; the kernel holds "
            f"{L.TTLH_MAX_STACK}"
        )
    return prog


def structure_key(e: Expr, leaf_ids: Dict[int, int]) -> Tuple:
    """Key of an expression up to leaf identity: leaves are numbered by first
    appearance, so two trees with the same shape / ops / dtypes and the same
    leaf-sharing pattern get the same key."""
    if isinstance(e, Leaf):
        i = leaf_ids.setdefault(id(e), len(leaf_ids))
        return ("L", i, str(e.dtype))
    if isinstance(e, Const):
        return ("C", float(e.value), str(e.dtype))
    if isinstance(e, Unary):
        return ("U", e.op, e.imm, e.imm2, str(e.dtype), structure_key(e.x, leaf_ids))
    if isinstance(e, Binary):
        return ("B", e.op, str(e.dtype), structure_key(e.a, leaf_ids), structure_key(e.b, leaf_ids))
    raise TypeError(e)
