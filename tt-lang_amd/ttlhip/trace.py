"""Vectorised tracer of tt-lang thread bodies.

The reference executes a kernel's three threads (reader, compute, writer) per
core: the simulator interleaves them as Python generators, one circular-buffer
operation at a time (python/sim/program.py:363-647); the compiler lowers them
to Tensix code (python/ttl/ttl_api.py:818-1122).  Here a thread body runs once
per core on the host, at trace time, to record *what* it moves and computes;
the MI355X kernels then do the work grid-wide.

Vectorisation.  Each `for v in range(...)` loop in a thread body is rewritten
(AST) to iterate a generator that yields once, binding `v` to a VInt: a numpy
array of all the loop's values on its own axis (one axis per nesting level).
Index arithmetic then computes every iteration at once, so a 128^3-tile
matmul traces in milliseconds instead of 2 M Python steps.  Loops whose body
carries a value from one iteration to the next, exits early, or assigns to
attributes / subscripts are left as ordinary loops.  Anything a VInt cannot
do (branching on it, using it as a Python int) raises Devectorize, and the
thread is traced again with every loop scalar.

What is recorded per thread is a tree of loop nodes whose leaves are events
(reserve / push / wait / pop on a CB, copies, stores).  The n-th block a
thread reserves or waits on a CB gets its index from the tree (count of
earlier events of that kind in program order), vectorised over the loop axes.
"""

from __future__ import annotations

import ast
import inspect
import itertools
import textwrap
import types
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

MAXD = 8  # loop axes available for vectorisation
TILE = 32


class Devectorize(Exception):
    """A thread body used a loop variable in a way that needs scalar values."""


class TraceError(ValueError):
    """The kernel program violates a tt-lang rule (shape mismatch, CB misuse)."""


_loop_ids = itertools.count(1)


# ---------------------------------------------------------------------------
# vector integers


def _as_array(x):
    if isinstance(x, VInt):
        return x.v, x.loops
    if isinstance(x, (bool, np.bool_)):
        return np.int64(int(x)), frozenset()
    if isinstance(x, (int, np.integer)):
        return np.int64(int(x)), frozenset()
    raise TypeError(f"unsupported operand {type(x).__name__} for tile-index arithmetic")


class VInt:
    """All values of an integer expression over the enclosing vectorised loops."""

    __slots__ = ("v", "loops")

    def __init__(self, v, loops: frozenset):
        self.v = np.asarray(v, dtype=np.int64)
        self.loops = loops

    def _bin(self, other, fn, rev=False):
        try:
            b, lb = _as_array(other)
        except TypeError:
            return NotImplemented
        a, la = self.v, self.loops
        r = fn(b, a) if rev else fn(a, b)
        return VInt(r, la | lb)

    def __add__(self, o): return self._bin(o, np.add)
    def __radd__(self, o): return self._bin(o, np.add, True)
    def __sub__(self, o): return self._bin(o, np.subtract)
    def __rsub__(self, o): return self._bin(o, np.subtract, True)
    def __mul__(self, o): return self._bin(o, np.multiply)
    def __rmul__(self, o): return self._bin(o, np.multiply, True)
    def __floordiv__(self, o): return self._bin(o, np.floor_divide)
    def __rfloordiv__(self, o): return self._bin(o, np.floor_divide, True)
    def __mod__(self, o): return self._bin(o, np.mod)
    def __rmod__(self, o): return self._bin(o, np.mod, True)
    def __neg__(self): return VInt(-self.v, self.loops)
    def __pos__(self): return self

    def _cmp(self, *_):
        raise Devectorize("comparison of a vectorised loop variable")

    __lt__ = __le__ = __gt__ = __ge__ = __eq__ = __ne__ = _cmp

    def __bool__(self):
        raise Devectorize("truth value of a vectorised loop variable")

    def __index__(self):
        raise Devectorize("vectorised loop variable used as a Python int")

    __int__ = __index__
    __hash__ = None  # type: ignore[assignment]

    def __format__(self, spec):
        return format(self.v.ravel().tolist(), spec) if spec == "" else str(self.v.ravel().tolist())

    def __repr__(self):
        return f"VInt({self.v.ravel().tolist()})"


def is_index(k) -> bool:
    return isinstance(k, (int, np.integer, slice, VInt))


def to_scalar(x) -> int:
    if isinstance(x, VInt):
        raise Devectorize("vectorised value where a scalar is required")
    return int(x)


# ---------------------------------------------------------------------------
# loop tree and events


class LoopNode:
    __slots__ = ("id", "depth", "n", "children", "parent")

    def __init__(self, depth: int, n: int, parent: Optional["LoopNode"]):
        self.id = next(_loop_ids)
        self.depth = depth
        self.n = n
        self.children: List[Any] = []
        self.parent = parent

    def enclosing(self) -> List["LoopNode"]:
        out, p = [], self
        while p is not None and p.depth >= 0:
            out.append(p)
            p = p.parent
        return out[::-1]


class Event:
    """One CB / copy / store operation, recorded once per vectorised instance."""

    __slots__ = ("kind", "cb", "node", "index", "data", "domain")

    def __init__(self, kind: str, cb, node: LoopNode, data=None):
        self.kind = kind          # reserve | push | wait | pop | copy_in | copy_out | store
        self.cb = cb
        self.node = node
        self.index = None         # block index (reserve / wait), set after tracing
        self.data = data or {}
        self.domain = tuple(n for n in node.enclosing())  # vectorised loops around it

    def domain_shape(self) -> Tuple[int, ...]:
        shape = [1] * MAXD
        for n in self.domain:
            shape[n.depth] = n.n
        return tuple(shape)


class TraceContext:
    """State of one thread trace on one core."""

    def __init__(self, core: int, grid: Tuple[int, ...], thread, scalar: bool):
        self.core = core
        self.grid = grid
        self.thread = thread
        self.scalar = scalar
        self.root = LoopNode(-1, 1, None)
        self.cur = self.root
        self.pending_reserve: Dict[int, Any] = {}
        self.pending_wait: Dict[int, Any] = {}

    def add(self, ev: Event) -> Event:
        self.cur.children.append(ev)
        return ev

    def check_loops(self, x, what: str) -> None:
        """A VInt recorded in an event must only vary over loops that enclose it."""
        if isinstance(x, VInt):
            live = set()
            p = self.cur
            while p is not None and p.depth >= 0:
                live.add(p.id)
                p = p.parent
            if not x.loops <= live:
                raise Devectorize(f"{what} depends on a loop that has already ended")


_ctx: Optional[TraceContext] = None
_kernel_grid: Optional[Tuple[int, ...]] = None


def current() -> Optional[TraceContext]:
    return _ctx


def vrange(*args):
    """Replacement for `range` in traced loops (see module docstring)."""
    ctx = _ctx
    ints = [to_scalar(a) for a in args]
    r = range(*ints)
    if ctx is None or ctx.scalar or ctx.cur.depth + 1 >= MAXD:
        yield from r
        return
    if len(r) == 0:
        return
    node = LoopNode(ctx.cur.depth + 1, len(r), ctx.cur)
    ctx.cur.children.append(node)
    ctx.cur = node
    try:
        shape = [1] * MAXD
        shape[node.depth] = len(r)
        vals = (np.arange(len(r), dtype=np.int64) * r.step + r.start).reshape(shape)
        yield VInt(vals, frozenset([node.id]))
    finally:
        ctx.cur = node.parent


# ---------------------------------------------------------------------------
# AST rewrite of thread bodies


class _LoopRewriter(ast.NodeTransformer):
    def visit_For(self, node: ast.For):
        self.generic_visit(node)
        if not (isinstance(node.iter, ast.Call) and isinstance(node.iter.func, ast.Name)
                and node.iter.func.id == "range" and not node.iter.keywords
                and isinstance(node.target, ast.Name) and not node.orelse):
            return node
        if not _vectorisable_body(node):
            return node
        node.iter = ast.Call(func=ast.Name(id="__ttl_vrange__", ctx=ast.Load()),
                             args=node.iter.args, keywords=[])
        return node


def _vectorisable_body(loop: ast.For) -> bool:
    """True when every iteration of `loop` is independent of the others."""
    assigned: set = set()
    for n in ast.walk(loop):
        if isinstance(n, (ast.Break, ast.Continue, ast.Return, ast.Yield, ast.YieldFrom,
                          ast.Global, ast.Nonlocal, ast.AugAssign)):
            return False
        if isinstance(n, (ast.Assign, ast.AnnAssign)):
            targets = n.targets if isinstance(n, ast.Assign) else [n.target]
            for t in targets:
                for tn in ast.walk(t):
                    if isinstance(tn, (ast.Attribute, ast.Subscript)):
                        return False
                    if isinstance(tn, ast.Name):
                        assigned.add(tn.id)
        if isinstance(n, ast.NamedExpr):
            assigned.add(n.target.id)
    # a name read before it is (re)assigned in the body carries a value across
    # iterations
    seen: set = set()

    def walk_stmts(stmts) -> bool:
        for st in stmts:
            if isinstance(st, (ast.Assign, ast.AnnAssign)):
                val = st.value
                if val is not None and not reads_ok(val):
                    return False
                targets = st.targets if isinstance(st, ast.Assign) else [st.target]
                for t in targets:
                    for tn in ast.walk(t):
                        if isinstance(tn, ast.Name):
                            seen.add(tn.id)
            elif isinstance(st, ast.For):
                if not reads_ok(st.iter):
                    return False
                seen.add(getattr(st.target, "id", ""))
                if not walk_stmts(st.body):
                    return False
            elif isinstance(st, ast.With):
                for it in st.items:
                    if not reads_ok(it.context_expr):
                        return False
                    if it.optional_vars is not None:
                        for tn in ast.walk(it.optional_vars):
                            if isinstance(tn, ast.Name):
                                seen.add(tn.id)
                if not walk_stmts(st.body):
                    return False
            elif isinstance(st, ast.If):
                if not reads_ok(st.test) or not walk_stmts(st.body) or not walk_stmts(st.orelse):
                    return False
            else:
                if not reads_ok(st):
                    return False
        return True

    def reads_ok(node) -> bool:
        for n in ast.walk(node):
            if isinstance(n, ast.Name) and isinstance(n.ctx, ast.Load):
                if n.id in assigned and n.id not in seen:
                    return False
        return True

    seen.add(loop.target.id)
    return walk_stmts(loop.body)


def rewrite_thread(func: types.FunctionType) -> types.FunctionType:
    """Returns `func` with its range loops rewritten to vrange (same closure)."""
    try:
        src = textwrap.dedent(inspect.getsource(func))
    except (OSError, TypeError):
        return func
    tree = ast.parse(src)
    ast.increment_lineno(tree, func.__code__.co_firstlineno - 1)
    fdef = tree.body[0]
    if not isinstance(fdef, (ast.FunctionDef, ast.AsyncFunctionDef)):
        return func
    fdef.decorator_list = []
    fdef = _LoopRewriter().visit(fdef)
    freevars = func.__code__.co_freevars
    # wrap in a factory so the rewritten function closes over the same names
    factory = ast.FunctionDef(
        name="__ttl_factory__",
        args=ast.arguments(posonlyargs=[], args=[ast.arg(arg=v) for v in freevars],
                           vararg=None, kwonlyargs=[], kw_defaults=[], kwarg=None, defaults=[]),
        body=[fdef, ast.Return(value=ast.Name(id=fdef.name, ctx=ast.Load()))],
        decorator_list=[], returns=None)
    mod = ast.Module(body=[factory], type_ignores=[])
    ast.fix_missing_locations(mod)
    filename = inspect.getsourcefile(func) or "<ttl-thread>"
    code = compile(mod, filename, "exec")
    fcode = next(c for c in code.co_consts if isinstance(c, types.CodeType))
    inner = next(c for c in fcode.co_consts if isinstance(c, types.CodeType)
                 and c.co_name == func.__name__)
    cells = dict(zip(freevars, func.__closure__ or ()))
    closure = tuple(cells[n] for n in inner.co_freevars)
    g = dict(func.__globals__)
    g["__ttl_vrange__"] = vrange
    new = types.FunctionType(inner, g, func.__name__, func.__defaults__, closure)
    return new


# ---------------------------------------------------------------------------
# tensor slices (tile-coordinate views)


class TensorSlice:
    """`tensor[rows, cols]` in tile coordinates (python/sim/tensoraccessor.py:85-159):
    ints become length-1 ranges, slices need explicit start and stop, no step."""

    __slots__ = ("tensor", "r0", "nr", "c0", "nc")

    def __init__(self, tensor, r0, nr: int, c0, nc: int):
        self.tensor, self.r0, self.nr, self.c0, self.nc = tensor, r0, nr, c0, nc

    @staticmethod
    def _axis(k, name: str):
        if isinstance(k, slice):
            if k.start is None:
                raise ValueError(f"Slice {name} must have explicit start value, got {k}")
            if k.stop is None:
                raise ValueError(f"Slice {name} must have explicit stop value, got {k}")
            if k.step is not None:
                raise ValueError(f"Slice {name} must not have step value, got {k}")
            n = k.stop - k.start
            if isinstance(n, VInt):
                vals = np.unique(n.v)
                if vals.size != 1:
                    raise Devectorize(f"slice {name} length varies across iterations")
                n = int(vals[0])
            return k.start, int(n)
        return k, 1

    @classmethod
    def from_key(cls, tensor, key):
        r0, nr = cls._axis(key[0], "row")
        c0, nc = cls._axis(key[1], "col")
        return cls(tensor, r0, nr, c0, nc)

    def shape_in_tiles(self) -> Tuple[int, int]:
        """Tile shape with size-1 tensor dimensions kept as 1
        (python/sim/copyhandlers.py:103-131)."""
        h, w = self.tensor.shape
        return (1 if h == 1 else self.nr, 1 if w == 1 else self.nc)

    def check_bounds(self) -> None:
        h, w = self.tensor.shape
        for start, n, dim, nm in ((self.r0, self.nr, h, "row"), (self.c0, self.nc, w, "col")):
            tiles = 1 if dim == 1 else dim // TILE
            arr = start.v if isinstance(start, VInt) else np.int64(start)
            lo, hi = int(np.min(arr)), int(np.max(arr)) + n
            if lo < 0 or hi > tiles:
                raise TraceError(f"{nm} tiles [{lo}, {hi}) out of range for a tensor of "
                                 f"{tiles} {nm} tiles (shape {tuple(self.tensor.shape)})")

    @property
    def _tensor(self) -> torch.Tensor:
        """Element view, for eager (non-kernel) use with integer indices."""
        r0, c0 = to_scalar(self.r0), to_scalar(self.c0)
        t = self.tensor._tensor
        return t[r0 * TILE:(r0 + self.nr) * TILE, c0 * TILE:(c0 + self.nc) * TILE]

    def to_torch(self) -> torch.Tensor:
        return self._tensor.detach().cpu()

    @property
    def shape(self):
        return tuple(self._tensor.shape)


# ---------------------------------------------------------------------------
# helpers used by the resolver: block indices from the loop tree


def _per_iter_counts(node: LoopNode, memo: Dict) -> Dict[Tuple[int, str], int]:
    """Number of events of each (cb id, kind) in one execution of `node`'s body."""
    if node.id in memo:
        return memo[node.id]
    c: Dict[Tuple[int, str], int] = {}
    for ch in node.children:
        if isinstance(ch, Event):
            if ch.kind in ("reserve", "wait"):
                k = (ch.cb.id, ch.kind)
                c[k] = c.get(k, 0) + 1
        else:
            for k, v in _per_iter_counts(ch, memo).items():
                c[k] = c.get(k, 0) + ch.n * v
    memo[node.id] = c
    return c


def assign_indices(root: LoopNode) -> Dict[Tuple[int, str], int]:
    """Sets Event.index (the block number within its CB, as an array over the
    event's loop axes) for every reserve / wait; returns total counts."""
    memo: Dict = {}

    def walk(node: LoopNode, base: Dict[Tuple[int, str], Any]):
        running: Dict[Tuple[int, str], int] = {}
        for ch in node.children:
            if isinstance(ch, Event):
                if ch.kind in ("reserve", "wait"):
                    k = (ch.cb.id, ch.kind)
                    ch.index = base.get(k, np.int64(0)) + running.get(k, 0)
                    running[k] = running.get(k, 0) + 1
            else:
                per = _per_iter_counts(ch, memo)
                shape = [1] * MAXD
                shape[ch.depth] = ch.n
                it = np.arange(ch.n, dtype=np.int64).reshape(shape)
                child_base = {}
                for k, v in per.items():
                    child_base[k] = base.get(k, np.int64(0)) + running.get(k, 0) + it * v
                walk(ch, child_base)
                for k, v in per.items():
                    running[k] = running.get(k, 0) + ch.n * v
        return running

    return walk(root, {})


def iter_events(node: LoopNode):
    for ch in node.children:
        if isinstance(ch, Event):
            yield ch
        else:
            yield from iter_events(ch)


def broadcast_to_domain(x, shape: Tuple[int, ...]) -> np.ndarray:
    if isinstance(x, VInt):
        x = x.v
    return np.broadcast_to(np.asarray(x, dtype=np.int64), shape)
