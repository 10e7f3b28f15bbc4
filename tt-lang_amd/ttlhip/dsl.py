"""tt-lang DSL objects for the MI355X backend: kernel, CBs, blocks, copy, math.

Semantics follow the reference simulator, which is the only executable
definition of the language here:
  kernel / grid / core / grid_size        python/sim/kernel.py:89-291
  circular buffers (reserve/push/wait/pop)  python/sim/cb.py:158-510
  copy between tensors and blocks           python/sim/copy.py:160, copyhandlers.py:295-380
  block expressions and store(acc)          python/sim/block.py:805-1013
  ttl.math.broadcast                        python/sim/math.py:20-106
plus the elementwise functions of the TTL op table
(include/ttlang/Dialect/TTL/TTLElementwiseOps.def:61-82) as ttl.math.<op>.

Nothing here computes on data: inside a kernel every call records what the
thread does (see trace.py); the recorded program becomes GPU launches
(plan.py).
"""

from __future__ import annotations

import inspect
import itertools
import re
import os
import sys
import types
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from . import trace as T
from .trace import Event, TensorSlice, TraceError, VInt

TILE_SHAPE = (32, 32)
MAX_CBS = 32  # python/sim/constants.py

_cb_ids = itertools.count()


# ---------------------------------------------------------------------------
# kernel context: grid / core


class _KernelState:
    def __init__(self, grid: Tuple[int, ...]):
        self.grid = grid
        self.threads: List["ThreadTemplate"] = []
        self.cbs: List["CircularBuffer"] = []
        # thread order given by an explicit Program(compute, dm0, dm1)()
        self.program_order: Optional[List["ThreadTemplate"]] = None


_kstate: Optional[_KernelState] = None
# grid of the most recent kernel body run in this process
_last_grid: Optional[Tuple[int, ...]] = None


def _grid() -> Tuple[int, ...]:
    """Inside a kernel its grid.  Outside one, the grid of the last kernel
    called, as the compiler's module-level grid (python/ttl/operators.py:36-47,
    read back by its hardware tests after a call, test/python/test_multicore.py:
    146-149); before any kernel, the simulator's error (python/sim/kernel.py:
    110-118)."""
    ctx = T.current()
    if ctx is not None:
        return ctx.grid
    if _kstate is not None:
        return _kstate.grid
    if _last_grid is not None:
        return _last_grid
    raise RuntimeError("grid not available - function must be called within a kernel context")


def grid_size(dims: int = 2):
    """Grid shape in `dims` dimensions: trailing dimensions flattened when fewer
    are asked for, padded with 1s when more are (python/sim/kernel.py:89-152)."""
    if dims <= 0:
        raise ValueError(f"dims must be positive, got {dims}")
    g = tuple(_grid())
    if dims == len(g):
        res = g
    elif dims < len(g):
        tail = int(np.prod(g[dims - 1:]))
        res = tuple(g[:dims - 1]) + (tail,)
    else:
        res = g + (1,) * (dims - len(g))
    return res[0] if dims == 1 else res


def core(dims: int = 2):
    """Coordinates of the current core: row-major decomposition of the linear
    core id over the grid; leading dimensions flattened when fewer are asked
    for, zeros appended when more are (python/sim/kernel.py:155-199)."""
    ctx = T.current()
    if ctx is None:
        raise RuntimeError("core not available - function must be called within Program context")
    g = tuple(ctx.grid)
    cid = ctx.core
    coords = []
    for s in reversed(g):
        coords.append(cid % s)
        cid //= s
    coords.reverse()
    if dims < len(coords):
        flat = coords[0]
        for i in range(1, len(coords) - dims + 1):
            flat = flat * g[i] + coords[i]
        coords = [flat] + coords[len(coords) - dims + 1:]
    while len(coords) < dims:
        coords.append(0)
    return coords[0] if dims == 1 else tuple(coords)


def flatten_core_index(core_coord) -> int:
    if isinstance(core_coord, (int, np.integer)):
        return int(core_coord)
    g = _grid()
    c = list(core_coord)
    lin = c[0]
    for i in range(1, len(c)):
        lin = lin * g[i] + c[i]
    return int(lin)


# ---------------------------------------------------------------------------
# threads


class ThreadTemplate:
    def __init__(self, func: types.FunctionType, kind: str):
        self.func = func
        self.kind = kind  # "compute" | "dm"
        self.__name__ = func.__name__
        self.__wrapped__ = func
        self._rewritten: Optional[types.FunctionType] = None

    def rewritten(self) -> types.FunctionType:
        if self._rewritten is None:
            self._rewritten = T.rewrite_thread(self.func)
        return self._rewritten

    def __call__(self, *a, **k):
        raise RuntimeError(f"thread {self.__name__} runs only as part of a ttl.kernel")


def _register(t: ThreadTemplate) -> ThreadTemplate:
    if _kstate is None:
        raise RuntimeError("ttl.compute / ttl.datamovement must be used inside a ttl.kernel body")
    _kstate.threads.append(t)
    return t


class _ProgramCall:
    def __init__(self, funcs: Tuple[Any, ...]):
        self.funcs = funcs

    def __call__(self, *args: Any, **kwargs: Any) -> None:
        if _kstate is None:
            raise RuntimeError("Program(...)() is only valid inside a ttl.kernel body")
        if len(self.funcs) != 3:
            raise ValueError(f"Kernel must define exactly 3 threads (compute, dm0, dm1), got "
                             f"{len(self.funcs)}")
        for f in self.funcs:
            if not isinstance(f, ThreadTemplate) or f not in _kstate.threads:
                raise ValueError("Program() takes the ttl.compute / ttl.datamovement functions "
                                 "defined in this kernel body")
        _kstate.program_order = list(self.funcs)


def Program(*funcs: Any, grid: Any = None) -> _ProgramCall:
    """Explicit thread list of a kernel body, `return Program(compute, dm0,
    dm1, grid=grid)()` (python/sim/program.py:100-255): fixes which data
    movement thread is dm0 / dm1; the kernel still runs when the body
    returns (on the grid the ttl.kernel decorator resolved)."""
    return _ProgramCall(funcs)


def compute():
    def deco(func):
        return _register(ThreadTemplate(func, "compute"))
    return deco


def datamovement():
    def deco(func):
        return _register(ThreadTemplate(func, "dm"))
    return deco


# ---------------------------------------------------------------------------
# circular buffers and blocks


def compute_dtype(dtype):
    """The torch dtype block arithmetic uses for a CB element type: itself,
    or bfloat16 for a block-float format (ttnn.bfloat8_b)."""
    return getattr(dtype, "compute_dtype", dtype)


class CircularBuffer:
    """A CB of `shape` tiles per block and `shape[0]*shape[1]*buffer_factor`
    tiles of capacity (python/sim/cb.py:158-300).  On the MI355X the ring
    is not materialised: blocks become tile coordinates of the grid-wide
    kernels (streaming through VGPRs / LDS)."""

    def __init__(self, element, shape: Tuple[int, int], buffer_factor: int = 2):
        if len(shape) != 2 or any(int(s) <= 0 for s in shape):
            raise ValueError(f"CB shape must be two positive tile counts, got {shape}")
        if buffer_factor < 1:
            raise ValueError(f"buffer_factor must be >= 1, got {buffer_factor}")
        self.id = next(_cb_ids)
        self.shape = (int(shape[0]), int(shape[1]))
        self.buffer_factor = int(buffer_factor)
        self.dtype = element.dtype
        self.capacity_tiles = self.shape[0] * self.shape[1] * self.buffer_factor
        self.name = _assigned_name(_user_location(), f"cb{self.id}")
        if _kstate is not None:
            _kstate.cbs.append(self)
            if len(_kstate.cbs) > MAX_CBS:
                raise ValueError(f"a kernel may create at most {MAX_CBS} circular buffers")

    def __repr__(self):
        return f"CircularBuffer(id={self.id}, shape={self.shape}, bf={self.buffer_factor})"

    def _ctx(self) -> T.TraceContext:
        ctx = T.current()
        if ctx is None:
            raise RuntimeError("CB operations are only valid inside a ttl.kernel thread")
        return ctx

    def reserve(self) -> "Block":
        ctx = self._ctx()
        if self.id in ctx.pending_reserve:
            raise RuntimeError("Cannot call reserve() again before push(): CircularBuffer already "
                               "has a pending reserved block. You must call push() before calling "
                               "reserve() again.")
        ev = ctx.add(Event("reserve", self, ctx.cur, {"thread": ctx.thread,
                                                       "loc": _user_location()}))
        blk = Block(self, "reserve", ev)
        ctx.pending_reserve[self.id] = blk
        return blk

    def wait(self) -> "Block":
        ctx = self._ctx()
        if self.id in ctx.pending_wait:
            raise RuntimeError("Cannot call wait() again before pop(): CircularBuffer already "
                               "has a pending waited block. You must call pop() before calling "
                               "wait() again.")
        ev = ctx.add(Event("wait", self, ctx.cur, {"thread": ctx.thread,
                                                    "loc": _user_location()}))
        blk = Block(self, "wait", ev)
        ctx.pending_wait[self.id] = blk
        return blk

    def push(self) -> None:
        ctx = self._ctx()
        blk = ctx.pending_reserve.get(self.id)
        if blk is None:
            raise RuntimeError("push() without a matching reserve()")
        blk._check_no_pending_copy("push()")
        del ctx.pending_reserve[self.id]
        ctx.add(Event("push", self, ctx.cur))

    def pop(self) -> None:
        ctx = self._ctx()
        blk = ctx.pending_wait.get(self.id)
        if blk is None:
            raise RuntimeError("pop() without a matching wait()")
        blk._check_no_pending_copy("pop()")
        del ctx.pending_wait[self.id]
        ctx.add(Event("pop", self, ctx.cur))

    def can_wait(self) -> bool:
        return True

    def can_reserve(self) -> bool:
        return True


def make_circular_buffer_like(element, shape: Tuple[int, int],
                              buffer_factor: int = 2) -> CircularBuffer:
    return CircularBuffer(element, shape, buffer_factor)


# block expressions ---------------------------------------------------------


class BExpr:
    """A block-shaped expression.  `tree` is one per-tile expression shared by
    every tile of the block; its leaves are ("leaf", block, rmap, cmap[, rep])
    where rmap[i] / cmap[j] give the leaf block's tile feeding output tile
    (i, j) (that is how block broadcasting, python/sim/block.py:886-920, is
    kept) and rep = (rows, cols) marks the in-tile broadcast of
    ttl.math.broadcast: each tile's row 0 / column 0 repeated over the tile."""

    __slots__ = ("shape", "tree", "dtype")

    def __init__(self, shape: Tuple[int, int], tree, dtype: torch.dtype):
        self.shape = shape
        self.tree = tree
        self.dtype = dtype

    # operators (python/sim/block.py:963-1013)
    def __add__(self, o): return _binary("add", self, o)
    def __radd__(self, o): return _binary("add", o, self)
    def __sub__(self, o): return _binary("sub", self, o)
    def __rsub__(self, o): return _binary("sub", o, self)
    def __mul__(self, o): return _binary("mul", self, o)
    def __rmul__(self, o): return _binary("mul", o, self)
    def __truediv__(self, o): return _binary("div", self, o)
    def __rtruediv__(self, o): return _binary("div", o, self)
    def __floordiv__(self, o): return _binary("floordiv", self, o)
    def __mod__(self, o): return _binary("mod", self, o)
    def __matmul__(self, o): return _binary("matmul", self, o)
    def __neg__(self): return _unary("neg", self)

    def __pow__(self, o):
        if isinstance(o, int):
            return BExpr(self.shape, ("powi", self.tree, o), self.dtype)
        return _binary("pow", self, o)

    def __len__(self):
        return self.shape[0] * self.shape[1]


def _as_bexpr(x) -> BExpr:
    if isinstance(x, BExpr):
        return x
    if isinstance(x, Block):
        return x.expr()
    raise TypeError(f"expected a block or block expression, got {type(x).__name__}")


class _SubCB:
    """Stand-in CB of a sub-expression leaf: its dtype and a name."""

    __slots__ = ("dtype", "id", "name")

    def __init__(self, dtype) -> None:
        self.dtype, self.id, self.name = dtype, None, "(reduction)"


class SubExpr:
    """A reduction used as an operand of a larger expression (the spec types
    reduce_sum / reduce_max BlockExpr -> BlockExpr, TTLangSpecification.md:
    754-755): a leaf of the enclosing tree whose block is this object.  The
    planner computes it into a plan-owned tensor first, as the simulator
    materialises every intermediate value of an expression in its dtype, and
    the enclosing program reads it there like any operand."""

    __slots__ = ("expr", "cb")

    def __init__(self, e: "BExpr") -> None:
        self.expr = e
        self.cb = _SubCB(e.dtype)


def _lift(e: BExpr) -> BExpr:
    """A reduction about to become an operand: a leaf over its own block."""
    if e.tree[0] == "reduce":
        r, c = e.shape
        return BExpr(e.shape, ("leaf", SubExpr(e), np.arange(r), np.arange(c)), e.dtype)
    return e


def _remap(tree, axis: int, new_len: int):
    """Broadcast a size-1 axis of every leaf map in `tree` to `new_len`."""
    tag = tree[0]
    if tag == "leaf":
        blk, rmap, cmap = tree[1], tree[2], tree[3]
        if axis == 0:
            rmap = np.repeat(rmap[:1], new_len)
        else:
            cmap = np.repeat(cmap[:1], new_len)
        return ("leaf", blk, rmap, cmap) + tuple(tree[4:])
    if tag == "const":
        return tree
    if tag == "powi":
        return ("powi", _remap(tree[1], axis, new_len), tree[2])
    if tag == "upar":
        return ("upar", _remap(tree[1], axis, new_len)) + tuple(tree[2:])
    return (tag,) + tuple(_remap(t, axis, new_len) for t in tree[1:])


def leaf_rep(leaf) -> Tuple[bool, bool]:
    """(rows, cols) in-tile broadcast flags of an expression leaf."""
    return leaf[4] if len(leaf) > 4 else (False, False)


def _tile_rep(tree, rows: bool, cols: bool):
    """Marks every leaf of `tree` for the in-tile broadcast of row 0 (rows)
    and / or column 0 (cols): elementwise ops commute with picking one row or
    column of every tile, so the broadcast of an expression is the expression
    of broadcast operands."""
    tag = tree[0]
    if tag == "leaf":
        r0, c0 = leaf_rep(tree)
        return tuple(tree[:4]) + ((r0 or rows, c0 or cols),)
    if tag == "const":
        return tree
    if tag in ("powi", "upar"):
        return (tag, _tile_rep(tree[1], rows, cols)) + tuple(tree[2:])
    if tag in ("reduce", "matmul", "bmatmul"):
        raise NotImplementedError(f"ttl.math.broadcast of a {tag} result inside one store() is not "
                                  "supported; store the result into a CB first and broadcast the "
                                  "block waited from it")
    return (tag,) + tuple(_tile_rep(t, rows, cols) for t in tree[1:])


def _is_block_matmul(sa, sb) -> bool:
    """Block shapes for which `a @ b` is the spec's block matmul
    (docs/sphinx/specs/TTLangSpecification.md:693: (M, K) @ (K, N) -> (M, N)):
    inner dimensions equal and above 1, and the shapes not compatible for
    the simulator's tile-wise pairing (python/sim/block.py:870-920, which
    raises for them).  Where both readings apply, the simulator's wins."""
    if len(sa) != 2 or len(sb) != 2 or sa[1] != sb[0] or sa[1] <= 1:
        return False
    return any(la != lb and la != 1 and lb != 1 for la, lb in zip(sa, sb))


def _block_matmul(aa: "BExpr", bb: "BExpr") -> "BExpr":
    """Output tile (i, j) = sum over k of a(i, k) @ b(k, j), accumulated in
    fp32 and rounded once (as a store(acc=True) loop of tile matmuls over k
    runs on the MI355X).  Operands may be computed block expressions
    (the spec types __matmul__(self, other: BlockExpr), TTLangSpecification.md:
    693); the planner materialises such an operand in its dtype first, as the
    simulator does (python/sim/block.py:1012-1013 pairs any blocks)."""
    K = aa.shape[1]
    return BExpr((aa.shape[0], bb.shape[1]), ("bmatmul", aa.tree, bb.tree, K),
                 torch.promote_types(aa.dtype, bb.dtype))


def _binary(op: str, a, b) -> BExpr:
    if isinstance(a, (int, float)) and not isinstance(a, bool):
        bb = _lift(_as_bexpr(b))
        return BExpr(bb.shape, (op, ("const", float(a)), bb.tree), bb.dtype)
    if isinstance(b, (int, float)) and not isinstance(b, bool):
        aa = _lift(_as_bexpr(a))
        return BExpr(aa.shape, (op, aa.tree, ("const", float(b))), aa.dtype)
    aa, bb = _lift(_as_bexpr(a)), _lift(_as_bexpr(b))
    sa, sb = aa.shape, bb.shape
    if op == "matmul" and _is_block_matmul(sa, sb):
        return _block_matmul(aa, bb)
    if len(sa) != len(sb):
        raise ValueError(f"Cannot broadcast: dimension mismatch between shapes {sa} and {sb}. "
                         "Shapes must have the same number of dimensions.")
    out = []
    ta, tb = aa.tree, bb.tree
    for i, (la, lb) in enumerate(zip(sa, sb)):
        if la != lb and la != 1 and lb != 1:
            raise ValueError(f"Cannot broadcast: incompatible shapes {sa} and {sb}. Dimension {i} "
                             f"has sizes {la} and {lb} which are incompatible (must be equal or one "
                             "must be 1).")
        n = max(la, lb)
        if la != n:
            ta = _remap(ta, i, n)
        if lb != n:
            tb = _remap(tb, i, n)
        out.append(n)
    return BExpr(tuple(out), (op, ta, tb), torch.promote_types(aa.dtype, bb.dtype))


def _unary(op: str, a, imm: Optional[float] = None) -> BExpr:
    aa = _lift(_as_bexpr(a))
    return BExpr(aa.shape, (op, aa.tree), aa.dtype)


def _unary_param(op: str, a, p0: float, p1: float = 0.0) -> BExpr:
    """A unary op with numeric parameters (the spec types them PositiveInt;
    their numeric value is used)."""
    aa = _lift(_as_bexpr(a))
    return BExpr(aa.shape, ("upar", aa.tree, op, float(p0), float(p1)), aa.dtype)


def _reduce(kind: str, x, scaler, dims) -> BExpr:
    """ttl.math.reduce_sum / reduce_max (docs/sphinx/specs/
    TTLangSpecification.md:754-755).  The reference specifies only the
    signature; the semantics implemented: every element of `x` times the
    scaler (the first element of a (1, 1) block, or a number), summed or
    maximised (NaN-propagating) over the element rows (dims [0]), columns
    ([1]) or both of the block, in fp32, rounded once to the block's dtype.
    The result block has size 1 along the reduced dims; each of its tiles
    holds the values in its first row / column ([0, 0] for both) and zeros
    elsewhere, so it can be copied to a full 32-wide tensor tile or to a
    size-1 tensor dimension."""
    if dims is None:
        raise ValueError(f"dims parameter is required for reduce_{kind}()")
    dl = [int(d) for d in dims]
    if not dl or len(set(dl)) != len(dl) or any(d not in (0, 1) for d in dl):
        raise ValueError(f"reduce_{kind}() dims must be [0], [1] or [0, 1], got {list(dims)}")
    e = _lift(_as_bexpr(x))
    if isinstance(scaler, (int, float)) and not isinstance(scaler, bool):
        st = ("const", float(scaler))
    else:
        se = _as_bexpr(scaler)
        if tuple(se.shape) != (1, 1):
            raise ValueError(f"reduce_{kind}() scaler must be a (1, 1) block, got shape {se.shape}")
        if se.tree[0] != "leaf":
            raise NotImplementedError(f"reduce_{kind}() scaler must be a block read from a CB "
                                      "(an expression as scaler is not supported)")
        st = se.tree
    shape = tuple(1 if i in dl else n for i, n in enumerate(e.shape))
    return BExpr(shape, ("reduce", kind, tuple(sorted(dl)), e.tree, tuple(e.shape), st), e.dtype)


class Block:
    """A block of a CB obtained from wait() (readable) or reserve() (writable).
    Used as a context manager it pops / pushes on exit (python/sim/cb.py:40-157)."""

    def __init__(self, cb: CircularBuffer, kind: str, event: Event):
        self.cb = cb
        self.kind = kind
        self.event = event
        self.shape = cb.shape
        self._stores = 0
        # a copy into ("dst") or out of ("src") this block whose wait() has not
        # run yet: the block is locked until then (python/sim/block.py:263-343,656-694)
        self._pending_copy: Optional[str] = None

    def _check_no_pending_copy(self, operation: str) -> None:
        if self._pending_copy is not None:
            state = "NAW" if self._pending_copy == "dst" else "NAR"
            raise RuntimeError(f"Cannot perform {operation}: Expected one of [TX_WAIT], but got "
                               f"{operation}. Current state: Acquisition={self.kind.upper()}, "
                               f"Thread=DM, Access={state}")

    def __enter__(self) -> "Block":
        return self

    def __exit__(self, exc_type, exc, tb) -> None:
        if exc_type is not None:
            return
        if self.kind == "reserve":
            self.cb.push()
        else:
            self.cb.pop()

    def block(self) -> "Block":
        return self

    def __len__(self) -> int:
        return self.shape[0] * self.shape[1]

    def __getitem__(self, idx):
        raise RuntimeError("Block indexing (block[index]) is not allowed. Blocks must be used as "
                           "whole units in operations like store() or arithmetic. Use block "
                           "directly without indexing.")

    def __setitem__(self, idx, value):
        raise RuntimeError("Direct assignment to Block is not allowed. Use block.store() or "
                           "copy() instead.")

    def expr(self) -> BExpr:
        if self._pending_copy == "dst":
            raise RuntimeError("Cannot read from Block: Block has no access (NAW state). Current "
                               "state: NAW, Expected operations: [TX_WAIT]")
        if self.kind != "wait":
            raise NotImplementedError("reading a reserved (output) block back is not supported by "
                                      "the MI355X backend; read blocks obtained from wait()")
        r, c = self.shape
        return BExpr(self.shape, ("leaf", self, np.arange(r), np.arange(c)),
                     compute_dtype(self.cb.dtype))

    # arithmetic delegates to BExpr
    def __add__(self, o): return _binary("add", self, o)
    def __radd__(self, o): return _binary("add", o, self)
    def __sub__(self, o): return _binary("sub", self, o)
    def __rsub__(self, o): return _binary("sub", o, self)
    def __mul__(self, o): return _binary("mul", self, o)
    def __rmul__(self, o): return _binary("mul", o, self)
    def __truediv__(self, o): return _binary("div", self, o)
    def __rtruediv__(self, o): return _binary("div", o, self)
    def __floordiv__(self, o): return _binary("floordiv", self, o)
    def __mod__(self, o): return _binary("mod", self, o)
    def __matmul__(self, o): return _binary("matmul", self, o)
    def __neg__(self): return _unary("neg", self)

    def __pow__(self, o):
        return self.expr() ** o

    def store(self, items, acc: bool = False) -> None:
        """Store a block expression into this reserved block.  acc=True: the first
        store assigns, later ones add (python/sim/block.py:805-868)."""
        if self._pending_copy == "dst":
            raise RuntimeError("Cannot write to Block: Block is locked as copy destination until "
                               "tx.wait() completes (copy lock error). Current state: NAW, "
                               "Expected operations: [TX_WAIT]")
        if self._pending_copy == "src":
            raise RuntimeError("Cannot write to Block: Block is locked as copy source until "
                               "tx.wait() completes. Current state: NAR, Expected operations: "
                               "[TX_WAIT]")
        if self.kind != "reserve":
            raise RuntimeError("store() needs a block obtained from reserve()")
        ctx = T.current()
        if ctx is None:
            raise RuntimeError("store() is only valid inside a ttl.kernel thread")
        e = _as_bexpr(items)
        if len(e) != len(self):
            raise ValueError("Length mismatch in store()")
        if e.tree[0] == "reduce" and tuple(e.shape) != tuple(self.shape):
            raise ValueError(f"store() of a reduction of shape {tuple(e.shape)} into a block of "
                             f"shape {tuple(self.shape)}: the block must have the reduced shape")
        ctx.add(Event("store", self.cb, ctx.cur,
                      {"target": self, "expr": e, "acc": bool(acc), "thread": ctx.thread,
                       "loc": _user_location()}))
        self._stores += 1


# ---------------------------------------------------------------------------
# copy


_PKG_DIR = os.path.dirname(os.path.abspath(__file__))


def _assigned_name(loc: Tuple[str, int], default: str) -> str:
    """The variable a `name = ...` source line assigns (the name a deadlock
    report shows, as the simulator does: python/sim/program.py:184)."""
    import linecache

    m = re.match(r"\s*([A-Za-z_]\w*)\s*=[^=]", linecache.getline(loc[0], loc[1]))
    return m.group(1) if m else default


def _user_location() -> Tuple[str, int]:
    """(file, line) of the innermost caller outside this package: the kernel
    source line a traced operation came from."""
    f = sys._getframe(1)
    while f is not None and os.path.dirname(os.path.abspath(f.f_code.co_filename)) == _PKG_DIR:
        f = f.f_back
    return (f.f_code.co_filename, f.f_lineno) if f is not None else ("?", 0)


class CopyTransaction:
    """Handle of one tensor<->block copy; wait() releases the block's copy
    lock (python/sim/copy.py:37-195).  The transfer itself is part of the
    planned kernel, so the handle carries no data."""

    def __init__(self, block: "Block", role: str):
        if block._pending_copy is not None:
            op = "copy (as destination)" if role == "dst" else "copy (as source)"
            block._check_no_pending_copy(op)
        self._block: Optional[Block] = block
        block._pending_copy = role

    def wait(self) -> None:
        if self._block is not None:
            self._block._pending_copy = None
            self._block = None

    def is_done(self) -> bool:
        return True


def copy(src, dst) -> CopyTransaction:
    """Tensor slice -> reserved block, or waited block -> tensor slice.  Tiles
    go into block slots row-major over the block's tile grid
    (python/sim/copyhandlers.py:295-380)."""
    ctx = T.current()
    if ctx is None:
        raise RuntimeError("ttl.copy is only valid inside a ttl.kernel thread")
    if isinstance(src, TensorSlice) and isinstance(dst, Block):
        if dst.kind != "reserve":
            raise TraceError("copy into a block needs a block obtained from reserve()")
        _check_slice_shape(src, dst)
        for x, nm in ((src.r0, "row index"), (src.c0, "col index")):
            ctx.check_loops(x, nm)
        tx = CopyTransaction(dst, "dst")
        ctx.add(Event("copy_in", dst.cb, ctx.cur, {"block": dst, "slice": src}))
        return tx
    if isinstance(src, Block) and isinstance(dst, TensorSlice):
        if src.kind != "wait":
            raise TraceError("copy out of a block needs a block obtained from wait()")
        _check_slice_shape(dst, src)
        for x, nm in ((dst.r0, "row index"), (dst.c0, "col index")):
            ctx.check_loops(x, nm)
        tx = CopyTransaction(src, "src")
        ctx.add(Event("copy_out", src.cb, ctx.cur, {"block": src, "slice": dst}))
        return tx
    if isinstance(src, Block) and isinstance(dst, SrcPipeIdentity):
        tx = CopyTransaction(src, "src")
        ctx.add(Event("pipe_send", src.cb, ctx.cur, {"block": src, "pipe": dst.pipe}))
        return tx
    if isinstance(src, DstPipeIdentity) and isinstance(dst, Block):
        if dst.kind != "reserve":
            raise TraceError("a pipe delivers into a block obtained from reserve()")
        tx = CopyTransaction(dst, "dst")
        ctx.add(Event("pipe_recv", dst.cb, ctx.cur, {"block": dst, "pipe": src.pipe}))
        return tx
    raise NotImplementedError(
        f"ttl.copy({type(src).__name__} -> {type(dst).__name__}) is not supported (tensor <-> "
        "block and block <-> pipe copies are)")


# ---------------------------------------------------------------------------
# pipes: core-to-core block transfers (python/sim/pipe.py:1-270,
# python/sim/typedefs.py:41-90).  The tracer records sends and receives; the
# planner gives a received block the tensor-tile origin of the matching sent
# block (k-th send <-> k-th receive of a pipe), so on the GPU every receiving
# workgroup reads that tile itself (through L2) instead of a core forwarding it.


def _linear_core(coord) -> int:
    if isinstance(coord, (int, np.integer)):
        return int(coord)
    g = _grid()
    c = tuple(int(x) for x in coord)
    if len(c) != len(g):
        gs = grid_size(dims=len(c))
        lin = 0
        for x, s in zip(c, gs):
            lin = lin * s + x
        return lin
    return flatten_core_index(c)


def _expand_range(spec) -> List[int]:
    """Linear ids of a destination: a core (int or coordinate tuple), a tuple
    with slices (python/sim/pipe.py expand_core_range), or a (first, last)
    pair of coordinate tuples (inclusive rectangle)."""
    if isinstance(spec, (int, np.integer)):
        return [int(spec)]
    spec = tuple(spec)
    if len(spec) == 2 and all(isinstance(x, tuple) for x in spec):
        a, b = spec
        ranges = [range(min(x, y), max(x, y) + 1) for x, y in zip(a, b)]
    else:
        gs = grid_size(dims=len(spec))
        if not isinstance(gs, tuple):
            gs = (gs,)
        ranges = []
        for i, item in enumerate(spec):
            if isinstance(item, slice):
                start = 0 if item.start is None else item.start
                stop = gs[i] if item.stop is None else item.stop
                ranges.append(range(start, stop, 1 if item.step is None else item.step))
            else:
                ranges.append(range(int(item), int(item) + 1))
    out: List[int] = []

    def walk(i, acc):
        if i == len(ranges):
            out.append(_linear_core(tuple(acc)))
            return
        for v in ranges[i]:
            walk(i + 1, acc + [v])
    walk(0, [])
    return out


_pipe_ids = itertools.count()


class Pipe:
    """A block transfer from `src_core` to the core(s) of `dst_core_range`
    (unicast: one coordinate; multicast: a tuple with slices)."""

    def __init__(self, src_core, dst_core_range):
        self.id = next(_pipe_ids)
        self.src_core = src_core
        self.dst_core_range = dst_core_range

    def _src(self) -> int:
        return _linear_core(self.src_core)

    def _dsts(self) -> List[int]:
        return _expand_range(self.dst_core_range)

    def has_current_core(self) -> bool:
        """Whether the current core sends or receives on this pipe."""
        c = core(dims=1)
        return c == self._src() or c in self._dsts()

    def __repr__(self) -> str:
        return f"Pipe({self.src_core} -> {self.dst_core_range})"


class SrcPipeIdentity:
    """A pipe as seen by its source core (`dst` tells where blocks go)."""

    def __init__(self, pipe: Pipe):
        self.pipe = pipe

    @property
    def dst(self):
        return self.pipe.dst_core_range


class DstPipeIdentity:
    """A pipe as seen by a destination core (`src` tells where blocks come from)."""

    def __init__(self, pipe: Pipe):
        self.pipe = pipe

    @property
    def src(self):
        return self.pipe.src_core


class PipeNet:
    """Pipes grouped so a thread can run one callback per pipe it sends on
    (`if_src`) and one per pipe it receives on (`if_dst`)."""

    def __init__(self, pipes: Sequence[Pipe]):
        self._pipes = list(pipes)

    def if_src(self, fn: Callable[[SrcPipeIdentity], Any]) -> None:
        c = core(dims=1)
        for p in self._pipes:
            if p._src() == c:
                fn(SrcPipeIdentity(p))

    def if_dst(self, fn: Callable[[DstPipeIdentity], Any]) -> None:
        c = core(dims=1)
        for p in self._pipes:
            if c in p._dsts():
                fn(DstPipeIdentity(p))


def _check_slice_shape(s: TensorSlice, blk: Block) -> None:
    if len(s.tensor.shape) != 2:
        raise ValueError(f"Tensor must be 2-dimensional, got shape {s.tensor.shape}")
    tiles = s.shape_in_tiles()
    if tiles != tuple(blk.shape):
        h, w = s.tensor.shape
        elems = (1 if h == 1 else tiles[0] * TILE_SHAPE[0], 1 if w == 1 else tiles[1] * TILE_SHAPE[1])
        # the simulator's wording (the slice's element shape), which the
        # reference's tests match (test/sim/test_examples.py:134-145)
        raise ValueError(f"Tensor shape {elems} (={tiles} tiles) does not match Block shape "
                         f"{tuple(blk.shape)} tiles")
    s.check_bounds()


# ---------------------------------------------------------------------------
# ttl.math


class _Math:
    """ttl.math: broadcast, the elementwise tile ops and the scaled reductions."""

    @staticmethod
    def broadcast(block, out=None, dims: Optional[Sequence[int]] = None) -> BExpr:
        """Two forms.  With `out`, the compiler's tile broadcast (the only form
        it has, python/ttl/operators.py:333-360; tile op unary_bcast Row / Col
        / Scalar, TTLElementwiseOps.def:82): every tile becomes its row 0
        (dims=[0]), column 0 ([1]) or element [0, 0] ([0, 1]) repeated over
        the tile, and a block dimension of size 1 along a broadcast dim takes
        the size of the output block `out` (shape expansion,
        test/python/test_bcast_shape_expansion.py).  Without `out`, the
        simulator's form (python/sim/math.py:20-106): the broadcast block
        dims must have size 1, the block is returned unchanged and the
        enclosing binary op broadcasts it over the tile grid (and inside
        size-1 tensor dimensions); the tiles' own rows / columns are kept."""
        if dims is None:
            raise ValueError("dims parameter is required for broadcast()")
        e = _as_bexpr(block)
        if out is None:
            for d in dims:
                if d >= len(e.shape):
                    raise ValueError(f"Cannot broadcast along dimension {d}: block has shape "
                                     f"{e.shape} with only {len(e.shape)} dimensions")
                if e.shape[d] != 1:
                    raise ValueError(f"Cannot broadcast along dimension {d}: dimension must have "
                                     f"size 1, but has size {e.shape[d]}")
            return e
        e = _lift(e)
        target = tuple(out.shape)
        shape, tree = list(e.shape), e.tree
        for d in dims:
            if d >= len(e.shape):
                raise ValueError(f"Cannot broadcast along dimension {d}: block has shape {e.shape} "
                                 f"with only {len(e.shape)} dimensions")
            n = e.shape[d]
            if n == 1 and target[d] != 1:
                tree = _remap(tree, d, target[d])
                shape[d] = target[d]
            elif n != 1 and target[d] != n:
                raise ValueError(f"Cannot broadcast along dimension {d}: dimension must have size "
                                 f"1, but has size {n}")
        if set(dims) - {0, 1}:
            raise ValueError(f"Invalid dims: {list(dims)}. Must be [0], [1], or [0, 1]")
        tree = _tile_rep(tree, 0 in dims, 1 in dims)
        return BExpr(tuple(shape), tree, e.dtype)

    @staticmethod
    def exp(x): return _unary("exp", x)
    @staticmethod
    def log(x): return _unary("log", x)
    @staticmethod
    def sqrt(x): return _unary("sqrt", x)
    @staticmethod
    def rsqrt(x): return _unary("rsqrt", x)
    @staticmethod
    def tanh(x): return _unary("tanh", x)
    @staticmethod
    def abs(x): return _unary("abs", x)
    @staticmethod
    def neg(x): return _unary("neg", x)
    @staticmethod
    def relu(x): return _unary("relu", x)
    @staticmethod
    def sigmoid(x): return _unary("sigmoid", x)
    @staticmethod
    def recip(x): return _unary("recip", x)
    @staticmethod
    def max(a, b): return _binary("max", a, b)
    @staticmethod
    def min(a, b): return _binary("min", a, b)
    maximum = max
    minimum = min

    # the spec's further math functions (TTLangSpecification.md:700-750;
    # the reference compiler's op table and simulator implement none of
    # them).  Each follows the torch function the spec links applied to a
    # bfloat16 tile: native ops compute in fp32 and round once, as those
    # torch kernels do; the compositions round where torch does (exact
    # partial results, or torch's own composition for softsign).
    @staticmethod
    def exp2(x): return _unary("exp2", x)
    @staticmethod
    def expm1(x): return _unary("expm1", x)
    @staticmethod
    def logp1(x): return _unary("logp1", x)
    @staticmethod
    def square(x): return _binary("mul", x, x)
    @staticmethod
    def rsub(a, b): return _binary("sub", b, a)
    @staticmethod
    def sin(x): return _unary("sin", x)
    @staticmethod
    def cos(x): return _unary("cos", x)
    @staticmethod
    def tan(x): return _unary("tan", x)
    @staticmethod
    def asin(x): return _unary("asin", x)
    @staticmethod
    def acos(x): return _unary("acos", x)
    @staticmethod
    def atan(x): return _unary("atan", x)
    @staticmethod
    def asinh(x): return _unary("asinh", x)
    @staticmethod
    def acosh(x): return _unary("acosh", x)
    @staticmethod
    def atanh(x): return _unary("atanh", x)
    @staticmethod
    def gelu(x): return _unary("gelu", x)
    @staticmethod
    def silu(x): return _unary("silu", x)
    @staticmethod
    def softsign(x):
        # torch's softsign is the composition x / (|x| + 1), rounded per op
        return _binary("div", x, _binary("add", _unary("abs", x), 1.0))
    @staticmethod
    def hardsigmoid(x): return _unary("hardsigmoid", x)
    @staticmethod
    def relu_max(x, upper_limit): return _unary("relu", _binary("min", x, upper_limit))
    @staticmethod
    def relu_min(x, lower_limit): return _unary("relu", _binary("max", x, lower_limit))
    @staticmethod
    def hardtanh(x, min, max):  # noqa: A002 (the spec's parameter names)
        return _binary("min", _binary("max", x, min), max)
    @staticmethod
    def leaky_relu(x, slope):
        # relu(x) + slope * min(x, 0): one of the two terms is zero
        return _binary("add", _unary("relu", x), _binary("mul", _binary("min", x, 0.0), slope))
    @staticmethod
    def prelu(x, alpha): return _Math.leaky_relu(x, alpha)
    @staticmethod
    def elu(x, slope): return _unary_param("elu", x, slope)
    @staticmethod
    def celu(x, alpha, alpha_recip=None): return _unary_param("celu", x, alpha)
    @staticmethod
    def selu(x, scale, alpha): return _unary_param("selu", x, scale, alpha)
    @staticmethod
    def softplus(x, beta, beta_reciprocal=None, threshold=20.0):
        return _unary_param("softplus", x, beta, threshold)

    @staticmethod
    def reduce_sum(expr, scaler, dims=None) -> BExpr:
        """Scaled sum over `dims` (spec TTLangSpecification.md:754)."""
        return _reduce("sum", expr, scaler, dims)

    @staticmethod
    def reduce_max(expr, scaler, dims=None) -> BExpr:
        """Scaled maximum over `dims` (spec TTLangSpecification.md:755)."""
        return _reduce("max", expr, scaler, dims)


math = _Math()


def signpost(*_a, **_k) -> None:
    """Profiling marker (python/ttl/ttl.py:23-26); timing on the MI355X comes
    from rocprofv3 kernel traces."""
    return None


# ---------------------------------------------------------------------------
# kernel


def kernel(grid: Union[str, Tuple[int, ...]] = "auto", **options) -> Callable:
    """@ttl.kernel(grid=...): runs the kernel body to collect its CBs and its
    three threads, traces every core, and executes the resulting tile program
    on the GPU.  grid="auto" is the simulator's (8, 8) (python/sim/kernel.py:226).
    The output tensors are written in place; the call returns None after the
    device work has finished (the reference's synchronous semantics)."""
    actual_grid = (8, 8) if grid == "auto" else tuple(int(g) for g in grid)
    if any(g <= 0 for g in actual_grid):
        raise ValueError(f"grid dimensions must be positive, got {grid}")

    def decorator(func):
        from . import runner

        return runner.KernelRunner(func, actual_grid, grid, options)

    return decorator
