"""Eager CPU executor of tt-lang kernels with the simulator's semantics
(TEST ORACLE ONLY - never imported by the product).

Each core runs its three threads as real Python threads that block on
circular buffers, one torch op per 32x32 tile, exactly the execution model of
the reference simulator (python/sim/program.py:100-255 runs cores one after
another, threads cooperatively; here threads block on condition variables,
which yields the same dataflow).  Restated rules, with the reference lines
they follow:
  - CB: capacity = shape0 * shape1 * buffer_factor tiles; reserve() blocks
    until a block is free and zero-fills it in the CB dtype; push() publishes;
    wait() blocks until a block is visible; pop() frees (cb.py:302-408).
  - copy(tensor[rows, cols] -> block): tile (h, w) of the slice goes to slot
    h * width + w; size-1 tensor dimensions stay size 1 (copyhandlers.py:
    103-131, 295-336; tensoraccessor.py:125-159); block -> tensor is the
    inverse (copyhandlers.py:339-380).
  - block ops: equal shapes are tile-wise; otherwise tiles are stacked and
    torch-broadcast over the tile grid (block.py:870-959,
    ttnnsim.py:67-109); every result is materialised in its torch dtype.
  - store(acc=True): first store assigns, later ones add in the stored
    tensors' dtype (block.py:805-868).
  - grid / core / grid_size (kernel.py:89-291); grid "auto" = (8, 8).
  - ttl.math.reduce_sum / reduce_max (spec TTLangSpecification.md:754-755;
    no reference implementation exists, the semantics are the ones the
    backend defines): every element times the scaler (first element of its
    tile, or a number), summed / maximised (NaN-propagating) in float64 over
    the block's element rows ([0]), columns ([1]) or both, rounded to the
    block dtype (via fp32); result tiles are 32x32 with the values in row /
    column 0 ([0, 0] for both) and zeros elsewhere.  Copying such a tile to a
    size-1 tensor dimension keeps its first row / column.
The oracle takes plain CPU torch tensors and is driven through `make_ttl()`,
which returns a namespace with the same names as `ttl`.
"""

from __future__ import annotations

import operator
import threading
import types
from typing import Any, List, Optional, Tuple

import torch

TILE = 32
TIMEOUT_S = 30.0


class OracleTensor:
    """CPU tensor with tt-lang tile indexing."""

    def __init__(self, t: torch.Tensor):
        self.t = t

    @property
    def shape(self):
        return tuple(self.t.shape)

    @property
    def dtype(self):
        return self.t.dtype

    def __getitem__(self, key):
        rows, cols = key
        return _Slice(self, rows, cols)


class _Slice:
    def __init__(self, tensor: OracleTensor, rows, cols):
        def norm(k):
            if isinstance(k, slice):
                assert k.start is not None and k.stop is not None and k.step is None
                return k.start, k.stop
            return int(k), int(k) + 1
        self.tensor = tensor
        self.rows = norm(rows)
        self.cols = norm(cols)

    def elements(self) -> torch.Tensor:
        (r0, r1), (c0, c1) = self.rows, self.cols
        return self.tensor.t[r0 * TILE:r1 * TILE, c0 * TILE:c1 * TILE]

    def tiles_shape(self) -> Tuple[int, int]:
        e = self.elements()
        h, w = e.shape
        return (1 if h == 1 else h // TILE, 1 if w == 1 else w // TILE)


class _CB:
    def __init__(self, element, shape, buffer_factor):
        self.dtype = element.dtype
        self.shape = tuple(shape)
        self.n = shape[0] * shape[1]
        self.capacity = self.n * buffer_factor
        self.reset()

    def reset(self):
        self.cond = threading.Condition()
        self.slots: List[Optional[torch.Tensor]] = [None] * self.capacity
        self.head = 0      # first visible tile
        self.visible = 0
        self.reserved = 0  # tiles reserved (not yet pushed)

    def _wait_for(self, pred, what):
        if not self.cond.wait_for(pred, timeout=TIMEOUT_S):
            raise RuntimeError(f"deadlock: timed out in {what}")

    def reserve(self):
        with self.cond:
            self._wait_for(lambda: self.capacity - self.visible - self.reserved >= self.n, "reserve")
            start = (self.head + self.visible) % self.capacity
            self.reserved = self.n
            idx = [(start + i) % self.capacity for i in range(self.n)]
            for i in idx:  # zero-fill in the CB dtype (cb.py:343-346)
                self.slots[i] = torch.zeros(TILE, TILE, dtype=self.dtype)
        return _Block(self, idx, "reserve")

    def push(self):
        with self.cond:
            self.visible += self.n
            self.reserved = 0
            self.cond.notify_all()

    def wait(self):
        with self.cond:
            self._wait_for(lambda: self.visible >= self.n, "wait")
            idx = [(self.head + i) % self.capacity for i in range(self.n)]
        return _Block(self, idx, "wait")

    def pop(self):
        with self.cond:
            self.head = (self.head + self.n) % self.capacity
            self.visible -= self.n
            self.cond.notify_all()


class _Tiles:
    """A block-shaped list of tiles (result of block arithmetic)."""

    def __init__(self, tiles: List[torch.Tensor], shape: Tuple[int, int]):
        self.tiles = tiles
        self.shape = shape

    def _bin(self, other, op, rev=False):
        if isinstance(other, (int, float)) and not isinstance(other, bool):
            # a Python number: one op per tile in the tile dtype (block.py:963-1010)
            return self.map((lambda t: op(other, t)) if rev else (lambda t: op(t, other)))
        other = _tiles_of(other)
        if self.shape == other.shape:
            return _Tiles([op(a, b) for a, b in zip(self.tiles, other.tiles)], self.shape)
        for i, (l, r) in enumerate(zip(self.shape, other.shape)):
            if l != r and l != 1 and r != 1:
                raise ValueError(f"Cannot broadcast: incompatible shapes {self.shape} and "
                                 f"{other.shape}")
        a = torch.stack(self.tiles).reshape(*self.shape, *self.tiles[0].shape)
        b = torch.stack(other.tiles).reshape(*other.shape, *other.tiles[0].shape)
        res = op(a, b)
        shape = (res.shape[0], res.shape[1])
        flat = res.reshape(shape[0] * shape[1], *res.shape[2:])
        return _Tiles([flat[i] for i in range(flat.shape[0])], shape)

    def __add__(self, o): return self._bin(o, operator.add)
    def __radd__(self, o): return self._bin(o, operator.add, True)
    def __sub__(self, o): return self._bin(o, operator.sub)
    def __rsub__(self, o): return self._bin(o, operator.sub, True)
    def __mul__(self, o): return self._bin(o, operator.mul)
    def __rmul__(self, o): return self._bin(o, operator.mul, True)
    def __truediv__(self, o): return self._bin(o, operator.truediv)
    def __floordiv__(self, o): return self._bin(o, operator.floordiv)
    def __mod__(self, o): return self._bin(o, operator.mod)
    def __matmul__(self, o):
        o = _tiles_of(o)
        (m, k), (k2, n) = self.shape, o.shape
        if k == k2 and k > 1 and any(l != r and l != 1 and r != 1
                                     for l, r in zip(self.shape, o.shape)):
            # the spec's block matmul (TTLangSpecification.md:693), defined
            # where the simulator's tile-wise pairing raises: tile (i, j) =
            # sum over k of a(i, k) @ b(k, j) in fp32, rounded once
            dt = torch.promote_types(self.tiles[0].dtype, o.tiles[0].dtype)
            out = []
            for i in range(m):
                for j in range(n):
                    acc = sum(self.tiles[i * k + t].float() @ o.tiles[t * n + j].float()
                              for t in range(k))
                    out.append(acc.to(dt))
            return _Tiles(out, (m, n))
        return self._bin(o, operator.matmul)

    def __pow__(self, o):
        if isinstance(o, int):
            return _Tiles([t ** o for t in self.tiles], self.shape)
        return self._bin(o, operator.pow)

    def map(self, fn):
        return _Tiles([fn(t) for t in self.tiles], self.shape)


def _tiles_of(x) -> _Tiles:
    if isinstance(x, _Tiles):
        return x
    if isinstance(x, _Block):
        return _Tiles([x.cb.slots[i] for i in x.idx], x.cb.shape)
    raise TypeError(type(x))


class _Block(_Tiles):
    def __init__(self, cb: _CB, idx: List[int], kind: str):
        self.cb, self.idx, self.kind = cb, idx, kind
        self.shape = cb.shape
        self._first_acc = True

    @property
    def tiles(self):
        return [self.cb.slots[i] for i in self.idx]

    def __enter__(self):
        return self

    def __exit__(self, et, e, tb):
        if et is None:
            (self.cb.push if self.kind == "reserve" else self.cb.pop)()

    def store(self, items, acc: bool = False):
        src = _tiles_of(items).tiles
        if len(src) != len(self.idx):
            raise ValueError("Length mismatch in store()")
        if acc and not self._first_acc:
            for k, i in enumerate(self.idx):
                self.cb.slots[i] = self.cb.slots[i] + src[k]
        else:
            for k, i in enumerate(self.idx):
                self.cb.slots[i] = src[k]
        if acc:
            self._first_acc = False


def _reduce(kind: str, x, scaler, dims) -> _Tiles:
    t = _tiles_of(x)
    dims = sorted(int(d) for d in dims)
    if isinstance(scaler, (int, float)):
        sv = float(scaler)
    else:
        sv = float(_tiles_of(scaler).tiles[0].reshape(-1)[0])
    R, C = t.shape
    th, tw = t.tiles[0].shape
    m = torch.stack(t.tiles).double().reshape(R, C, th, tw).permute(0, 2, 1, 3)
    m = m.reshape(R * th, C * tw) * sv
    fn = (lambda v, d: v.sum(d)) if kind == "sum" else (lambda v, d: v.amax(d))
    dtype = t.tiles[0].dtype
    def fin(v):
        return v.to(torch.float32).to(dtype)
    out = []
    if dims == [0, 1]:
        tile = torch.zeros(TILE, TILE, dtype=dtype)
        tile[0, 0] = fin(fn(m.reshape(-1), 0))
        return _Tiles([tile], (1, 1))
    if dims == [1]:  # one value per element row, tiles (R, 1)
        v = fin(fn(m, 1))
        for i in range(R):
            tile = torch.zeros(TILE, TILE, dtype=dtype)
            tile[:th, 0] = v[i * th:(i + 1) * th]
            out.append(tile)
        return _Tiles(out, (R, 1))
    v = fin(fn(m, 0))  # dims [0]: one value per element column, tiles (1, C)
    for j in range(C):
        tile = torch.zeros(TILE, TILE, dtype=dtype)
        tile[0, :tw] = v[j * tw:(j + 1) * tw]
        out.append(tile)
    return _Tiles(out, (1, C))


def _copy(src, dst):
    if isinstance(src, _Slice) and isinstance(dst, _Block):
        if src.tiles_shape() != dst.shape:
            raise ValueError("copy: tensor slice does not match the block shape")
        e = src.elements()
        h, w = dst.shape
        for k, i in enumerate(dst.idx):
            r, c = divmod(k, w)
            dst.cb.slots[i] = e[r * TILE:(r + 1) * TILE, c * TILE:(c + 1) * TILE].clone()
    elif isinstance(src, _Block) and isinstance(dst, _Slice):
        if dst.tiles_shape() != src.shape:
            raise ValueError("copy: tensor slice does not match the block shape")
        e = dst.elements()
        h, w = src.shape
        for k, i in enumerate(src.idx):
            r, c = divmod(k, w)
            view = e[r * TILE:(r + 1) * TILE, c * TILE:(c + 1) * TILE]
            tile = src.cb.slots[i]
            if tuple(tile.shape) != tuple(view.shape):  # a result tile into a size-1 dimension
                tile = tile[:view.shape[0], :view.shape[1]]
            view.copy_(tile)
    else:
        raise NotImplementedError("oracle copy supports tensor<->block only")

    class _Tx:
        def wait(self):
            return None
    return _Tx()


def make_ttl():
    """A `ttl`-compatible namespace backed by this eager executor."""
    state = threading.local()
    registry: List[Any] = []
    cbs: List[_CB] = []
    ns = types.SimpleNamespace()
    ns.TILE_SHAPE = (TILE, TILE)

    def grid_size(dims=2):
        g = tuple(state.grid)
        if dims == len(g):
            r = g
        elif dims < len(g):
            tail = 1
            for d in g[dims - 1:]:
                tail *= d
            r = tuple(g[:dims - 1]) + (tail,)
        else:
            r = g + (1,) * (dims - len(g))
        return r[0] if dims == 1 else r

    def core(dims=2):
        g = tuple(state.grid)
        cid = state.core
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

    def compute():
        def deco(f):
            registry.append(("compute", f))
            return f
        return deco

    def datamovement():
        def deco(f):
            registry.append(("dm", f))
            return f
        return deco

    def make_cb(element, shape, buffer_factor=2):
        cb = _CB(element, shape, buffer_factor)
        cbs.append(cb)
        return cb

    class _Math:
        @staticmethod
        def broadcast(block, out=None, dims=None):
            """Two forms.  With `out` (the compiler's only form,
            python/ttl/operators.py:333-360; unary_bcast Row / Col / Scalar,
            TTLElementwiseOps.def:82): every tile replaced by its row 0 (dims
            [0]), column 0 ([1]) or element [0, 0] ([0, 1]) repeated over the
            tile, and a size-1 block dimension along a broadcast dim repeated
            to `out`'s block size.  Without `out` (the simulator's form,
            python/sim/math.py:20-106): validation only (each broadcast block
            dim must be 1), the block returned unchanged, and the enclosing
            binary op broadcasts over the tile grid and inside size-1 tiles."""
            if dims is None:
                raise ValueError("dims parameter is required for broadcast()")
            t = _tiles_of(block)
            if out is None:
                for d in dims:
                    if d >= len(t.shape):
                        raise ValueError(f"Cannot broadcast along dimension {d}: block has shape "
                                         f"{t.shape} with only {len(t.shape)} dimensions")
                    if t.shape[d] != 1:
                        raise ValueError(f"Cannot broadcast along dimension {d}: dimension must "
                                         f"have size 1, but has size {t.shape[d]}")
                return _Tiles([x.clone() for x in t.tiles], t.shape)
            target = tuple(out.shape)
            for d in dims:
                if t.shape[d] != 1 and target[d] != t.shape[d]:
                    raise ValueError("broadcast dimension must have size 1")

            def rep(x):
                if 0 in dims:
                    x = x[:1, :].expand(x.shape[0], x.shape[1])
                if 1 in dims:
                    x = x[:, :1].expand(x.shape[0], x.shape[1])
                return x.clone()
            tiles = [rep(x) for x in t.tiles]
            R, C = t.shape
            nr = target[0] if (0 in dims and R == 1) else R
            nc = target[1] if (1 in dims and C == 1) else C
            tiles = [tiles[(i if R > 1 else 0) * C + (j if C > 1 else 0)]
                     for i in range(nr) for j in range(nc)]
            return _Tiles(tiles, (nr, nc))

    for name, fn in (("exp", torch.exp), ("log", torch.log), ("sqrt", torch.sqrt),
                     ("rsqrt", torch.rsqrt), ("tanh", torch.tanh), ("abs", torch.abs),
                     ("neg", torch.neg), ("relu", torch.relu), ("sigmoid", torch.sigmoid),
                     ("recip", torch.reciprocal)):
        setattr(_Math, name, staticmethod(lambda x, _f=fn: _tiles_of(x).map(_f)))
    _Math.max = staticmethod(lambda a, b: _tiles_of(a)._bin(b, torch.maximum))
    _Math.min = staticmethod(lambda a, b: _tiles_of(a)._bin(b, torch.minimum))
    # the spec's further math functions (TTLangSpecification.md:700-750) as
    # the torch functions it links, one op per tile in the tile dtype
    from oracle.tile_ops import PARAM_UNARY, UNARY
    for name in ("exp2", "expm1", "logp1", "sin", "cos", "tan", "asin", "acos", "atan", "asinh",
                 "acosh", "atanh", "gelu", "silu", "softsign", "hardsigmoid"):
        setattr(_Math, name, staticmethod(lambda x, _f=UNARY[name]: _tiles_of(x).map(_f)))
    _Math.square = staticmethod(lambda x: _tiles_of(x).map(torch.square))
    _Math.rsub = staticmethod(lambda a, b: _tiles_of(a).map(lambda t: b - t))
    _Math.relu_max = staticmethod(
        lambda x, u: _tiles_of(x).map(lambda t: torch.relu(torch.clamp(t, max=u))))
    _Math.relu_min = staticmethod(
        lambda x, lo: _tiles_of(x).map(lambda t: torch.relu(torch.clamp(t, min=lo))))
    _Math.hardtanh = staticmethod(lambda x, mn, mx: _tiles_of(x).map(
        lambda t: torch.nn.functional.hardtanh(t, mn, mx)))
    _Math.leaky_relu = staticmethod(lambda x, s: _tiles_of(x).map(
        lambda t: torch.nn.functional.leaky_relu(t, s)))
    _Math.prelu = staticmethod(_Math.leaky_relu)
    _Math.elu = staticmethod(lambda x, a: _tiles_of(x).map(lambda t: PARAM_UNARY["elu"](t, a, 0)))
    _Math.celu = staticmethod(lambda x, a, _ar=None: _tiles_of(x).map(
        lambda t: PARAM_UNARY["celu"](t, a, 0)))
    _Math.selu = staticmethod(lambda x, sc, a: _tiles_of(x).map(
        lambda t: PARAM_UNARY["selu"](t, sc, a)))
    _Math.softplus = staticmethod(lambda x, beta, _br=None, threshold=20.0: _tiles_of(x).map(
        lambda t: PARAM_UNARY["softplus"](t, beta, threshold)))
    _Math.reduce_sum = staticmethod(lambda x, scaler, dims=None: _reduce("sum", x, scaler, dims))
    _Math.reduce_max = staticmethod(lambda x, scaler, dims=None: _reduce("max", x, scaler, dims))

    def kernel(grid="auto"):
        actual = (8, 8) if grid == "auto" else tuple(grid)

        def deco(func):
            def run(*args, **kwargs):
                registry.clear()
                cbs.clear()
                g = dict(func.__globals__)
                g["grid"] = actual
                body = types.FunctionType(func.__code__, g, func.__name__, func.__defaults__,
                                          func.__closure__)
                state.grid = actual
                body(*args, **kwargs)
                threads = list(registry)
                if len(threads) != 3:
                    raise ValueError("Kernel must define exactly 3 threads (compute, dm0, dm1), "
                                     f"got {len(threads)}")
                ncores = 1
                for d in actual:
                    ncores *= d
                for c in range(ncores):
                    for cb in cbs:
                        cb.reset()
                    errors = []

                    def runner(f, c=c):
                        state.grid = actual
                        state.core = c
                        try:
                            f()
                        except BaseException as e:  # surfaced after join
                            errors.append(e)

                    ts = [threading.Thread(target=runner, args=(f,)) for _, f in threads]
                    for t in ts:
                        t.start()
                    for t in ts:
                        t.join()
                    if errors:
                        raise errors[0]
            return run
        return deco

    ns.kernel = kernel
    ns.grid_size = grid_size
    ns.core = core
    ns.compute = compute
    ns.datamovement = datamovement
    ns.make_circular_buffer_like = make_cb
    ns.copy = _copy
    ns.math = _Math()
    return ns
