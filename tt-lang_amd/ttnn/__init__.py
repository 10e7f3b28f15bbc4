"""Drop-in `ttnn` for tt-lang kernels running on one MI355X.

Mirrors the subset of ttnn that tt-lang programs use (the surface of the
reference simulator's ttnn stand-in, python/sim/ttnnsim.py): device
open/close, a Tensor wrapper with tile indexing, tensor creation and
conversion, dtypes / layouts / memory configs, core-grid helpers and
split_work_to_cores, plus elementwise ttnn ops.

Storage: a Tensor wraps a torch tensor that lives in HBM on the GPU (torch
for allocation and interop only).  Layout is row-major; "TILE_LAYOUT" is a
logical 32x32 tiling (the kernels address tiles in place).  Without a GPU
(CPU-only hosts) tensors stay in host memory so kernels can still be traced
and planned; running a kernel then raises.
"""

from __future__ import annotations

import operator as _op
from typing import Any, List, Optional, Sequence, Tuple, Union

import torch

TILE_SIZE = 32
TILE_SHAPE = (32, 32)


class _Layout:
    def __init__(self, name: str):
        self.name = name

    def __repr__(self) -> str:
        return f"Layout.{self.name}"


TILE_LAYOUT = _Layout("TILE")
ROW_MAJOR_LAYOUT = _Layout("ROW_MAJOR")
class MemoryConfig:
    """Where a ttnn tensor lives (DRAM or L1, interleaved).  On the MI355X
    every tensor is in HBM; the config is kept only so programs can read it
    back (tensor.memory_config())."""

    def __init__(self, buffer_type: str, layout: str = "INTERLEAVED") -> None:
        self.buffer_type = buffer_type
        self.memory_layout = layout

    def __repr__(self) -> str:
        return (f"MemoryConfig(memory_layout=TensorMemoryLayout::{self.memory_layout}, "
                f"buffer_type=BufferType::{self.buffer_type})")

    def __eq__(self, o) -> bool:
        return isinstance(o, MemoryConfig) and (o.buffer_type, o.memory_layout) == (
            self.buffer_type, self.memory_layout)

    def __hash__(self) -> int:
        return hash((self.buffer_type, self.memory_layout))


DRAM_MEMORY_CONFIG = MemoryConfig("DRAM")
L1_MEMORY_CONFIG = MemoryConfig("L1")

bfloat16 = torch.bfloat16
float32 = torch.float32


class BlockFloatType:
    """A block-floating-point tile format (ttnn.bfloat8_b): tensors of this
    dtype hold packed 32x32 tiles, `tile_bytes` each (the reference fixes the
    size, python/ttl/dtype_utils.py:151-181).  Arithmetic on them happens in
    bfloat16 (`compute_dtype`)."""

    compute_dtype = torch.bfloat16

    def __init__(self, name: str, tile_bytes: int, codec: str):
        self.name = name
        self.tile_bytes = tile_bytes
        self.codec = codec  # "bfp8" | "bfp4": the ttlhip.kernels function prefix

    def __repr__(self) -> str:
        return f"DataType.{self.name.upper()}"

    def _fn(self, what: str):
        from ttlhip import kernels as K

        return getattr(K, f"{self.codec}_{what}")

    def pack(self, t: torch.Tensor) -> torch.Tensor:
        """fp32 [rows, cols] (host) -> packed tile bytes (host)."""
        return self._fn("pack_host")(t)

    def unpack(self, q: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
        """Packed tiles -> bf16 [rows, cols] on q's device."""
        if q.is_cuda:
            return self._fn("unpack")(q, rows, cols)
        return self._fn("unpack_host")(q, rows, cols)

    def matmul(self, a: torch.Tensor, q: torch.Tensor, c: torch.Tensor, stream=None) -> None:
        """c = a @ dequant(q) on the GPU (bf16 a and c)."""
        from ttlhip import kernels as K

        (K.matmul_bfp8w if self.codec == "bfp8" else K.matmul_bfp4w)(a, q, c, stream=stream)


bfloat8_b = BlockFloatType("bfloat8_b", 1088, "bfp8")
bfloat4_b = BlockFloatType("bfloat4_b", 576, "bfp4")

TTNN_AVAILABLE = True

# While a ttl.kernel body runs, the tensors it creates are appended here, so a
# cached kernel plan can be bound to the same tensors of a later call (the
# body is run again; tensors are matched by creation order).
_created: Optional[List["Tensor"]] = None


def _device() -> torch.device:
    return torch.device("cuda") if torch.cuda.is_available() else torch.device("cpu")


class Tensor:
    """ttnn tensor: a torch tensor in device memory with tt-lang tile indexing.

    `t[r, c]`, `t[r0:r1, c0:c1]` (tile coordinates, explicit start/stop, no
    step; python/sim/tensoraccessor.py:85-159) return a TensorSlice that
    ttl.copy moves between the tensor and a circular-buffer block.
    """

    def __init__(self, tensor: torch.Tensor, *, block: Optional[BlockFloatType] = None,
                 logical_shape: Optional[Tuple[int, ...]] = None, layout: Any = None) -> None:
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"ttnn.Tensor wraps a torch.Tensor, got {type(tensor)}")
        self._tensor = tensor
        # storage stays row-major either way (the kernels address it so); the
        # layout is the one the tensor was created / converted with, checked
        # at kernel calls like the reference's compiled path does
        self._layout = TILE_LAYOUT if layout is None else layout
        if _created is not None:  # created while a kernel body runs
            _created.append(self)
        # block-float tensors: _tensor holds the packed tile bytes (uint8)
        self._block = block
        self._logical_shape = tuple(logical_shape) if logical_shape is not None else None
        self._memory_config = DRAM_MEMORY_CONFIG

    def memory_config(self) -> MemoryConfig:
        return self._memory_config

    # -- metadata -----------------------------------------------------------
    @property
    def shape(self) -> Tuple[int, ...]:
        if self._block is not None:
            return self._logical_shape
        return tuple(self._tensor.shape)

    @property
    def dtype(self):
        return self._block if self._block is not None else self._tensor.dtype

    @property
    def is_block_float(self) -> bool:
        return self._block is not None

    @property
    def layout(self):
        return self._layout

    def tiled_data(self) -> torch.Tensor:
        """The tensor in tilized element order (32x32 tiles row-major over the
        tile grid, four 16x16 faces each: the storage order of a TILE_LAYOUT
        ttnn tensor), as a 1-D device tensor; block-float tensors return their
        packed tile bytes."""
        if self._block is not None:
            return self._tensor
        from ttlhip import kernels as K

        return K.tilize(self._tensor)

    def to_torch(self) -> torch.Tensor:
        """Host copy; block-float tensors come back as float32 values (the
        conversion ttnn.to_torch applies to bfloat8_b)."""
        if self._block is not None:
            rows, cols = self._logical_shape
            return self._block.unpack(self._tensor, rows, cols).float().cpu()
        return self._tensor.detach().cpu()

    def __repr__(self) -> str:
        return f"ttnn.Tensor(shape={self.shape}, dtype={self.dtype}, device={self._tensor.device})"

    # -- tile indexing ------------------------------------------------------
    def _tile_indexable(self) -> bool:
        if len(self.shape) != 2:
            return False
        return all(d == 1 or d % t == 0 for d, t in zip(self.shape, TILE_SHAPE))

    def __getitem__(self, key: Any):
        if isinstance(key, tuple) and len(key) == 2 and self._tile_indexable():
            from ttlhip.trace import TensorSlice, is_index

            if all(is_index(k) for k in key):
                return TensorSlice.from_key(self, key)
        if self._block is not None:
            raise TypeError(f"a {self._block.name} tensor is indexed by tiles only")
        return Tensor(self._tensor[key])

    def __setitem__(self, key: Any, value: Any) -> None:
        if isinstance(value, Tensor):
            value = value._tensor
        self._tensor[key] = value

    # -- host-side arithmetic (user code around kernels, e.g. goldens) -------
    def _binop(self, other: Any, fn, reverse: bool = False) -> "Tensor":
        o = other._tensor if isinstance(other, Tensor) else other
        if isinstance(o, torch.Tensor) and o.device != self._tensor.device:
            o = o.to(self._tensor.device)
        return Tensor(fn(o, self._tensor) if reverse else fn(self._tensor, o))

    def __add__(self, o): return self._binop(o, _op.add)
    def __sub__(self, o): return self._binop(o, _op.sub)
    def __mul__(self, o): return self._binop(o, _op.mul)
    def __truediv__(self, o): return self._binop(o, _op.truediv)
    def __floordiv__(self, o): return self._binop(o, _op.floordiv)
    def __mod__(self, o): return self._binop(o, _op.mod)
    def __pow__(self, o): return self._binop(o, _op.pow)
    def __matmul__(self, o): return self._binop(o, _op.matmul)
    def __radd__(self, o): return self._binop(o, _op.add, True)
    def __rsub__(self, o): return self._binop(o, _op.sub, True)
    def __rmul__(self, o): return self._binop(o, _op.mul, True)
    def __rtruediv__(self, o): return self._binop(o, _op.truediv, True)
    def __neg__(self): return Tensor(-self._tensor)


# ---------------------------------------------------------------------------
# device


class Device:
    def __init__(self, device_id: int = 0) -> None:
        self.device_id = device_id

    def __repr__(self) -> str:
        return f"Device(id={self.device_id}, MI355X)"

    def compute_with_storage_grid_size(self) -> "CoreCoord":
        """The logical core grid tt-lang programs see: (8, 8), the simulator's
        "auto" grid (python/sim/ttnnsim.py:215-226).  The MI355X executes the
        whole tile program grid-wide regardless."""
        return CoreCoord(8, 8)


def open_device(device_id: int = 0, **_: Any) -> Device:
    return Device(device_id)


def close_device(device: Device) -> None:
    return None


def synchronize_device(device: Optional[Device] = None) -> None:
    if torch.cuda.is_available():
        torch.cuda.synchronize()


# ---------------------------------------------------------------------------
# creation / conversion


def _shape(shape: Union[Sequence[int], int]) -> Tuple[int, ...]:
    return (shape,) if isinstance(shape, int) else tuple(shape)


def _block_from_fp32(t: torch.Tensor, block: BlockFloatType) -> Tensor:
    """fp32 [rows, cols] -> packed tiles in device memory (host codec)."""
    if t.dim() != 2:
        raise ValueError(f"{block.name} tensors are 2-D, got shape {tuple(t.shape)}")
    packed = block.pack(t.to(torch.float32))
    return Tensor(packed.to(_device()), block=block, logical_shape=tuple(t.shape))


def rand(shape, dtype=bfloat16, layout: Any = None, **_: Any) -> Tensor:
    """U[0, 1) drawn in fp32 from torch's global generator, then cast - the
    same stream and rounding as python/sim/ttnnsim.py:521-531."""
    t = torch.rand(_shape(shape), dtype=torch.float32)
    if isinstance(dtype, BlockFloatType):
        return _block_from_fp32(t, dtype)
    return Tensor(t.to(dtype).to(_device()), layout=layout)


def empty(shape, dtype=bfloat16, layout: Any = None, **_: Any) -> Tensor:
    if isinstance(dtype, BlockFloatType):
        return _block_from_fp32(torch.zeros(_shape(shape)), dtype)
    return Tensor(torch.empty(_shape(shape), dtype=dtype, device=_device()), layout=layout)


def zeros(shape, dtype=bfloat16, layout: Any = None, **_: Any) -> Tensor:
    if isinstance(dtype, BlockFloatType):
        return _block_from_fp32(torch.zeros(_shape(shape)), dtype)
    return Tensor(torch.zeros(_shape(shape), dtype=dtype, device=_device()), layout=layout)


def ones(shape, dtype=bfloat16, layout: Any = None, **_: Any) -> Tensor:
    if isinstance(dtype, BlockFloatType):
        return _block_from_fp32(torch.ones(_shape(shape)), dtype)
    return Tensor(torch.ones(_shape(shape), dtype=dtype, device=_device()), layout=layout)


def full(shape, fill_value: float, dtype=bfloat16, layout: Any = None, **_: Any) -> Tensor:
    if isinstance(dtype, BlockFloatType):
        return _block_from_fp32(torch.full(_shape(shape), float(fill_value)), dtype)
    return Tensor(torch.full(_shape(shape), fill_value, dtype=dtype, device=_device()),
                  layout=layout)


def zeros_like(t: Tensor, dtype=None, **_: Any) -> Tensor:
    return Tensor(torch.zeros_like(t._tensor, dtype=dtype), layout=t.layout)


def empty_like(t: Tensor, dtype=None, **_: Any) -> Tensor:
    return Tensor(torch.empty_like(t._tensor, dtype=dtype), layout=t.layout)


def from_torch(tensor: torch.Tensor, dtype=None, layout: Any = None,
               device: Any = None, memory_config: Any = None, **_: Any) -> Tensor:
    """Device copy of `tensor`; dtype=ttnn.bfloat8_b / bfloat4_b quantises it
    into packed tiles (shared exponent per 16-element face row, round half to
    even)."""
    t = tensor.detach()
    if isinstance(dtype, BlockFloatType):
        return _block_from_fp32(t.cpu(), dtype)
    if dtype is not None:
        t = t.to(dtype)
    out = Tensor(t.to(_device()).contiguous(), layout=layout)
    if isinstance(memory_config, MemoryConfig):
        out._memory_config = memory_config
    return out


def from_tiled_data(data: torch.Tensor, shape: Sequence[int], dtype=None,
                    **_: Any) -> Tensor:
    """A tensor from elements in tilized order (see Tensor.tiled_data), e.g.
    the storage of a TILE_LAYOUT ttnn tensor read from a file or another
    process."""
    from ttlhip import kernels as K

    rows, cols = (int(d) for d in shape)
    d = data.detach()
    if dtype is not None:
        d = d.to(dtype)
    return Tensor(K.untilize(d.to(_device()).reshape(-1), rows, cols))


def to_torch(t: Union[Tensor, torch.Tensor], **_: Any) -> torch.Tensor:
    if isinstance(t, Tensor):
        return t.to_torch()
    return t


def to_memory_config(t: Tensor, memory_config: Any = None, **_: Any) -> Tensor:
    """A copy of `t` tagged with `memory_config` (ttnn moves the data; here
    every tensor stays in HBM, so only the tag differs)."""
    if t.is_block_float:
        out = Tensor(t._tensor.clone(), block=t._block, logical_shape=t.shape, layout=t._layout)
    else:
        out = Tensor(t._tensor.clone(), layout=t._layout)
    if isinstance(memory_config, MemoryConfig):
        out._memory_config = memory_config
    return out


def to_layout(t: Tensor, layout: Any, **_: Any) -> Tensor:
    """The same data with `layout` (TILE_LAYOUT / ROW_MAJOR_LAYOUT); storage is
    row-major in both, see Tensor.tiled_data for the tilized element order."""
    if t.is_block_float:
        if "TILE" not in str(layout):
            raise ValueError(f"a {t.dtype.name} tensor exists in TILE_LAYOUT only")
        return t
    return Tensor(t._tensor, layout=layout)


def tilize(t: Tensor, **_: Any) -> Tensor:
    return to_layout(t, TILE_LAYOUT)


def untilize(t: Tensor, **_: Any) -> Tensor:
    return to_layout(t, ROW_MAJOR_LAYOUT)


def repeat(t: Tensor, repeats: Sequence[int], **_: Any) -> Tensor:
    """torch.Tensor.repeat semantics (leading dimensions added as needed)."""
    if t.is_block_float:
        raise NotImplementedError("ttnn.repeat of a block-float tensor")
    return Tensor(t._tensor.repeat(*[int(r) for r in repeats]))


def squeeze(t: Tensor, dim: Optional[int] = None, **_: Any) -> Tensor:
    if t.is_block_float:
        raise NotImplementedError("ttnn.squeeze of a block-float tensor")
    return Tensor(t._tensor.squeeze() if dim is None else t._tensor.squeeze(dim))


def reshape(t: Tensor, shape: Sequence[int], **_: Any) -> Tensor:
    if t.is_block_float:
        raise NotImplementedError("ttnn.reshape of a block-float tensor")
    return Tensor(t._tensor.reshape(tuple(shape)))


def typecast(t: Tensor, dtype, **_: Any) -> Tensor:
    """Converts between bfloat16 / float32 and the block-float formats."""
    if isinstance(dtype, BlockFloatType):
        return _block_from_fp32(t.to_torch().float(), dtype)
    if t.is_block_float:
        return Tensor(t.to_torch().to(dtype).to(_device()))
    return Tensor(t._tensor.to(dtype))


def matmul(a: Tensor, b: Tensor, **_: Any) -> Tensor:
    """a @ b on the MI355X (bf16 / f32 MFMA, fp32 accumulation; a block-float
    `b` goes through the bf16 x bfloat8_b GEMM or, for bfloat4_b, a
    dequantisation pass and the bf16 GEMM).  The result is bfloat16 for
    bfloat16 / block-float inputs, float32 for float32 ones."""
    from ttlhip import _lib
    from ttlhip import kernels as K

    _lib.require_device()
    if a.is_block_float:
        raise NotImplementedError("ttnn.matmul takes a block-float tensor as the second operand only")
    ta = a._tensor.contiguous()
    M, Ka = ta.shape
    Kb, N = b.shape
    if Ka != Kb:
        raise ValueError(f"matmul shapes {tuple(ta.shape)} @ {tuple(b.shape)} do not chain")
    if b.is_block_float:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=ta.device)
        b.dtype.matmul(ta.to(torch.bfloat16), b._tensor, out)
        return Tensor(out)
    tb = b._tensor.contiguous()
    out_dtype = torch.float32 if torch.float32 in (ta.dtype, tb.dtype) else torch.bfloat16
    if ta.dtype != tb.dtype:
        ta, tb = ta.to(out_dtype), tb.to(out_dtype)
    out = torch.empty((M, N), dtype=out_dtype, device=ta.device)
    K.matmul(ta, tb, out)
    return Tensor(out)


def to_device(t: Tensor, device: Any = None, **_: Any) -> Tensor:
    return t


def from_device(t: Tensor, **_: Any) -> Tensor:
    return t


def isclose(a: Tensor, b: Tensor, rtol: float = 1e-05, atol: float = 1e-08,
            equal_nan: bool = False) -> Tensor:
    ta = a._tensor if isinstance(a, Tensor) else a
    tb = b._tensor if isinstance(b, Tensor) else b
    if isinstance(tb, torch.Tensor) and isinstance(ta, torch.Tensor) and tb.device != ta.device:
        tb = tb.to(ta.device)
    return Tensor(torch.isclose(ta, tb, rtol=rtol, atol=atol, equal_nan=equal_nan))


# ---------------------------------------------------------------------------
# elementwise ttnn ops, executed by the MI355X eltwise kernel


def _eltwise(op: str, a: Tensor, b: Optional[Tensor]) -> Tensor:
    from ttlhip import _lib, expr as X
    from ttlhip.kernels import OperandMap, eltwise

    _lib.require_device()
    ta = a._tensor.contiguous()
    leaves = [X.Leaf(OperandMap(ta), ta.dtype)]
    shape = list(ta.shape)
    if b is not None:
        tb = b._tensor.contiguous()
        if ta.dim() != 2 or tb.dim() != 2:
            raise ValueError("ttnn elementwise ops take 2-D tensors")
        for i in range(2):
            if ta.shape[i] != tb.shape[i] and 1 not in (ta.shape[i], tb.shape[i]):
                raise ValueError(f"shapes {tuple(ta.shape)} and {tuple(tb.shape)} do not broadcast")
            shape[i] = max(ta.shape[i], tb.shape[i])
        leaves.append(X.Leaf(OperandMap(tb), tb.dtype))
        e = X.Binary(op, leaves[0], leaves[1], X.promote(ta.dtype, tb.dtype))
    else:
        e = X.Unary(op, leaves[0], ta.dtype)
    out = torch.empty(shape, dtype=e.dtype, device=ta.device)
    prog = X.compile_expr(e)
    eltwise(prog, [s.leaf.ref if s.leaf is not None else None for s in prog.steps], out)
    return Tensor(out)


def add(a: Tensor, b: Tensor, **_: Any) -> Tensor: return _eltwise("add", a, b)
def subtract(a: Tensor, b: Tensor, **_: Any) -> Tensor: return _eltwise("sub", a, b)
def multiply(a: Tensor, b: Tensor, **_: Any) -> Tensor: return _eltwise("mul", a, b)
def divide(a: Tensor, b: Tensor, **_: Any) -> Tensor: return _eltwise("div", a, b)
def maximum(a: Tensor, b: Tensor, **_: Any) -> Tensor: return _eltwise("max", a, b)
def minimum(a: Tensor, b: Tensor, **_: Any) -> Tensor: return _eltwise("min", a, b)
def exp(a: Tensor, **_: Any) -> Tensor: return _eltwise("exp", a, None)
def log(a: Tensor, **_: Any) -> Tensor: return _eltwise("log", a, None)
def sqrt(a: Tensor, **_: Any) -> Tensor: return _eltwise("sqrt", a, None)
def rsqrt(a: Tensor, **_: Any) -> Tensor: return _eltwise("rsqrt", a, None)
def tanh(a: Tensor, **_: Any) -> Tensor: return _eltwise("tanh", a, None)
def abs(a: Tensor, **_: Any) -> Tensor: return _eltwise("abs", a, None)  # noqa: A001
def neg(a: Tensor, **_: Any) -> Tensor: return _eltwise("neg", a, None)
def relu(a: Tensor, **_: Any) -> Tensor: return _eltwise("relu", a, None)
def sigmoid(a: Tensor, **_: Any) -> Tensor: return _eltwise("sigmoid", a, None)
def reciprocal(a: Tensor, **_: Any) -> Tensor: return _eltwise("recip", a, None)


# ---------------------------------------------------------------------------
# core grid helpers (python/sim/ttnnsim.py:111-189)


class CoreCoord:
    def __init__(self, x: int, y: int):
        self.x = x
        self.y = y

    def __repr__(self) -> str:
        return f"CoreCoord(x={self.x}, y={self.y})"

    def __eq__(self, other: object) -> bool:
        return isinstance(other, CoreCoord) and self.x == other.x and self.y == other.y

    def __hash__(self) -> int:
        return hash((self.x, self.y))


class CoreRange:
    def __init__(self, start: CoreCoord, end: CoreCoord):
        self.start = start
        self.end = end

    def __repr__(self) -> str:
        return f"CoreRange(start={self.start}, end={self.end})"

    def num_cores(self) -> int:
        return (self.end.x - self.start.x + 1) * (self.end.y - self.start.y + 1)


class CoreRangeSet:
    def __init__(self, ranges: List[CoreRange]):
        self._ranges = list(ranges)

    def ranges(self) -> List[CoreRange]:
        return self._ranges

    def num_cores(self) -> int:
        return sum(r.num_cores() for r in self._ranges)

    def __repr__(self) -> str:
        return f"CoreRangeSet(ranges={self._ranges})"


def _ordered_cores(core_grid: Union[CoreCoord, CoreRangeSet], row_wise: bool) -> List[CoreCoord]:
    if isinstance(core_grid, CoreCoord):
        if row_wise:
            return [CoreCoord(x, y) for y in range(core_grid.y) for x in range(core_grid.x)]
        return [CoreCoord(x, y) for x in range(core_grid.x) for y in range(core_grid.y)]
    out = []
    for r in core_grid.ranges():
        ys, xs = range(r.start.y, r.end.y + 1), range(r.start.x, r.end.x + 1)
        if row_wise:
            out.extend(CoreCoord(x, y) for y in ys for x in xs)
        else:
            out.extend(CoreCoord(x, y) for x in xs for y in ys)
    return out


def split_work_to_cores(core_grid: Union[CoreCoord, CoreRangeSet], units_to_divide: int,
                        row_wise: bool = False):
    """Divides `units_to_divide` work units over the cores of `core_grid`.

    Same assignment as the reference (python/sim/ttnnsim.py:583-752): min(cores,
    units) cores are used; with a remainder, the first `remainder` cores
    (group 1) get one unit more than the rest (group 2); cores are taken y-outer
    / x-inner when row_wise (x-outer otherwise), range by range for a
    CoreRangeSet.  (The simulator takes a CoreRangeSet's cores y-outer either
    way; tt-metal's ttnn, which the reference's hardware tests compare with,
    test/python/test_block_allocation.py:54-120, honours row_wise.)  Each
    group lists single-core ranges.
    Returns (num_cores, all_cores, group_1, group_2, units_1, units_2).
    """
    if isinstance(core_grid, CoreCoord):
        n_cores = core_grid.x * core_grid.y
        all_cores = CoreRangeSet([CoreRange(CoreCoord(0, 0),
                                            CoreCoord(core_grid.x - 1, core_grid.y - 1))])
    else:
        n_cores = core_grid.num_cores()
        all_cores = core_grid
    used = min(n_cores, units_to_divide)
    if used == 0:
        e = CoreRangeSet([])
        return 0, e, e, e, 0, 0
    base, rem = divmod(units_to_divide, used)
    if rem:
        u1, u2, n1 = base + 1, base, rem
    else:
        u1, u2, n1 = base, 0, used
    cores = _ordered_cores(core_grid, row_wise)[:used]
    g1 = CoreRangeSet([CoreRange(c, c) for c in cores[:n1]])
    g2 = CoreRangeSet([CoreRange(c, c) for c in cores[n1:used]])
    return used, all_cores, g1, g2, u1, u2


def num_cores_to_corerangeset(n: int, grid: CoreCoord, row_wise: bool = False) -> CoreRangeSet:
    return CoreRangeSet([CoreRange(c, c) for c in _ordered_cores(grid, row_wise)[:n]])
