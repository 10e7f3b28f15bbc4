"""From traced thread events to MI355X kernel launches.

A circular buffer is a FIFO between exactly one producer and one consumer
thread (python/sim/cb.py:302-408, one pending block per side), so the n-th
block a producer reserves is the n-th block its consumer waits on.  With the
block indices the tracer assigns, every stored tile resolves to

    output tensor tile  <-  store(expr, acc)  <-  leaf blocks  <-  input tensor tiles

as numpy arrays over all cores and loop iterations at once.  Each store site
becomes one launch:
  * every output tile written once by an elementwise expression -> one
    ttlh_eltwise over the covered rectangle, operands addressed as identity
    (+offset), fixed-tile reuse or size-1 broadcast (what the simulator's
    block broadcasting and degenerate tiles produce);
  * A(m,k) @ B(k,n) accumulated with store(acc=True) over all k into every
    output tile of a rectangle -> one ttlh_matmul;
  * ttl.math.reduce_sum / reduce_max of an elementwise expression, every
    output tile reducing the same contiguous run of expression tiles (one
    block, or several accumulated with store(acc=True) for sums) -> one
    ttlh_reduce.
Six consecutive store sites that spell out attention over intermediate CBs
(S = Q K^T, M = row max, P = exp(S*scale - M), L = row sum of P, O = P V,
Y = O / L, every tile where the attention indexing puts it) become one
ttlh_sdpa_fwd instead (_match_attention).
Anything else raises NotImplementedError naming the unsupported pattern.
"""

from __future__ import annotations

import dataclasses
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from . import dsl as D
from . import expr as X
from . import trace as T

TILE = 32


class PlanError(NotImplementedError):
    """The traced tile program uses a pattern the MI355X backend does not run."""


# ---------------------------------------------------------------------------
# launches


@dataclass
class TensorRef:
    """A tensor the plan reads or writes: kernel argument `arg` (by position or
    name), a tensor the kernel body created (arg = ("created", i), i-th in
    creation order; obj = the trace-time one) or, for tensors captured from
    an enclosing scope, the object."""

    arg: Any = None
    obj: Any = None

    def resolve(self, args: Dict[Any, Any]):
        t = self.resolve_obj(args)
        return t._tensor if hasattr(t, "_tensor") else t

    def resolve_obj(self, args: Dict[Any, Any]):
        if self.arg is None:
            return self.obj
        if isinstance(self.arg, tuple) and self.arg not in args:
            return self.obj  # a body-created tensor: the one from the trace
        return args[self.arg]


@dataclass
class OperandSpec:
    ref: TensorRef
    row_mask: int
    col_mask: int
    row_off: int
    col_off: int


@dataclass
class EltwiseLaunch:
    prog: X.StackProgram
    operands: List[Optional[OperandSpec]]  # per step
    out: TensorRef
    region: Tuple[int, int, int, int]      # y0, x0, h, w (elements)
    tiles: int = 0
    loc: Optional[Tuple[str, int]] = None  # kernel source line of the store()

    def describe(self) -> str:
        return (f"eltwise {len(self.prog.steps)} steps over {self.region[2]}x{self.region[3]} "
                f"elements at ({self.region[0]}, {self.region[1]})")


@dataclass
class MatmulLaunch:
    a: TensorRef
    b: TensorRef
    c: TensorRef
    rows: Tuple[int, int]   # output element rows [r0, r1)
    cols: Tuple[int, int]   # output element cols [c0, c1)
    k: int
    b_block: bool = False   # B is a block-float (bfloat8_b / bfloat4_b) tensor
    loc: Optional[Tuple[str, int]] = None  # kernel source line of the store()
    a_rows: Optional[Tuple[int, int]] = None  # A element rows (default: `rows`)
    b_cols: Optional[Tuple[int, int]] = None  # B element cols (default: `cols`)
    k_range: Optional[Tuple[int, int]] = None  # A cols / B rows summed (default: [0, k))

    def describe(self) -> str:
        return (f"matmul C[{self.rows[0]}:{self.rows[1]}, {self.cols[0]}:{self.cols[1]}] = "
                f"A . B over K={self.k}")

    def operand_ranges(self) -> Tuple[Tuple[int, int], Tuple[int, int]]:
        return self.a_rows or self.rows, self.b_cols or self.cols

    def k_slice(self) -> slice:
        k0, k1 = self.k_range or (0, self.k)
        return slice(k0, k1)


@dataclass
class FusedMatmulLaunch:
    """A tile matmul into a plan-owned tensor followed by the elementwise
    launch that alone reads it, at each output element itself (the product
    of `relu(a @ b + c)` and the like, laid out like the output): one
    ttlh_matmul_eltwise launch, the product rounded to its dtype and handed
    to the program in registers, never stored.  Where that entry point does
    not take the problem (small GEMMs, ops outside its set) the two launches
    run as planned."""

    mm: MatmulLaunch
    ew: EltwiseLaunch
    prod_step: int          # the program step that reads the product
    loc: Optional[Tuple[str, int]] = None

    def describe(self) -> str:
        return (f"{self.mm.describe()} with the store's {len(self.ew.prog.steps)}-step "
                "program fused into the epilogue")


@dataclass
class ReduceLaunch:
    prog: X.StackProgram
    operands: List[Optional[OperandSpec]]  # per step, addressed from iteration (y, x)
    out: TensorRef
    kind: str                              # "sum" or "max"
    dims: Tuple[int, ...]                  # reduced axes
    region: Tuple[int, int, int, int]      # iteration y0, x0, h, w (elements)
    out_origin: Tuple[int, int]            # first result element of `out`
    out_pad: bool                          # whole zero-padded 32-wide result tiles
    scaler: Optional[TensorRef] = None     # tensor holding the scaler tile, or None
    scaler_at: Tuple[int, int] = (0, 0)    # its element (row, col)
    scale: float = 1.0                     # constant scaler (times the tensor's)
    tiles: int = 0
    loc: Optional[Tuple[str, int]] = None

    def describe(self) -> str:
        return (f"reduce_{self.kind} over dims {list(self.dims)} of {self.region[2]}x"
                f"{self.region[3]} elements at ({self.region[0]}, {self.region[1]})")


@dataclass
class ReduceEltwiseLaunch:
    """Row reductions over one region followed by the elementwise launch
    over the same region that reads their results, e.g. a softmax in one
    store (reduce_max, reduce_sum, then the normalising program): one
    ttlh_reduce_rows_eltwise launch reading each row once, with the results
    of the separate launches in every output.  Where that entry point does
    not take the combination, the launches run as planned."""

    reds: List[ReduceLaunch]
    ew: EltwiseLaunch
    loc: Optional[Tuple[str, int]] = None

    def describe(self) -> str:
        kinds = ", ".join(f"reduce_{r.kind}" for r in self.reds)
        return f"{kinds} and {self.ew.describe()} in one launch"


@dataclass
class SdpaLaunch:
    """Attention spelled out tile by tile with the spec's ops
    (docs/sphinx/specs/TTLangSpecification.md:693-761: @, reduce_max, exp,
    broadcast, reduce_sum, recip): for every 32-row tile of queries of
    Q [B*H*S, D], the S key rows of its head in K (read as K^T [D, B*H*S]),
    Y = softmax(Q K^T * scale) V, as one ttlh_sdpa_fwd over [1, B*H, S, D]."""

    q: TensorRef
    kt: TensorRef           # K^T: the transposed view of a contiguous K [B*H*S, D]
    v: TensorRef
    out: TensorRef
    heads: int              # B*H
    seq: int                # S
    scale: float
    loc: Optional[Tuple[str, int]] = None
    # plan-owned K [B*H*S, D], written from K^T by ttlh_transpose_bf16 when
    # K^T is not the transposed view of contiguous K rows (allocated on the
    # first such call, kept with the cached plan)
    kbuf: Any = None

    def describe(self) -> str:
        return (f"sdpa over {self.heads} heads of {self.seq} rows, scale {self.scale:g} "
                "(fused attention)")


@dataclass
class Plan:
    launches: List[Any] = field(default_factory=list)
    # tensors the kernel body created at trace time (bound by creation order
    # on later calls) and whether any launch refers to one
    created: List[Any] = field(default_factory=list)
    uses_created: bool = False

    def describe(self) -> str:
        return "\n".join(l.describe() for l in self.launches)


# ---------------------------------------------------------------------------
# resolution


@dataclass
class _CopyTable:
    """Per (core, CB): tensor tile origin of every block index."""

    tensor: Any
    r0: np.ndarray
    c0: np.ndarray


def _thread_events(root) -> List[T.Event]:
    return list(T.iter_events(root))


def _copy_table(events: List[T.Event], cb, n: int, kind: str, received=None) -> _CopyTable:
    """Tile origin of every block of `cb` from its copy events; with kind
    "copy_in", blocks delivered by a pipe take their origin from `received`
    (event -> (tensor, r0, c0) arrays over the event's instances)."""
    r0 = np.full(n, -1, dtype=np.int64)
    c0 = np.full(n, -1, dtype=np.int64)
    tensor = None
    for ev in events:
        if ev.cb is not cb:
            continue
        if ev.kind == kind:
            blk, sl = ev.data["block"], ev.data["slice"]
            src_t = sl.tensor
            shape = ev.domain_shape()
            vr = T.broadcast_to_domain(sl.r0, shape).ravel()
            vc = T.broadcast_to_domain(sl.c0, shape).ravel()
        elif kind == "copy_in" and ev.kind == "pipe_recv":
            blk = ev.data["block"]
            shape = ev.domain_shape()
            src_t, vr, vc = received(ev)
        else:
            continue
        if tensor is None:
            tensor = src_t
        elif src_t is not tensor:
            raise PlanError("one circular buffer is filled from / drained to more than one "
                            "tensor on a core; use one CB per tensor")
        idx = T.broadcast_to_domain(blk.event.index, shape).ravel()
        if np.any(r0[idx] >= 0):
            raise PlanError("a block is copied more than once")
        r0[idx] = vr
        c0[idx] = vc
    if n and (tensor is None or np.any(r0 < 0)):
        what = "filled by ttl.copy" if kind == "copy_in" else "copied out"
        raise PlanError(f"every block of CB {cb.id} must be {what} exactly once "
                        "(blocks pushed without a copy are not supported)")
    return _CopyTable(tensor, r0, c0)


class _Temp:
    """A device tensor the plan owns (allocated on first use, then kept with
    the cached plan): the value of a subexpression split off a store whose
    fused program exceeds the kernel's limits, in the output's coordinates."""

    is_block_float = False

    def __init__(self, shape: Tuple[int, int], dtype: torch.dtype) -> None:
        self._shape = tuple(shape)
        self.dtype = dtype
        self._t: Optional[torch.Tensor] = None

    @property
    def shape(self) -> Tuple[int, int]:
        return self._shape

    @property
    def _tensor(self) -> torch.Tensor:
        if self._t is None or tuple(self._t.shape) != tuple(self.shape):
            dev = "cuda" if torch.cuda.is_available() else "cpu"
            self._t = torch.zeros(self.shape, dtype=self.dtype, device=dev)
        return self._t


class _Scratch(_Temp):
    """Device memory standing in for an intermediate CB: one the compute
    thread both stores into and waits on (test/python/test_intermediate_cb.py,
    the two-stage broadcast kernels of test/python/test_bcast_ops.py).  Every
    block of the CB gets its own tiles, placed at the tile coordinates of the
    store that reads it, so the storing launch writes the block there and the
    reading launch finds it where an operand filled by ttl.copy from a tensor
    would be.  The two launches run in trace order (the store first)."""

    def __init__(self, cb):
        if not isinstance(cb.dtype, torch.dtype):
            raise PlanError(f"CB {cb.name}: an intermediate CB of a block-float dtype is not "
                            "supported")
        self.cb = cb
        self.dtype = cb.dtype
        self.rows = 0
        self.cols = 0
        self._tiles: List[np.ndarray] = []
        self._t: Optional[torch.Tensor] = None

    @property
    def shape(self) -> Tuple[int, int]:
        return (self.rows * TILE, self.cols * TILE)

    def place(self, r0: np.ndarray, c0: np.ndarray) -> None:
        R, C = self.cb.shape
        if r0.size:
            self.rows = max(self.rows, int(r0.max()) + R)
            self.cols = max(self.cols, int(c0.max()) + C)
        i, j = np.divmod(np.arange(R * C), C)
        self._tiles.append(np.stack([(r0[:, None] + i[None, :]).ravel(),
                                     (c0[:, None] + j[None, :]).ravel()], 1))

    def check(self) -> None:
        rc = np.concatenate(self._tiles, 0)
        if rc.size and _unique_tiles(rc) != rc.shape[0]:
            raise PlanError(f"CB {self.cb.name}: its blocks are read by stores whose output blocks "
                            "overlap once laid out at the CB's block shape; an intermediate CB "
                            "needs one output block of the reading store per block")



def _intermediate_tables(threads, events, cbs, count, inter, fill, drain,
                         scratch: Dict[int, _Scratch]) -> None:
    """Copy tables of the intermediate CBs `inter` on one core: block k of
    such a CB sits at the output tile origin of the store that reads it
    (resolved through chains of intermediate CBs); the table serves both as
    the CB's drain (for the store into it) and its fill (for the reads)."""
    comp = [tmpl for tmpl, _ in threads if tmpl.kind == "compute"]
    stores = [ev for ev in events[id(comp[0])] if ev.kind == "store"] if comp else []
    inter_set = set(inter)
    state: Dict[int, str] = {}

    def table(cid):
        if cid in drain:
            return drain[cid]
        if state.get(cid) == "busy":
            raise PlanError("intermediate CBs feed each other in a cycle")
        state[cid] = "busy"
        cb = cbs[cid]
        n = count[cid]
        r0 = np.full(n, -1, dtype=np.int64)
        c0 = np.full(n, -1, dtype=np.int64)
        for ev in stores:
            tree = ev.data["expr"].tree
            leaves = _tree_leaves(tree, [])
            if tree[0] == "reduce" and tree[5][0] == "leaf":
                leaves.append(tree[5])
            mine = [lf for lf in leaves if lf[1].cb.id == cid]
            if not mine:
                continue
            target = ev.data["target"]
            tcid = target.cb.id
            if tcid not in drain and tcid not in inter_set:
                raise PlanError(f"CB {target.cb.name} is stored into but never copied to a tensor "
                                "or read by the compute thread")
            dt = table(tcid)
            shape = ev.domain_shape()
            rout = T.broadcast_to_domain(target.event.index, shape).ravel()
            sr, sc = dt.r0[rout], dt.c0[rout]
            for lf in mine:
                w = T.broadcast_to_domain(lf[1].event.index, shape).ravel()
                seen = r0[w] >= 0
                if np.any(seen & ((r0[w] != sr) | (c0[w] != sc))):
                    raise PlanError(f"a block of intermediate CB {cb.name} is read by stores "
                                    "into different output positions")
                r0[w] = sr
                c0[w] = sc
        if np.any(r0 < 0):
            raise PlanError(f"every block stored into CB {cb.name} must be read by a later "
                            "store of the compute thread")
        sc_ = scratch.get(cid)
        if sc_ is None:
            sc_ = scratch[cid] = _Scratch(cb)
        sc_.place(r0, c0)
        tab = _CopyTable(sc_, r0, c0)
        drain[cid] = fill[cid] = tab
        state[cid] = "done"
        return tab

    for cid in inter:
        table(cid)


@dataclass
class _Group:
    """All instances of one store site (same expression, tensors, acc)."""

    tree: Any
    leaf_blocks: List[Any]        # first-core leaf descriptors (for dtypes)
    leaf_tensors: List[Any]
    out_tensor: Any
    acc: bool
    dtype: torch.dtype
    loc: Optional[Tuple[str, int]] = None
    out_rc: List[np.ndarray] = field(default_factory=list)     # [(N,2)]
    leaf_rc: List[List[np.ndarray]] = field(default_factory=list)
    order: List[np.ndarray] = field(default_factory=list)
    # reductions: the scaler's tensor and its tile per store instance
    scaler_tensor: Any = None
    scaler_rc: List[np.ndarray] = field(default_factory=list)
    # repeated store instances may be planned once (_dedupe_writes): set by
    # build_plan when no other store site writes an operand of this one or
    # reads its output, so no value changes between the repeats
    dedupe_ok: bool = True
    # the output is a tensor the plan owns for this site alone (a hoisted
    # matmul operand), read only by the consuming matmul
    private_out: bool = False


def _leaf_rep(leaf) -> Tuple[bool, bool]:
    """(rows, cols) in-tile broadcast flags of an expression leaf (5th item)."""
    return leaf[4] if len(leaf) > 4 else (False, False)


def _tree_leaves(tree, out: List):
    """Leaves of an elementwise tree (of the reduced expression for a
    reduction; its scaler is not an operand)."""
    tag = tree[0]
    if tag == "leaf":
        out.append(tree)
    elif tag == "const":
        pass
    elif tag in ("powi", "upar"):
        _tree_leaves(tree[1], out)
    elif tag == "reduce":
        _tree_leaves(tree[3], out)
    elif tag == "bmatmul":
        _tree_leaves(tree[1], out)
        _tree_leaves(tree[2], out)
    else:
        for t in tree[1:]:
            _tree_leaves(t, out)
    return out


def _tree_key(tree, leaf_ids: Dict[int, int]):
    tag = tree[0]
    if tag == "leaf":
        return ("leaf", leaf_ids.setdefault(id(tree), len(leaf_ids)), str(tree[1].cb.dtype),
                _leaf_rep(tree))
    if tag == "const":
        return ("const", tree[1])
    if tag == "powi":
        return ("powi", _tree_key(tree[1], leaf_ids), tree[2])
    if tag == "upar":
        return ("upar", _tree_key(tree[1], leaf_ids)) + tuple(tree[2:])
    if tag == "reduce":
        _, kind, dims, inner, ishape, scaler = tree
        sk = ("const", scaler[1]) if scaler[0] == "const" else ("scaler", str(scaler[1].cb.dtype))
        return ("reduce", kind, dims, _tree_key(inner, leaf_ids), ishape, sk)
    if tag == "bmatmul":
        return ("bmatmul", _tree_key(tree[1], leaf_ids), _tree_key(tree[2], leaf_ids), tree[3])
    return (tag,) + tuple(_tree_key(t, leaf_ids) for t in tree[1:])


def _pipe_instances(ev: T.Event) -> int:
    return int(np.prod(ev.domain_shape())) if ev.domain_shape() else 1


class _PipeSends:
    """pipe id -> origins of the blocks its source core sends, in send order:
    one (tensor, r0, c0) per send event (arrays over the event's instances),
    resolved on demand.  A sent block is filled by ttl.copy from a tensor on
    the source core, or received there from another pipe and forwarded (the
    simulator's BlockToPipeHandler takes any block, python/sim/
    copyhandlers.py:229): its origin is then that pipe's matching send,
    resolved the same way; pipes that forward to each other in a cycle never
    deliver a first block (the simulator deadlocks) and are refused."""

    def __init__(self, core_traces, pre) -> None:
        self.cores, self.pre = core_traces, pre
        self.src: Dict[int, int] = {}
        for ci, (ct, (events, _)) in enumerate(zip(core_traces, pre)):
            for tmpl, _ in ct["threads"]:
                for ev in events[id(tmpl)]:
                    if ev.kind != "pipe_send":
                        continue
                    pipe = ev.data["pipe"]
                    if self.src.setdefault(pipe.id, ci) != ci:
                        raise PlanError(f"{pipe} is sent on from two cores")
        self.memo: Dict[int, List[Tuple[Any, np.ndarray, np.ndarray]]] = {}
        self.busy: set = set()

    def receiver(self, core: int):
        """The `received` resolver of core `core`: its k-th receive on a pipe
        takes the origin of that pipe's k-th send."""
        pos: Dict[int, int] = {}

        def received(ev):
            pipe = ev.data["pipe"]
            k = pos.get(pipe.id, 0)
            pos[pipe.id] = k + 1
            lst = self.get(pipe.id)
            if k >= len(lst):
                raise RuntimeError(f"Deadlock: core {core} receives more blocks on {pipe} than its "
                                   "source core sends")
            tens, r0, c0 = lst[k]
            n = _pipe_instances(ev)
            if r0.size != n:
                raise PlanError(f"{pipe}: a receive and the matching send run a different number "
                                "of times")
            return tens, r0, c0
        return received

    def get(self, pid: int) -> List[Tuple[Any, np.ndarray, np.ndarray]]:
        if pid in self.memo:
            return self.memo[pid]
        if pid not in self.src:
            return []
        if pid in self.busy:
            raise PlanError("pipes forward blocks to each other in a cycle (the simulator "
                            "deadlocks: no block is ever delivered)")
        self.busy.add(pid)
        ci = self.src[pid]
        ct, (events, totals) = self.cores[ci], self.pre[ci]
        received = self.receiver(ct["core"])
        out = []
        for tmpl, _ in ct["threads"]:
            if tmpl.kind != "dm":
                continue
            evs = events[id(tmpl)]
            tables: Dict[int, _CopyTable] = {}
            for ev in evs:
                if ev.kind != "pipe_send" or ev.data["pipe"].id != pid:
                    continue
                blk = ev.data["block"]
                cb = blk.cb
                if cb.id not in tables:
                    n = totals[id(tmpl)].get((cb.id, "reserve"), 0)
                    try:
                        tables[cb.id] = _copy_table(evs, cb, n, "copy_in", received)
                    except PlanError as err:
                        raise PlanError("a block sent on a pipe must be filled by ttl.copy from a "
                                        "tensor on the sending core, or received there from "
                                        f"another pipe ({err})") from None
                ft = tables[cb.id]
                shape = ev.domain_shape()
                idx = T.broadcast_to_domain(blk.event.index, shape).ravel()
                out.append((ft.tensor, ft.r0[idx], ft.c0[idx]))
        self.busy.discard(pid)
        self.memo[pid] = out
        return out


_SIM_OP_LIMIT = 2_000_000  # operations replayed per core by the deadlock report


def _raise_deadlock_or(ct: Dict[str, Any], err: Exception) -> None:
    """A CB inconsistency: raise the simulator-style deadlock report when the
    threads of the core really block, else `err`."""
    rep = _deadlock_report(ct)
    if rep is not None:
        raise RuntimeError(rep)
    raise err


def _flat_ops(node):
    """The CB operations of a traced thread in program order, loops unrolled."""
    for ch in node.children:
        if isinstance(ch, T.Event):
            if ch.kind in ("reserve", "push", "wait", "pop"):
                yield ch
        else:
            for _ in range(ch.n):
                yield from _flat_ops(ch)


def _deadlock_report(ct: Dict[str, Any], failed: Sequence[int] = ()) -> Optional[str]:
    """Replays one core's three threads cooperatively against its CBs (the
    simulator's scheduler, python/sim/program.py:363-647: a reserve needs a
    free block, a wait a visible one) and, if they block, returns the
    simulator's report: "Deadlock detected: all generators blocked" with one
    line per blocked thread (operation, CB variable, source line).  None when
    the threads run to completion (or past the replay limit).  `failed` names
    the threads whose trace stopped at an error: one that reaches the end of
    its partial trace raises that error before any deadlock, so the replay
    returns None as soon as one does."""
    names, it, nxt = [], [], []
    ndm = 0
    for tmpl, root in ct["threads"]:
        if tmpl.kind == "compute":
            names.append(f"core{ct['core']}-compute")
        else:
            names.append(f"core{ct['core']}-dm{ndm}")
            ndm += 1
        g = _flat_ops(root)
        it.append(g)
        nxt.append(next(g, None))
        if nxt[-1] is None and len(it) - 1 in failed:
            return None
    visible: Dict[int, int] = {}
    reserved: Dict[int, int] = {}
    steps = 0
    while any(e is not None for e in nxt):
        progress = False
        for k in range(len(it)):
            while nxt[k] is not None:
                ev = nxt[k]
                cid, bf = ev.cb.id, ev.cb.buffer_factor
                if ev.kind == "reserve":
                    if visible.get(cid, 0) + reserved.get(cid, 0) >= bf:
                        break
                    reserved[cid] = reserved.get(cid, 0) + 1
                elif ev.kind == "push":
                    reserved[cid] = reserved.get(cid, 0) - 1
                    visible[cid] = visible.get(cid, 0) + 1
                elif ev.kind == "wait":
                    if visible.get(cid, 0) < 1:
                        break
                else:  # pop
                    visible[cid] = visible.get(cid, 0) - 1
                nxt[k] = next(it[k], None)
                if nxt[k] is None and k in failed:
                    return None
                progress = True
                steps += 1
                if steps > _SIM_OP_LIMIT:
                    return None
        if not progress:
            lines = []
            for k, ev in enumerate(nxt):
                if ev is None:
                    continue
                f, ln = ev.data.get("loc", ("?", 0))
                lines.append(f"  {names[k]}: blocked on {ev.kind}() on "
                             f"CircularBuffer({ev.cb.name}) at {f}:{ln}")
            return "Deadlock detected: all generators blocked\n" + "\n".join(lines)
    return None


def resolve(core_traces: List[Dict[str, Any]]) -> List[_Group]:
    """core_traces[c] = {"threads": [(template, root_node), ...]} for core c."""
    groups: Dict[Tuple, _Group] = {}
    hoisted: Dict[Tuple, Tuple[Any, Any]] = {}
    # pass 1: events of every core; the blocks each pipe carries are resolved
    # on demand (a forwarded block through the pipe it was received from)
    pre = []
    for ct in core_traces:
        threads = ct["threads"]
        events = {id(tmpl): _thread_events(root) for tmpl, root in threads}
        totals = {id(tmpl): T.assign_indices(root) for tmpl, root in threads}
        pre.append((events, totals))
    sends = _PipeSends(core_traces, pre)
    scratch: Dict[int, _Scratch] = {}

    for ct, (events, totals) in zip(core_traces, pre):
        threads = ct["threads"]
        # k-th receive of a pipe on this core <-> k-th send of that pipe
        received = sends.receiver(ct["core"])
        # producer / consumer of every CB on this core
        producers: Dict[int, Any] = {}
        consumers: Dict[int, Any] = {}
        cbs: Dict[int, Any] = {}
        for tmpl, root in threads:
            for ev in events[id(tmpl)]:
                if ev.kind == "reserve":
                    if producers.setdefault(ev.cb.id, tmpl) is not tmpl:
                        _raise_deadlock_or(ct, PlanError(
                            f"CB {ev.cb.name} is reserved by two threads"))
                    cbs[ev.cb.id] = ev.cb
                elif ev.kind == "wait":
                    if consumers.setdefault(ev.cb.id, tmpl) is not tmpl:
                        _raise_deadlock_or(ct, PlanError(
                            f"CB {ev.cb.name} is waited on by two threads"))
                    cbs[ev.cb.id] = ev.cb
        count = {}
        for cid, cb in cbs.items():
            np_ = totals[id(producers[cid])].get((cid, "reserve"), 0) if cid in producers else 0
            nc_ = totals[id(consumers[cid])].get((cid, "wait"), 0) if cid in consumers else 0
            if np_ != nc_:
                _raise_deadlock_or(ct, RuntimeError(
                    f"Deadlock: CB {cb.name} has {np_} blocks pushed but {nc_} blocks waited on "
                    f"core {ct['core']} (producer and consumer disagree)"))
            count[cid] = np_
        # copy tables
        fill: Dict[int, _CopyTable] = {}
        drain: Dict[int, _CopyTable] = {}
        for cid, cb in cbs.items():
            if cid in producers and producers[cid].kind == "dm":
                fill[cid] = _copy_table(events[id(producers[cid])], cb, count[cid], "copy_in",
                                        received)
            if cid in consumers and consumers[cid].kind == "dm":
                drain[cid] = _copy_table(events[id(consumers[cid])], cb, count[cid], "copy_out")
        inter = [cid for cid in cbs if producers.get(cid) is not None
                 and consumers.get(cid) is not None and producers[cid].kind == "compute"
                 and consumers[cid].kind == "compute"]
        if inter:
            _intermediate_tables(threads, events, cbs, count, inter, fill, drain, scratch)
        # stores
        acc_count: Dict[Tuple[int, int], int] = {}  # (CB, block) -> acc stores so far
        for tmpl, root in threads:
            for ev in events[id(tmpl)]:
                if ev.kind != "store":
                    continue
                target = ev.data["target"]
                e = ev.data["expr"]
                cid = target.cb.id
                if cid not in drain:
                    raise PlanError(f"blocks stored into CB {target.cb.name} must be copied to a "
                                    "tensor by a data-movement thread or read back by the compute "
                                    "thread")
                shape = ev.domain_shape()
                rout = T.broadcast_to_domain(target.event.index, shape).ravel()
                dt = drain[cid]
                R, C = target.shape
                site = (ev.data.get("loc"), _tree_key(e.tree, {}), id(dt.tensor))
                rounds = None
                if ev.data["acc"]:
                    rounds = _acc_rounds(cid, rout, acc_count)
                    if rounds.max(initial=0) > 0 and _has_sub(e.tree):
                        raise PlanError("store(acc=True) into a block stored before, of an "
                                        "expression with a reduction inside, is not supported")
                e = _hoist_subexprs(ev, e, target, rout, dt, fill, shape, groups, hoisted, site)
                e = _hoist_operands(ev, e, fill, shape, groups, hoisted, site)
                if e.tree[0] == "reduce":
                    _resolve_reduce(ev, e, target, rout, dt, fill, shape, groups)
                    continue
                if e.tree[0] == "bmatmul":
                    _resolve_block_matmul(ev, e, target, rout, dt, fill, shape, groups)
                    continue
                inner_mm = e.tree[0] != "matmul" and (_has(e.tree, "matmul")
                                                      or _has(e.tree, "bmatmul"))
                if rounds is not None and e.tree[0] != "matmul" and (
                        inner_mm or rounds.max(initial=0) > 0):
                    _resolve_acc_rounds(ev, e, target, rout, dt, fill, shape, groups, hoisted,
                                        site, rounds)
                    continue
                if inner_mm:
                    e = _hoist_matmuls(ev, e, target, rout, dt, fill, shape, groups, hoisted)
                _store_group(ev, e, target, rout, dt, fill, shape, groups)
    for sc in scratch.values():
        sc.check()
    return list(groups.values())


def _dom(index, shape, sel=None) -> np.ndarray:
    """An event's per-instance index over the store's domain (raveled), the
    instances `sel` selects only."""
    w = T.broadcast_to_domain(index, shape).ravel()
    return w if sel is None else w[sel]


def _store_group(ev, e, target, rout, dt, fill, shape, groups, sel=None, key_extra=()) -> None:
    """The store's instances (those `sel` selects) join the group of their
    expression, tensors and acc flag (extended by key_extra)."""
    R, C = target.shape
    er, ec = e.shape
    nslot = R * C
    rsel = rout if sel is None else rout[sel]
    inst = np.arange(rout.size) if sel is None else np.nonzero(sel)[0]
    # output tile of every (instance, slot)
    slot = np.arange(nslot)
    oi, oj = slot // C, slot % C
    out_r = (dt.r0[rsel][:, None] + oi[None, :]).ravel()
    out_c = (dt.c0[rsel][:, None] + oj[None, :]).ravel()
    leaves = _tree_leaves(e.tree, [])
    leaf_rc = []
    leaf_tensors = []
    ei, ej = slot // ec, slot % ec  # expression slot of each target slot
    for lf in leaves:
        blk, rmap, cmap = lf[1], lf[2], lf[3]
        lcid = blk.cb.id
        if lcid not in fill:
            raise PlanError("expression operands must come from blocks filled by "
                            "ttl.copy from a tensor")
        ft = fill[lcid]
        w = _dom(blk.event.index, shape, sel)
        lr = (ft.r0[w][:, None] + np.asarray(rmap)[ei][None, :]).ravel()
        lc = (ft.c0[w][:, None] + np.asarray(cmap)[ej][None, :]).ravel()
        leaf_rc.append(np.stack([lr, lc], 1))
        leaf_tensors.append(ft.tensor)
    acc = ev.data["acc"] and not key_extra
    order = np.repeat(inst, nslot)
    key = (_tree_key(e.tree, {}), tuple(id(t) for t in leaf_tensors), id(dt.tensor),
           acc) + tuple(key_extra)
    g = groups.get(key)
    if g is None:
        g = _Group(e.tree, leaves, leaf_tensors, dt.tensor, acc, e.dtype, ev.data.get("loc"))
        groups[key] = g
    g.out_rc.append(np.stack([out_r, out_c], 1))
    g.leaf_rc.append(leaf_rc)
    g.order.append(order)


def _acc_rounds(cid: int, rout: np.ndarray, acc_count: Dict[Tuple[int, int], int]) -> np.ndarray:
    """Round of every instance of a store(acc=True) event: how many acc stores
    into the same block came before it (earlier events, then earlier
    instances of this one in loop order).  Counts the event's stores in."""
    rounds = np.zeros(rout.size, dtype=np.int64)
    if rout.size == 0:
        return rounds
    srt = np.argsort(rout, kind="stable")
    rs = rout[srt]
    start = np.r_[0, np.nonzero(np.diff(rs))[0] + 1]
    rank = np.arange(rs.size) - np.repeat(start, np.diff(np.r_[start, rs.size]))
    base = np.array([acc_count.get((cid, int(b)), 0) for b in rs], dtype=np.int64)
    rounds[srt] = rank + base
    for b, n in zip(*np.unique(rs, return_counts=True)):
        acc_count[(cid, int(b))] = acc_count.get((cid, int(b)), 0) + int(n)
    return rounds


def _resolve_acc_rounds(ev, e, target, rout, dt, fill, shape, groups, hoisted, site,
                        rounds) -> None:
    """store(expr, acc=True) whose expression is not a lone tile matmul: the
    simulator assigns on a block's first acc store and adds on the later ones,
    block = block + value, rounded to the block's dtype (python/sim/block.py:
    850-864).  The instances are split into rounds by how many acc stores into
    their block came before; round 0 stores the expression, round r > 0 stores
    out + expression, out read from the output tensor at the block's own
    tiles, each round one store group planned after the one before (a tile
    matmul inside the expression gets a plan-owned product tensor per round,
    planned just before its round)."""
    R, C = target.shape
    for r in np.unique(rounds):
        sel = rounds == r
        rsite = site + (("acc", int(r)),)
        er = e
        if _has(e.tree, "matmul") or _has(e.tree, "bmatmul"):
            er = _hoist_matmuls(ev, e, target, rout, dt, fill, shape, groups, hoisted, sel=sel,
                                site=rsite)
        if r > 0:
            key = rsite + ("out",)
            if key not in hoisted:
                cb = _HoistedCB(-1 - len(hoisted), target.cb.dtype, "(accumulated block)")
                hoisted[key] = (None, cb)
            cb = hoisted[key][1]
            fill[cb.id] = _CopyTable(dt.tensor, dt.r0, dt.c0)
            out_leaf = ("leaf", _HoistedBlock(cb, target.event), list(range(R)), list(range(C)))
            tree = ("add", out_leaf, er.tree)
            dtype = (torch.promote_types(target.cb.dtype, er.dtype)
                     if isinstance(er.dtype, torch.dtype)
                     and isinstance(target.cb.dtype, torch.dtype) else er.dtype)
            er = _Expr(tree, (R, C), dtype)
        _store_group(ev, er, target, rout, dt, fill, shape, groups, sel=sel,
                     key_extra=(("acc round", int(r)),))


def _has_sub(tree) -> bool:
    return any(_is_sub(lf) for lf in _tree_leaves(tree, []))


class _HoistedCB:
    """The stand-in CB of a product split off a store expression."""

    def __init__(self, cid: int, dtype, name: str) -> None:
        self.id, self.dtype, self.name = cid, dtype, name


class _HoistedBlock:
    def __init__(self, cb: _HoistedCB, event) -> None:
        self.cb, self.event = cb, event


class _Expr:
    def __init__(self, tree, shape, dtype) -> None:
        self.tree, self.shape, self.dtype = tree, tuple(shape), dtype


def _hoist_matmuls(ev, e, target, rout, dt, fill, shape, groups, hoisted, sel=None, site=None):
    """A store whose expression holds a tile or block matmul below its root,
    e.g. relu(a @ b + c): the simulator materialises the product block (in
    the dtype its operands promote to) before the other ops read it
    (python/sim/block.py:870-920), so the plan does the same: each product
    becomes a matmul launch into a plan-owned tensor laid out like the
    output, and the expression reads that tensor at the output's tile
    positions as an ordinary operand.  Only products of blocks filled from
    tensors, of the target's block shape.  For the instances `sel` selects
    (one accumulation round of an acc store: `site` names the round, so each
    round's product gets its own tensor)."""
    R, C = target.shape
    if tuple(e.shape) != (R, C):
        raise PlanError(f"an expression of block shape {tuple(e.shape)} holding a tile matmul, "
                        f"stored into a block of shape {(R, C)}")
    slot = np.arange(R * C)
    oi, oj = slot // C, slot % C
    rsel = rout if sel is None else rout[sel]
    inst = np.arange(rout.size) if sel is None else np.nonzero(sel)[0]
    out_r = (dt.r0[rsel][:, None] + oi[None, :]).ravel()
    out_c = (dt.c0[rsel][:, None] + oj[None, :]).ravel()
    order = np.repeat(inst, R * C)
    if site is None:
        site = (ev.data.get("loc"), _tree_key(e.tree, {}), id(dt.tensor))
    count = [0]

    def walk(tree):
        tag = tree[0]
        if tag in ("matmul", "bmatmul"):
            node = count[0]  # the product's place in the expression: its temp's identity
            count[0] += 1
            la, lb = tree[1], tree[2]
            if la[0] != "leaf" or lb[0] != "leaf":
                raise PlanError("a tile matmul's operands must be blocks filled by ttl.copy from "
                                "a tensor")
            # leaf maps: a block matmul's over its operand blocks (M, K) / (K, N), a tile-wise
            # product's over the expression's slots
            shp = (len(la[2]), len(lb[3]))
            if shp != (R, C):
                raise PlanError(f"a tile matmul of block shape {shp} inside a store into a "
                                f"block of shape {(R, C)}")
            fa, fb = fill.get(la[1].cb.id), fill.get(lb[1].cb.id)
            if fa is None or fb is None:
                raise PlanError("a tile matmul's operands must be blocks filled by ttl.copy from "
                                "a tensor")
            da, db = la[1].cb.dtype, lb[1].cb.dtype
            pdt = (torch.promote_types(da, db) if isinstance(da, torch.dtype)
                   and isinstance(db, torch.dtype) else da)
            key = site + (node,)
            if key not in hoisted:
                cb = _HoistedCB(-1 - len(hoisted), pdt, "(matmul product)")
                hoisted[key] = (_Temp(tuple(dt.tensor.shape), pdt), cb)
            temp, cb = hoisted[key]
            tab = _CopyTable(temp, dt.r0, dt.c0)
            if tag == "bmatmul":
                _resolve_block_matmul(ev, _Expr(tree, (R, C), pdt), target, rout, tab, fill, shape,
                                      groups, sel)
            else:
                leaf_rc = []
                for lf in (la, lb):
                    ft = fill[lf[1].cb.id]
                    w = _dom(lf[1].event.index, shape, sel)
                    lr = (ft.r0[w][:, None] + np.asarray(lf[2])[oi][None, :]).ravel()
                    lc = (ft.c0[w][:, None] + np.asarray(lf[3])[oj][None, :]).ravel()
                    leaf_rc.append(np.stack([lr, lc], 1))
                gkey = (_tree_key(tree, {}), (id(fa.tensor), id(fb.tensor)), id(temp), False)
                g = groups.get(gkey)
                if g is None:
                    g = groups[gkey] = _Group(tree, [la, lb], [fa.tensor, fb.tensor], temp, False,
                                              pdt, ev.data.get("loc"))
                g.out_rc.append(np.stack([out_r, out_c], 1))
                g.leaf_rc.append(leaf_rc)
                g.order.append(order)
            fill[cb.id] = tab
            return ("leaf", _HoistedBlock(cb, target.event), list(range(R)), list(range(C)))
        if tag in ("leaf", "const"):
            return tree
        if tag in ("powi", "upar"):
            return (tag, walk(tree[1])) + tuple(tree[2:])
        if tag == "reduce":
            raise PlanError("a reduction combined with a tile matmul in one store() is not "
                            "supported")
        return (tag,) + tuple(walk(t) for t in tree[1:])

    return _Expr(walk(e.tree), e.shape, e.dtype)


def _is_sub(leaf) -> bool:
    return leaf[0] == "leaf" and isinstance(leaf[1], D.SubExpr)


def _tree_dtype(tree):
    """dtype of an elementwise tree: its leaves' dtypes promoted (numbers do
    not promote a block, as in torch)."""
    dt = None
    for lf in _tree_leaves(tree, []):
        d = lf[1].cb.dtype
        dt = d if dt is None else torch.promote_types(dt, d)
    return dt


class _SubTarget:
    """The block a hoisted sub-expression is stored into: the store's target
    block's instances, the sub-expression's block shape."""

    def __init__(self, shape, event) -> None:
        self.shape, self.event = tuple(shape), event


def _hoist_subexprs(ev, e, target, rout, dt, fill, shape, groups, hoisted, site, done=None):
    """Leaves whose block is a sub-expression (a reduction used as an operand,
    dsl.SubExpr): the reduction is planned first into a plan-owned tensor laid
    out like the output, its result tile (i, j) at the target block's tile
    (i, j) (a reduced block is never larger than the expression it feeds),
    and the leaf reads that tensor with the leaf's own maps and in-tile
    broadcast.  Nested sub-expressions are hoisted first; one sub-expression
    used at several places (x - m and a reduction of exp(x - m)) is computed
    once."""
    count = [0]
    done = {} if done is None else done  # id(SubExpr) -> its hoisted block

    def walk(tree):
        tag = tree[0]
        if tag == "leaf":
            if not _is_sub(tree):
                return tree
            if id(tree[1]) in done:
                return ("leaf", done[id(tree[1])]) + tuple(tree[2:])
            sub = tree[1].expr
            node = count[0]
            count[0] += 1
            inner = _hoist_subexprs(ev, sub, target, rout, dt, fill, shape, groups, hoisted,
                                    site + (("sub", node),), done)
            if inner.tree[0] != "reduce":
                raise PlanError("only reductions are computed ahead of the expression using them")
            Rr, Cr = inner.shape
            R, C = target.shape
            if Rr > R or Cr > C:
                raise PlanError(f"a reduction of block shape {(Rr, Cr)} inside a store into a "
                                f"block of shape {(R, C)}")
            key = site + ("sub", node)
            if key not in hoisted:
                cb = _HoistedCB(-1 - len(hoisted), inner.dtype, "(reduction)")
                hoisted[key] = (_Temp(tuple(dt.tensor.shape), inner.dtype), cb)
            temp, cb = hoisted[key]
            tab = _CopyTable(temp, dt.r0, dt.c0)
            _resolve_reduce(ev, inner, _SubTarget((Rr, Cr), target.event), rout, tab, fill, shape,
                            groups)
            fill[cb.id] = tab
            done[id(tree[1])] = _HoistedBlock(cb, target.event)
            return ("leaf", done[id(tree[1])]) + tuple(tree[2:])
        if tag == "const":
            return tree
        if tag in ("powi", "upar"):
            return (tag, walk(tree[1])) + tuple(tree[2:])
        if tag == "reduce":
            _, kind, dims, inner, ishape, scaler = tree
            return ("reduce", kind, dims, walk(inner), ishape, walk(scaler))
        if tag == "bmatmul":
            return ("bmatmul", walk(tree[1]), walk(tree[2]), tree[3])
        return (tag,) + tuple(walk(t) for t in tree[1:])

    return _Expr(walk(e.tree), e.shape, e.dtype)


def _hoist_operands(ev, e, fill, shape, groups, hoisted, site):
    """Tile or block matmuls whose operand is a computed block expression,
    e.g. (a * s) @ b (the spec types __matmul__(self, other: BlockExpr),
    TTLangSpecification.md:693; the simulator pairs any blocks,
    python/sim/block.py:1012-1013, after materialising the operand in its
    dtype): the operand is planned first as an elementwise store into a
    plan-owned tensor laid out like one of its leaves (the anchor: a leaf
    whose maps take every slot of the operand to a distinct tile), each
    operand tile at its anchor tile, and the matmul reads that tensor where it
    would have read the anchor.  Two instances that need different values in
    one anchor tile make that store write a tile twice, which is refused."""
    count = [0]

    def hoist(t):
        node = count[0]
        count[0] += 1
        if t[0] == "leaf" and not any(_leaf_rep(t)):
            return t
        leaves = _tree_leaves(t, [])
        anchor = None
        for lf in leaves:
            rm, cm = np.asarray(lf[2]), np.asarray(lf[3])
            if (lf[1].cb.id in fill and len(set(rm.tolist())) == rm.size
                    and len(set(cm.tolist())) == cm.size):
                anchor = lf
                break
        if anchor is None:
            raise PlanError("a tile matmul operand computed from blocks none of which covers the "
                            "operand tile for tile (all broadcast or not filled from a tensor)")
        for lf in leaves:
            if lf[1].cb.id not in fill:
                raise PlanError("expression operands must come from blocks filled by ttl.copy from "
                                "a tensor")
        Ro, Co = len(anchor[2]), len(anchor[3])
        slot = np.arange(Ro * Co)
        oi, oj = slot // Co, slot % Co
        fa = fill[anchor[1].cb.id]
        wa = T.broadcast_to_domain(anchor[1].event.index, shape).ravel()
        out_r = (fa.r0[wa][:, None] + np.asarray(anchor[2])[oi][None, :]).ravel()
        out_c = (fa.c0[wa][:, None] + np.asarray(anchor[3])[oj][None, :]).ravel()
        leaf_rc, leaf_tensors = [], []
        for lf in leaves:
            ft = fill[lf[1].cb.id]
            w = T.broadcast_to_domain(lf[1].event.index, shape).ravel()
            lr = (ft.r0[w][:, None] + np.asarray(lf[2])[oi][None, :]).ravel()
            lc = (ft.c0[w][:, None] + np.asarray(lf[3])[oj][None, :]).ravel()
            leaf_rc.append(np.stack([lr, lc], 1))
            leaf_tensors.append(ft.tensor)
        dtype = _tree_dtype(t)
        key = site + ("operand", node)
        if key not in hoisted:
            cb = _HoistedCB(-1 - len(hoisted), dtype, "(matmul operand)")
            hoisted[key] = (_Temp(tuple(fa.tensor.shape), dtype), cb)
        temp, cb = hoisted[key]
        gkey = (_tree_key(t, {}), tuple(id(x) for x in leaf_tensors), id(temp), False)
        g = groups.get(gkey)
        if g is None:
            g = groups[gkey] = _Group(t, leaves, leaf_tensors, temp, False, dtype,
                                      ev.data.get("loc"), private_out=True)
        g.out_rc.append(np.stack([out_r, out_c], 1))
        g.leaf_rc.append(leaf_rc)
        g.order.append(np.repeat(np.arange(wa.size), Ro * Co))
        fill[cb.id] = _CopyTable(temp, fa.r0, fa.c0)
        return ("leaf", _HoistedBlock(cb, anchor[1].event), anchor[2], anchor[3])

    def walk(tree):
        tag = tree[0]
        if tag in ("leaf", "const"):
            return tree
        if tag == "matmul":
            return ("matmul", hoist(walk(tree[1])), hoist(walk(tree[2])))
        if tag == "bmatmul":
            return ("bmatmul", hoist(walk(tree[1])), hoist(walk(tree[2])), tree[3])
        if tag in ("powi", "upar"):
            return (tag, walk(tree[1])) + tuple(tree[2:])
        if tag == "reduce":
            _, kind, dims, inner, ishape, scaler = tree
            return ("reduce", kind, dims, walk(inner), ishape, scaler)
        return (tag,) + tuple(walk(t) for t in tree[1:])

    return _Expr(walk(e.tree), e.shape, e.dtype)


def _resolve_block_matmul(ev, e, target, rout, dt, fill, shape, groups, sel=None) -> None:
    """Store of a block matmul (the spec's (M, K) @ (K, N) blocks): output
    tile (i, j) accumulates a(i, k) @ b(k, j) over k, which is the tile
    matmul accumulation of K store(acc=True) instances; it joins that group
    (`("matmul", a, b)` with acc), one instance per (store, k)."""
    _, la, lb, K = e.tree
    R, C = target.shape
    if tuple(e.shape) != (R, C):
        raise PlanError(f"a block matmul of shape {tuple(e.shape)} stored into a block of shape "
                        f"{(R, C)}")
    slot = np.arange(R * C)
    oi, oj = slot // C, slot % C
    rsel = rout if sel is None else rout[sel]
    inst = np.arange(rout.size) if sel is None else np.nonzero(sel)[0]
    out_r = (dt.r0[rsel][:, None] + oi[None, :]).ravel()
    out_c = (dt.c0[rsel][:, None] + oj[None, :]).ravel()
    ops = []
    for lf in (la, lb):
        blk = lf[1]
        if blk.cb.id not in fill:
            raise PlanError("expression operands must come from blocks filled by ttl.copy from a "
                            "tensor")
        ft = fill[blk.cb.id]
        w = _dom(blk.event.index, shape, sel)
        ops.append((ft, w, np.asarray(lf[2]), np.asarray(lf[3])))
    (fa, wa, ra, ca), (fb, wb, rb, cb) = ops
    outs, a_rc, b_rc = [], [], []
    for k in range(K):
        a_r = (fa.r0[wa][:, None] + ra[oi][None, :]).ravel()
        a_c = (fa.c0[wa][:, None] + np.full(slot.size, ca[k])[None, :]).ravel()
        b_r = (fb.r0[wb][:, None] + np.full(slot.size, rb[k])[None, :]).ravel()
        b_c = (fb.c0[wb][:, None] + cb[oj][None, :]).ravel()
        outs.append(np.stack([out_r, out_c], 1))
        a_rc.append(np.stack([a_r, a_c], 1))
        b_rc.append(np.stack([b_r, b_c], 1))
    tree = ("matmul", la, lb)
    key = (_tree_key(tree, {}), (id(fa.tensor), id(fb.tensor)), id(dt.tensor), True)
    g = groups.get(key)
    if g is None:
        g = _Group(tree, [la, lb], [fa.tensor, fb.tensor], dt.tensor, True, e.dtype,
                   ev.data.get("loc"))
        groups[key] = g
    base = sum(o.size for o in g.order)
    g.out_rc.append(np.concatenate(outs, 0))
    g.leaf_rc.append([np.concatenate(a_rc, 0), np.concatenate(b_rc, 0)])
    g.order.append(base + np.tile(np.repeat(inst, R * C), K))


def _resolve_reduce(ev, e, target, rout, dt, fill, shape, groups) -> None:
    """Store of a reduction: every (instance, slot of the reduced expression)
    contributes its expression tile to the output tile of the target slot it
    collapses onto."""
    _, kind, dims, inner, ishape, stree = e.tree
    R, C = target.shape
    if tuple(e.shape) != (R, C):
        raise PlanError(f"a reduction of shape {tuple(e.shape)} stored into a block of shape "
                        f"{(R, C)}: the target block must have the reduced shape")
    IR, IC = ishape
    islot = np.arange(IR * IC)
    ii, ij = islot // IC, islot % IC
    ti = np.zeros_like(ii) if 0 in dims else ii
    tj = np.zeros_like(ij) if 1 in dims else ij
    out_r = (dt.r0[rout][:, None] + ti[None, :]).ravel()
    out_c = (dt.c0[rout][:, None] + tj[None, :]).ravel()
    leaves = _tree_leaves(inner, [])
    if not leaves:
        raise PlanError("a reduction needs at least one operand read from a tensor")
    leaf_rc, leaf_tensors = [], []
    for lf in leaves:
        blk, rmap, cmap = lf[1], lf[2], lf[3]
        if blk.cb.id not in fill:
            raise PlanError("expression operands must come from blocks filled by ttl.copy from a "
                            "tensor")
        ft = fill[blk.cb.id]
        w = T.broadcast_to_domain(blk.event.index, shape).ravel()
        lr = (ft.r0[w][:, None] + np.asarray(rmap)[ii][None, :]).ravel()
        lc = (ft.c0[w][:, None] + np.asarray(cmap)[ij][None, :]).ravel()
        leaf_rc.append(np.stack([lr, lc], 1))
        leaf_tensors.append(ft.tensor)
    s_tensor, s_rc = None, None
    if stree[0] == "leaf":
        sblk, srm, scm = stree[1], stree[2], stree[3]
        if sblk.cb.id not in fill:
            raise PlanError("a reduction's scaler block must be filled by ttl.copy from a tensor")
        ft = fill[sblk.cb.id]
        w = T.broadcast_to_domain(sblk.event.index, shape).ravel()
        s_tensor = ft.tensor
        s_rc = np.stack([ft.r0[w] + int(srm[0]), ft.c0[w] + int(scm[0])], 1)
    order = np.repeat(np.arange(rout.size), IR * IC)
    key = (_tree_key(e.tree, {}), tuple(id(t) for t in leaf_tensors), id(s_tensor),
           id(dt.tensor), ev.data["acc"])
    g = groups.get(key)
    if g is None:
        g = _Group(e.tree, leaves, leaf_tensors, dt.tensor, ev.data["acc"], e.dtype,
                   ev.data.get("loc"), scaler_tensor=s_tensor)
        groups[key] = g
    g.out_rc.append(np.stack([out_r, out_c], 1))
    g.leaf_rc.append(leaf_rc)
    g.order.append(order + sum(o.size for o in g.order))
    if s_rc is not None:
        g.scaler_rc.append(s_rc)


# ---------------------------------------------------------------------------
# classification


def _rect(rc: np.ndarray) -> Tuple[int, int, int, int]:
    r0, c0 = rc.min(0)
    r1, c1 = rc.max(0) + 1
    return int(r0), int(r1), int(c0), int(c1)


def _unique_tiles(rc: np.ndarray) -> int:
    key = rc[:, 0] * (int(rc[:, 1].max()) + 1) + rc[:, 1]
    return int(np.unique(key).size)


def _axis_map(out_t: np.ndarray, in_t: np.ndarray, dim: int,
              rep: bool = False) -> Tuple[int, int]:
    """(mask, element offset) reproducing in_tile = f(out_tile) on one axis;
    rep: element 0 of the axis in every tile (in-tile broadcast)."""
    if dim == 1:  # degenerate tensor dimension: stride 0, only tile 0 exists
        return 31, 0
    d = in_t - out_t
    if np.all(d == d[0]):
        return (~31 if rep else -1), int(d[0]) * TILE
    if np.all(in_t == in_t[0]):
        return (0 if rep else 31), int(in_t[0]) * TILE
    raise _NotAffine("an operand's tiles are not an affine image of the output tiles "
                     "(only identity, offset, fixed-tile reuse and size-1 broadcast map onto the "
                     "grid-wide kernel)")


class _NotAffine(PlanError):
    """An operand's tile map is not one the kernels address; `leaf` and
    `axis` name it."""

    leaf: int = -1
    axis: int = -1


# most launches one store site may be split into (see _plan_eltwise_parts)
_MAX_PARTS = 4096


_BIN = {"add", "sub", "mul", "div", "max", "min", "pow", "floordiv", "mod"}
_UN = {"exp", "log", "sqrt", "rsqrt", "tanh", "abs", "neg", "relu", "sigmoid", "recip",
       "exp2", "expm1", "logp1", "sin", "cos", "tan", "asin", "acos", "atan", "asinh", "acosh",
       "atanh", "gelu", "silu", "softsign", "hardsigmoid"}


def _to_expr(tree, leaf_nodes: Dict[int, X.Leaf]) -> X.Expr:
    tag = tree[0]
    if tag == "leaf":
        return leaf_nodes[id(tree)]
    if tag == "const":
        return X.Const(tree[1])
    if tag == "powi":
        x = _to_expr(tree[1], leaf_nodes)
        return X.Unary("powi", x, x.dtype, imm=float(tree[2]))
    if tag == "upar":
        x = _to_expr(tree[1], leaf_nodes)
        return X.Unary(tree[2], x, x.dtype, imm=float(tree[3]), imm2=float(tree[4]))
    if tag in _UN:
        x = _to_expr(tree[1], leaf_nodes)
        return X.Unary(tag, x, x.dtype)
    if tag in _BIN:
        a, b = _to_expr(tree[1], leaf_nodes), _to_expr(tree[2], leaf_nodes)
        if isinstance(a, X.Const):
            dt = b.dtype
        elif isinstance(b, X.Const):
            dt = a.dtype
        else:
            dt = X.promote(a.dtype, b.dtype)
        return X.Binary(tag, a, b, dt)
    if tag == "matmul":
        raise PlanError("a tile matmul combined with other ops in one store() is not supported; "
                        "store the product on its own (acc=True accumulates over K)")
    raise PlanError(f"unsupported tile op {tag!r}")


def _has(tree, tag) -> bool:
    if tree[0] == tag:
        return True
    if tree[0] in ("leaf", "const"):
        return False
    if tree[0] == "reduce":
        return _has(tree[3], tag)
    if tree[0] in ("powi", "upar"):
        return _has(tree[1], tag)
    return any(_has(t, tag) for t in tree[1:] if isinstance(t, tuple))


def _compose_axis(mb: int, ob: int, ma: int, oa: int) -> Tuple[int, int]:
    """(mask, offset) of c -> (((c & mb) + ob) & ma) + oa, for masks in
    {-1, 31, 0, ~31} and offsets that are multiples of 32."""
    if mb == -1:
        return ma, oa + (ob if ma in (-1, ~31) else 0)
    if mb == ~31:
        return (~31, ob + oa) if ma in (-1, ~31) else (0, oa)
    if mb == 31:
        if ma == -1:
            return 31, ob + oa
        if ma == ~31:
            return 0, ob + oa
        return ma, oa
    return 0, oa + (ob if ma in (-1, ~31) else 0)


class _Inliner:
    """Elementwise stages into intermediate CBs, inlined into their readers:
    a scratch tensor written by one plain elementwise launch (no acc, its
    value's dtype = the CB's, so the store rounds nothing) is replaced in
    every reading program by the writer's expression, operand maps composed
    (_compose_axis); when every reader took it, the writer's launch is
    dropped and the intermediate never touches HBM.

    Inlining moves the stage's operand reads to its reader's launch, so a
    stage stops being inlinable once a later store writes a tensor it reads
    (the reader would see the new values), and a reader that itself writes
    such a tensor does not take it (its lanes would read elements other
    lanes of the same launch overwrite)."""

    def __init__(self, groups: List[_Group]) -> None:
        self.writers: Dict[int, int] = {}
        for g in groups:
            if isinstance(g.out_tensor, _Scratch):
                self.writers[id(g.out_tensor)] = self.writers.get(id(g.out_tensor), 0) + 1
        self.exprs: Dict[int, Tuple[X.Expr, Dict[int, OperandSpec], Any]] = {}
        # scratch id -> ids of the tensors its inlined expression reads
        self.sources: Dict[int, set] = {}
        self.reads: Dict[int, List[bool]] = {}

    def register(self, g: _Group, launch, subbed=()) -> None:
        out = g.out_tensor
        e = getattr(launch, "_expr", None)
        if (isinstance(out, _Scratch) and not g.acc and self.writers.get(id(out)) == 1
                and e is not None and e.dtype == out.dtype):
            src = {id(t) for t in g.leaf_tensors}
            for t in subbed:  # stages this one inlined: their operands too
                src |= self.sources.get(t, set())
            self.exprs[id(out)] = (e, launch._specs, launch)
            self.sources[id(out)] = src

    def note_write(self, tens) -> None:
        """A store into `tens` ran: stages reading it can no longer be inlined
        into later readers (their launches stay, in trace order)."""
        for sid in [s for s, src in self.sources.items() if id(tens) in src and s in self.exprs]:
            del self.exprs[sid]

    def substitute(self, tens, rspec: OperandSpec, specs: Dict[int, OperandSpec], out=None):
        """The writer's expression for a read of `tens` through rspec (new
        leaves added to specs), or None.  `out` is the reader's output."""
        if id(tens) not in self.exprs:
            return None
        if out is not None and id(out) in self.sources[id(tens)]:
            return None
        e, wspecs, _ = self.exprs[id(tens)]
        memo: Dict[int, X.Expr] = {}

        def remap(n):
            if isinstance(n, X.Leaf):
                if id(n) not in memo:
                    ws = wspecs[n.ref]
                    rm, ro = _compose_axis(rspec.row_mask, rspec.row_off, ws.row_mask, ws.row_off)
                    cm, co = _compose_axis(rspec.col_mask, rspec.col_off, ws.col_mask, ws.col_off)
                    k = max(specs) + 1 if specs else 0
                    specs[k] = OperandSpec(ws.ref, rm, cm, ro, co)
                    memo[id(n)] = X.Leaf(k, n.dtype)
                return memo[id(n)]
            if isinstance(n, X.Unary):
                return dataclasses.replace(n, x=remap(n.x))
            if isinstance(n, X.Binary):
                return dataclasses.replace(n, a=remap(n.a), b=remap(n.b))
            return n
        return remap(e)

    def note_read(self, tens, inlined: bool) -> None:
        if isinstance(tens, _Scratch):
            self.reads.setdefault(id(tens), []).append(inlined)

    def note_reads(self, tensors, subbed=()) -> None:
        """Reads of a launch's operand tensors; `subbed` = ids of those it
        inlined."""
        for t in tensors:
            self.note_read(t, id(t) in subbed)

    def finish(self, plan: "Plan") -> None:
        drop = {id(l) for sid, (_, _, l) in self.exprs.items()
                if self.reads.get(sid) and all(self.reads[sid])}
        plan.launches = [l for l in plan.launches if id(l) not in drop]


def _leaf_operands(g: _Group, it_rc, leaf_rc, tensor_ref, inl: Optional[_Inliner]):
    """Operand specs and expression nodes of a group's leaves over iteration
    tiles it_rc, with intermediate stages inlined where inl allows.  Returns
    (specs, leaf_nodes, plain_nodes, subbed): plain_nodes maps every leaf to
    its own operand (the fallback when the inlined program does not fit),
    subbed holds the ids of the tensors whose stage was inlined."""
    specs: Dict[int, OperandSpec] = {}
    plain: Dict[int, X.Expr] = {}
    for k, lf in enumerate(g.leaf_blocks):
        tens = g.leaf_tensors[k]
        h, w = tens.shape
        rr, cr = _leaf_rep(lf)
        try:
            axis = 0
            rm, ro = _axis_map(it_rc[:, 0], leaf_rc[k][:, 0], h, rr)
            axis = 1
            cm, co = _axis_map(it_rc[:, 1], leaf_rc[k][:, 1], w, cr)
        except _NotAffine as err:
            err.leaf, err.axis = k, axis
            raise
        specs[k] = OperandSpec(tensor_ref(tens), rm, cm, ro, co)
        plain[id(lf)] = X.Leaf(k, lf[1].cb.dtype)
    nodes = dict(plain)
    subbed = set()
    if inl is not None:
        for k, lf in enumerate(g.leaf_blocks):
            sub = inl.substitute(g.leaf_tensors[k], specs[k], specs, out=g.out_tensor)
            if sub is not None:
                nodes[id(lf)] = sub
                subbed.add(id(g.leaf_tensors[k]))
    return specs, nodes, plain, subbed


# ---------------------------------------------------------------------------
# attention


def _plain_leaf(t, rep=(False, False)) -> bool:
    return t[0] == "leaf" and _leaf_rep(t) == rep


def _is_const(t) -> bool:
    return t[0] == "const" and isinstance(t[1], (int, float))


def _scaled(t) -> Optional[Tuple[Any, float]]:
    """(x, c) for x * c or c * x with x a plain leaf; (x, 1.0) for x."""
    if _plain_leaf(t):
        return t, 1.0
    if t[0] == "mul":
        a, b = t[1], t[2]
        if _plain_leaf(a) and _is_const(b):
            return a, float(b[1])
        if _plain_leaf(b) and _is_const(a):
            return b, float(a[1])
    return None


def _softmax_numerator(t, m_scale: float):
    """(S leaf, M leaf, scale) of exp(S*c - bcast(M)) with M = reduce_max(S, c)
    (`m_scale` = c), or of exp((S - bcast(M)) * c) with M = reduce_max(S, 1);
    both are exp(c*S - max_j c*S) for c > 0.  None for anything else."""
    if t[0] != "exp":
        return None
    x, col = t[1], (False, True)
    if x[0] == "sub" and _plain_leaf(x[2], col):
        sx = _scaled(x[1])
        if sx is not None and sx[1] == m_scale:
            return sx[0], x[2], sx[1]
    if x[0] == "mul" and m_scale == 1.0:
        diff, c = (x[1], x[2]) if _is_const(x[2]) else (x[2], x[1])
        if (_is_const(c) and diff[0] == "sub" and _plain_leaf(diff[1])
                and _plain_leaf(diff[2], col)):
            return diff[1], diff[2], float(c[1])
    return None


def _attention_trees(gs: Sequence[_Group]):
    """The six store sites' expressions, if they have the attention shape:
    (S leaf of P, M leaf of P, L leaf of Y, O leaf of Y, scale) else None.
    S and O are tile matmuls accumulated over K, M = reduce_max(S) and
    L = reduce_sum(P, 1) along dim 1, P as _softmax_numerator takes it, Y is
    O * recip(bcast(L)) or O / bcast(L)."""
    g1, g2, g3, g4, g5, g6 = gs
    for g in (g1, g5):
        if not (g.tree[0] == "matmul" and _plain_leaf(g.tree[1]) and _plain_leaf(g.tree[2])
                and g.acc):
            return None
    for g, kind in ((g2, "max"), (g4, "sum")):
        t = g.tree
        if not (t[0] == "reduce" and t[1] == kind and tuple(t[2]) == (1,) and _plain_leaf(t[3])
                and _is_const(t[5]) and not g.acc):
            return None
    if g3.acc or g6.acc or float(g4.tree[5][1]) != 1.0:
        return None
    num = _softmax_numerator(g3.tree, float(g2.tree[5][1]))
    if num is None:
        return None
    s_leaf, m_leaf, scale = num
    col = (False, True)
    t6 = g6.tree
    if t6[0] == "mul" and _plain_leaf(t6[1]) and t6[2][0] == "recip" and _plain_leaf(t6[2][1], col):
        o_leaf, l_leaf = t6[1], t6[2][1]
    elif t6[0] == "mul" and _plain_leaf(t6[2]) and t6[1][0] == "recip" and _plain_leaf(t6[1][1], col):
        o_leaf, l_leaf = t6[2], t6[1][1]
    elif t6[0] == "div" and _plain_leaf(t6[1]) and _plain_leaf(t6[2], col):
        o_leaf, l_leaf = t6[1], t6[2]
    else:
        return None
    return s_leaf, m_leaf, l_leaf, o_leaf, scale


def _leaf_index(g: _Group, leaf) -> int:
    for i, lf in enumerate(_tree_leaves(g.tree, [])):
        if lf is leaf:
            return i
    raise AssertionError("leaf not in the group's tree")


def _tile_keys(rc: np.ndarray) -> np.ndarray:
    return rc[:, 0].astype(np.int64) * (1 << 31) + rc[:, 1]


class _TileMap:
    """A bijection from logical indices 0..n-1 to the tiles (keys) of one
    tensor, read off the instances of one store site and checked: every index
    lands on one tile, distinct indices on distinct tiles."""

    def __init__(self, n: int, idx: np.ndarray, keys: np.ndarray, what: str) -> None:
        tab = np.full(n, -1, dtype=np.int64)
        tab[idx] = keys
        if np.any(tab[idx] != keys) or np.any(tab < 0) or np.unique(tab).size != n:
            raise _NoAttention(what)
        self.tab = tab
        self.order = np.argsort(tab)

    def index(self, keys: np.ndarray, what: str) -> np.ndarray:
        pos = np.searchsorted(self.tab, keys, sorter=self.order)
        pos = np.minimum(pos, self.tab.size - 1)
        idx = self.order[pos]
        if np.any(self.tab[idx] != keys):
            raise _NoAttention(what)
        return idx


class _NoAttention(Exception):
    pass


def _all_once(keys: np.ndarray, n: int, what: str) -> None:
    if keys.size != n or np.unique(keys).size != n:
        raise _NoAttention(what)


def _match_attention(gs: Sequence[_Group], tensor_ref) -> Optional[SdpaLaunch]:
    """The six store sites as one SdpaLaunch, or None when they are not
    attention.  Checked beyond the expression shapes: Q, K^T, V and the
    output are bf16 kernel tensors [N, D] / [D, N] with D = 64 or 128 and
    S, M, P, L, O intermediate CBs; and every tile instance is where
    attention puts it — for query tile r of head h = r // (S/32), S(r, j)
    accumulates Q(r, k) K^T(k, h*S/32 + j) over all k, M(r) reduces
    S(r, 0..), P(r, j) reads S(r, j) and M(r), L(r) reduces P(r, 0..),
    O(r, d) accumulates P(r, j) V(h*S/32 + j, d) over all j, and Y(r, d)
    reads O(r, d) and L(r)."""
    g1, g2, g3, g4, g5, g6 = gs
    m = _attention_trees(gs)
    if m is None:
        return None
    s_leaf, m_leaf, l_leaf, o_leaf, scale = m
    q_t, kt_t = g1.leaf_tensors
    p_t, v_t = g5.leaf_tensors
    s_t, m_t, p_out, l_t, o_t, y_t = (g.out_tensor for g in gs)
    if not all(isinstance(t, _Scratch) for t in (s_t, m_t, p_out, l_t, o_t)):
        return None
    if (g2.leaf_tensors[0] is not s_t or g4.leaf_tensors[0] is not p_out or p_t is not p_out
            or g3.leaf_tensors[_leaf_index(g3, s_leaf)] is not s_t
            or g3.leaf_tensors[_leaf_index(g3, m_leaf)] is not m_t
            or g6.leaf_tensors[_leaf_index(g6, o_leaf)] is not o_t
            or g6.leaf_tensors[_leaf_index(g6, l_leaf)] is not l_t):
        return None
    for t in (q_t, kt_t, v_t, y_t):
        if isinstance(t, _Temp) or getattr(t, "is_block_float", False) or len(t.shape) != 2:
            return None
    if any(t.dtype != torch.bfloat16 for t in (q_t, kt_t, v_t, y_t)):
        raise PlanError("fused attention takes bfloat16 Q, K^T, V and output tensors")
    N, D = q_t.shape
    if (tuple(kt_t.shape) != (D, N) or tuple(v_t.shape) != (N, D) or tuple(y_t.shape) != (N, D)
            or D not in (64, 128) or N % TILE):
        raise PlanError("fused attention takes Q, V, output [B*H*S, D] and K^T [D, B*H*S] with "
                        "D = 64 or 128")
    if not scale > 0:
        raise PlanError("fused attention needs a positive softmax scale")
    R, dt = N // TILE, D // TILE
    try:
        # S(r, j) = sum_k Q(r, k) K^T(k, h*st + j)
        out1 = np.concatenate(g1.out_rc)
        qrc, krc = (np.concatenate([li[i] for li in g1.leaf_rc]) for i in (0, 1))
        if out1.shape[0] % (R * dt):
            raise _NoAttention("S instances")
        st = out1.shape[0] // (R * dt)
        if st == 0 or N % (st * TILE):
            raise _NoAttention("sequence length")
        r, k = qrc[:, 0], qrc[:, 1]
        j = krc[:, 1] - (r // st) * st
        if (np.any(krc[:, 0] != k) or np.any((k < 0) | (k >= dt)) or np.any((r < 0) | (r >= R))
                or np.any((j < 0) | (j >= st))):
            raise _NoAttention("S operands")
        _all_once((r * st + j) * dt + k, R * st * dt, "S products")
        smap = _TileMap(R * st, r * st + j, _tile_keys(out1), "S tiles")
        # M(r) = max_j S(r, j)
        out2, in2 = np.concatenate(g2.out_rc), np.concatenate([li[0] for li in g2.leaf_rc])
        si = smap.index(_tile_keys(in2), "M operand")
        _all_once(si, R * st, "M reads")
        mmap = _TileMap(R, si // st, _tile_keys(out2), "M tiles")
        # P(r, j) = exp(S(r, j) * c - M(r))
        out3 = np.concatenate(g3.out_rc)
        s3 = np.concatenate([li[_leaf_index(g3, s_leaf)] for li in g3.leaf_rc])
        m3 = np.concatenate([li[_leaf_index(g3, m_leaf)] for li in g3.leaf_rc])
        si = smap.index(_tile_keys(s3), "P operand")
        _all_once(si, R * st, "P reads")
        if np.any(mmap.index(_tile_keys(m3), "P max operand") != si // st):
            raise _NoAttention("P max operand")
        pmap = _TileMap(R * st, si, _tile_keys(out3), "P tiles")
        # L(r) = sum_j P(r, j)
        out4, in4 = np.concatenate(g4.out_rc), np.concatenate([li[0] for li in g4.leaf_rc])
        pi = pmap.index(_tile_keys(in4), "L operand")
        _all_once(pi, R * st, "L reads")
        lmap = _TileMap(R, pi // st, _tile_keys(out4), "L tiles")
        # O(r, d) = sum_j P(r, j) V(h*st + j, d)
        out5 = np.concatenate(g5.out_rc)
        prc, vrc = (np.concatenate([li[i] for li in g5.leaf_rc]) for i in (0, 1))
        pi = pmap.index(_tile_keys(prc), "O operand")
        r, j, d = pi // st, pi % st, vrc[:, 1]
        if np.any(vrc[:, 0] != (r // st) * st + j) or np.any((d < 0) | (d >= dt)):
            raise _NoAttention("O operands")
        _all_once((r * st + j) * dt + d, R * st * dt, "O products")
        omap = _TileMap(R * dt, r * dt + d, _tile_keys(out5), "O tiles")
        # Y(r, d) = O(r, d) / L(r)
        out6 = np.concatenate(g6.out_rc)
        o6 = np.concatenate([li[_leaf_index(g6, o_leaf)] for li in g6.leaf_rc])
        l6 = np.concatenate([li[_leaf_index(g6, l_leaf)] for li in g6.leaf_rc])
        oi = omap.index(_tile_keys(o6), "Y operand")
        _all_once(oi, R * dt, "Y reads")
        if np.any(lmap.index(_tile_keys(l6), "Y sum operand") != oi // dt):
            raise _NoAttention("Y sum operand")
        if np.any(out6[:, 0] != oi // dt) or np.any(out6[:, 1] != oi % dt):
            raise _NoAttention("Y tiles")
    except _NoAttention:
        return None
    launch = SdpaLaunch(tensor_ref(q_t), tensor_ref(kt_t), tensor_ref(v_t), tensor_ref(y_t),
                        N // (st * TILE), st * TILE, float(scale), kbuf=_Temp((N, D), torch.bfloat16))
    launch._reads, launch._writes = (q_t, kt_t, v_t), y_t
    return launch


def _fuse_attention(groups: List[_Group], tensor_ref) -> List[Any]:
    """The groups with every run of six that is attention (_match_attention)
    replaced by its SdpaLaunch; its intermediates must be read by nothing
    else."""
    out: List[Any] = []
    i = 0
    while i < len(groups):
        win = groups[i:i + 6]
        launch = _match_attention(win, tensor_ref) if len(win) == 6 else None
        if launch is not None:
            inter = {id(g.out_tensor) for g in win[:5]}
            rest = groups[:i] + groups[i + 6:]
            if not any(id(t) in inter for g in rest for t in g.leaf_tensors + [g.out_tensor]):
                launch.loc = win[-1].loc
                out.append(launch)
                i += 6
                continue
        out.append(groups[i])
        i += 1
    return out


def _tile_codes(rcs: List[np.ndarray]) -> np.ndarray:
    """Sorted unique tile coordinates of (N, 2) arrays, one int64 each."""
    if not rcs:
        return np.zeros(0, dtype=np.int64)
    a = np.concatenate(rcs, 0).astype(np.int64)
    return np.unique(a[:, 0] * (1 << 32) + a[:, 1])


def _mark_dedupe(groups: List[_Group]) -> None:
    """Repeats of a store site are one launch only when nothing else touches
    their tiles in between.  Store sites run one launch each in trace order,
    so the repeats of a site are merged (g.dedupe_ok) only if no other site
    writes a tile they read (loop { out = x + 1; x = y * 2 } computes out
    from two values of x), writes a tile they write (the last writer would
    change), or reads a tile they write (unless the output is a tensor the
    plan owns for this site alone, read back by its consumer at the tiles
    each repeat wrote: a hoisted matmul operand)."""
    for g in groups:
        g.dedupe_ok = True
    rep = [g for g in groups if sum(x.shape[0] for x in g.out_rc) >
           _tile_codes(g.out_rc).size]
    if not rep:
        return

    def reads(h: _Group) -> Dict[int, List[np.ndarray]]:
        r: Dict[int, List[np.ndarray]] = {}
        for k, t in enumerate(h.leaf_tensors):
            r.setdefault(id(t), []).extend(li[k] for li in h.leaf_rc)
        if h.scaler_tensor is not None:
            r.setdefault(id(h.scaler_tensor), []).extend(h.scaler_rc)
        return r

    writes = {id(h): _tile_codes(h.out_rc) for h in groups}
    read_sets = {id(h): reads(h) for h in groups}
    for g in rep:
        g_reads = {k: _tile_codes(v) for k, v in read_sets[id(g)].items()}
        g_writes = writes[id(g)]
        for h in groups:
            if h is g:
                continue
            hw = writes[id(h)]
            if id(h.out_tensor) in g_reads and np.intersect1d(hw, g_reads[id(h.out_tensor)]).size:
                g.dedupe_ok = False
            elif h.out_tensor is g.out_tensor and np.intersect1d(hw, g_writes).size:
                g.dedupe_ok = False
            elif (not getattr(g, "private_out", False) and id(g.out_tensor) in read_sets[id(h)]
                  and np.intersect1d(_tile_codes(read_sets[id(h)][id(g.out_tensor)]),
                                     g_writes).size):
                g.dedupe_ok = False
            if not g.dedupe_ok:
                break


def build_plan(groups: List[_Group], tensor_ref) -> Plan:
    plan = Plan()
    _mark_dedupe(groups)
    inl = _Inliner(groups)
    for g in _fuse_attention(groups, tensor_ref):
        if isinstance(g, SdpaLaunch):
            plan.launches.append(g)
            inl.note_reads(g._reads)
            inl.note_write(g._writes)
            continue
        out_rc = np.concatenate(g.out_rc, 0)
        leaf_rc = [np.concatenate([li[k] for li in g.leaf_rc], 0) for k in range(len(g.leaf_blocks))]
        if g.tree[0] == "reduce":
            launch = _plan_reduce(g, out_rc, leaf_rc, np.concatenate(g.order), tensor_ref, inl)
        elif g.tree[0] == "matmul" and g.tree[1][0] == "leaf" and g.tree[2][0] == "leaf":
            launch = _plan_matmul(g, out_rc, leaf_rc, tensor_ref)
            inl.note_reads(g.leaf_tensors)
        elif _has(g.tree, "matmul"):
            raise PlanError("a tile matmul combined with other ops in one store() is not "
                            "supported; store the product on its own")
        else:
            launches = _plan_eltwise_parts(g, out_rc, leaf_rc, tensor_ref, inl)
            for launch in launches:
                launch.loc = g.loc
                plan.launches.append(launch)
            if len(launches) == 1:
                inl.register(g, launches[0], getattr(launches[0], "_subbed", ()))
            inl.note_write(g.out_tensor)
            continue
        launch.loc = g.loc
        plan.launches.append(launch)
        inl.note_write(g.out_tensor)
    inl.finish(plan)
    _fuse_epilogues(plan)
    _fuse_row_reductions(plan)
    return plan


def _launch_refs(l) -> List[TensorRef]:
    if isinstance(l, FusedMatmulLaunch):
        return _launch_refs(l.mm) + _launch_refs(l.ew)
    if isinstance(l, ReduceEltwiseLaunch):
        return [r for x in l.reds for r in _launch_refs(x)] + _launch_refs(l.ew)
    if isinstance(l, (EltwiseLaunch, ReduceLaunch)):
        r = [l.out] + [s.ref for s in l.operands if s is not None]
        if isinstance(l, ReduceLaunch) and l.scaler is not None:
            r.append(l.scaler)
        return r
    if isinstance(l, SdpaLaunch):
        return [l.q, l.kt, l.v, l.out]
    return [l.a, l.b, l.c]


def _fuse_epilogues(plan: Plan) -> None:
    """A matmul launch into a hoisted product tensor (_hoist_matmuls),
    immediately followed by the elementwise launch over the same output
    rectangle that reads the product at each output element (identity map)
    from exactly one step, the product tensor referenced by no other launch:
    the pair becomes one FusedMatmulLaunch."""
    L = plan.launches
    out: List[Any] = []
    i = 0
    while i < len(L):
        l = L[i]
        if (isinstance(l, MatmulLaunch) and not l.b_block and type(l.c.obj) is _Temp
                and i + 1 < len(L) and isinstance(L[i + 1], EltwiseLaunch)):
            ew = L[i + 1]
            temp = l.c.obj
            steps = [k for k, s in enumerate(ew.operands) if s is not None and s.ref.obj is temp]
            (r0, r1), (c0, c1) = l.rows, l.cols
            others = sum(1 for x in L if x is not l and x is not ew
                         for r in _launch_refs(x) if r.obj is temp)
            if (len(steps) == 1 and others == 0
                    and (ew.operands[steps[0]].row_mask, ew.operands[steps[0]].col_mask,
                         ew.operands[steps[0]].row_off, ew.operands[steps[0]].col_off)
                    == (-1, -1, 0, 0)
                    and tuple(ew.region) == (r0, c0, r1 - r0, c1 - c0)
                    and temp.dtype == torch.bfloat16):
                out.append(FusedMatmulLaunch(l, ew, steps[0], ew.loc or l.loc))
                i += 2
                continue
        out.append(l)
        i += 1
    plan.launches = out


_MAX_ROW_REDUCTIONS = 3  # ttlh_reduce_rows_eltwise's limit


def _fuse_row_reductions(plan: Plan) -> None:
    """One to three row reductions (dims [1]) over one region, immediately
    followed by the elementwise launch over that region: the run becomes one
    ReduceEltwiseLaunch.  Whether the library takes it (the later programs
    reading each result as their rows' value, the op set, the row width) is
    decided when it runs; otherwise the launches run as planned."""
    L = plan.launches
    out: List[Any] = []
    i = 0
    while i < len(L):
        j = i
        while (j < len(L) and j - i < _MAX_ROW_REDUCTIONS and isinstance(L[j], ReduceLaunch)
               and L[j].dims == (1,) and tuple(L[j].region) == tuple(L[i].region)):
            j += 1
        if (j > i and j < len(L) and isinstance(L[j], EltwiseLaunch)
                and tuple(L[j].region) == tuple(L[i].region)):
            out.append(ReduceEltwiseLaunch(list(L[i:j]), L[j], L[j].loc or L[i].loc))
            i = j + 1
            continue
        out.append(L[i])
        i += 1
    plan.launches = out


def _dedupe_writes(g: _Group, out_rc, leaf_rc):
    """Store instances that repeat another exactly (same output tile, same
    tile of every operand), e.g. every core of a grid running the same loop
    (examples/broadcast_demo.py with grid="auto"): the simulator writes the
    same values several times, one launch writes them once.  Only for plain
    stores whose output is not also an operand (then repeats are not
    idempotent) and whose tensors no other store site writes or reads
    between the repeats (g.dedupe_ok, _mark_dedupe); instances that write one
    tile with different operands stay and are refused by the caller."""
    n = out_rc.shape[0]
    if g.acc or n == 0 or _unique_tiles(out_rc) == n or not g.dedupe_ok:
        return out_rc, leaf_rc
    if any(t is g.out_tensor for t in g.leaf_tensors):
        return out_rc, leaf_rc
    rows = np.concatenate([out_rc] + list(leaf_rc), 1)
    _, keep = np.unique(rows, axis=0, return_index=True)
    keep.sort()
    if _unique_tiles(out_rc[keep]) != keep.size:
        return out_rc, leaf_rc
    return out_rc[keep], [x[keep] for x in leaf_rc]


def _plan_eltwise(g: _Group, out_rc, leaf_rc, tensor_ref,
                  inl: Optional["_Inliner"] = None) -> List[EltwiseLaunch]:
    out_rc, leaf_rc = _dedupe_writes(g, out_rc, leaf_rc)
    n = out_rc.shape[0]
    if _unique_tiles(out_rc) != n:
        if g.acc:
            raise PlanError("store(acc=True) of an elementwise expression into the same output "
                            "tile more than once is not supported (only tile matmul accumulates)")
        raise PlanError("an output tile is written more than once")
    r0, r1, c0, c1 = _rect(out_rc)
    if (r1 - r0) * (c1 - c0) != n:
        raise PlanError("the stored output tiles do not form a rectangle of the output tensor")
    out_t = g.out_tensor
    H, W = out_t.shape
    if getattr(out_t, "is_block_float", False):
        raise PlanError(f"storing into a {out_t.dtype.name} tensor is not supported (block-float "
                        "tensors are read-only tile-matmul weights here)")
    for tens in g.leaf_tensors:
        if getattr(tens, "is_block_float", False):
            raise PlanError(f"a {tens.dtype.name} tensor as an elementwise operand is not "
                            "supported; it can be the B operand of a tile matmul")
    specs, nodes, plain, subbed = _leaf_operands(g, out_rc, leaf_rc, tensor_ref, inl)
    e = _to_expr(g.tree, nodes)
    if subbed and _program_size(e) == 0:  # the fused program does not fit: keep the stage
        e, subbed = _to_expr(g.tree, plain), set()
    if inl is not None:
        inl.note_reads(g.leaf_tensors, subbed)
    y0, x0 = r0 * TILE, c0 * TILE
    h = min(r1 * TILE, H) - y0
    w = min(c1 * TILE, W) - x0
    pre, prog, operands = _fit_program(e, specs, (H, W), (y0, x0, h, w), n)
    launch = EltwiseLaunch(prog, operands, tensor_ref(out_t), (y0, x0, h, w), n)
    if not pre:
        launch._expr, launch._specs, launch._subbed = e, dict(specs), subbed
    return pre + [launch]


def _expr_nodes(e: X.Expr, out: List[X.Expr]) -> List[X.Expr]:
    out.append(e)
    if isinstance(e, X.Unary):
        _expr_nodes(e.x, out)
    elif isinstance(e, X.Binary):
        _expr_nodes(e.a, out)
        _expr_nodes(e.b, out)
    return out


def _expr_replace(e: X.Expr, old: X.Expr, new: X.Expr) -> X.Expr:
    if e is old:
        return new
    if isinstance(e, X.Unary):
        x = _expr_replace(e.x, old, new)
        return e if x is e.x else dataclasses.replace(e, x=x)
    if isinstance(e, X.Binary):
        a, b = _expr_replace(e.a, old, new), _expr_replace(e.b, old, new)
        return e if (a is e.a and b is e.b) else dataclasses.replace(e, a=a, b=b)
    return e


def _program_size(e: X.Expr) -> int:
    """Steps of e's program, or 0 when it exceeds the kernel's limits."""
    try:
        return len(X.compile_expr(e).steps)
    except NotImplementedError as err:
        if "fused tile expression needs" in str(err):
            return 0
        raise


def _fit_program(e: X.Expr, specs: Dict[int, OperandSpec], out_shape, region, n_tiles):
    """Compiles e.  When its fused program exceeds the kernel's step or stack
    limit (test/python/many_fused_ops.py chains 20 ops), the largest proper
    subexpression that fits is computed first, by a launch of its own into a
    temporary tensor of the output's shape (in its dtype, so the value is
    stored exactly), and read back as an operand; repeated until the rest
    fits.  Returns (launches to run first, program, operands)."""
    pre: List[EltwiseLaunch] = []
    while _program_size(e) == 0:
        best, size = None, 1
        for node in _expr_nodes(e, [])[1:]:
            if isinstance(node, (X.Leaf, X.Const)):
                continue
            k = _program_size(node)
            if k > size:
                best, size = node, k
        if best is None:
            X.compile_expr(e)  # raises the limit error
        tmp = _Temp(out_shape, best.dtype)
        sprog = X.compile_expr(best)
        pre.append(EltwiseLaunch(sprog, [specs[st.leaf.ref] if st.leaf is not None else None
                                         for st in sprog.steps], TensorRef(obj=tmp), region,
                                 n_tiles))
        k = max(specs) + 1 if specs else 0
        specs[k] = OperandSpec(TensorRef(obj=tmp), -1, -1, 0, 0)
        e = _expr_replace(e, best, X.Leaf(k, best.dtype))
    prog = X.compile_expr(e)
    return pre, prog, [specs[st.leaf.ref] if st.leaf is not None else None for st in prog.steps]


def _plan_eltwise_parts(g: _Group, out_rc, leaf_rc, tensor_ref,
                        inl: Optional["_Inliner"] = None) -> List[EltwiseLaunch]:
    """One launch when every operand is an affine image of the output tiles;
    otherwise the store's instances are split by the tile of the first
    operand that is not (that operand is then one fixed tile in each part)
    and each part planned the same way, e.g. a tile held across a loop over
    a block of output tiles (test/python/test_bcast_multicore.py).  Each part
    must still write a rectangle of output tiles.  The split is along the
    axis whose map failed only."""
    try:
        return _plan_eltwise(g, out_rc, leaf_rc, tensor_ref, inl)
    except _NotAffine as err:
        k = err.leaf
        if k < 0:
            raise
        if inl is not None:  # the parts read their operands as they are
            inl.note_reads(g.leaf_tensors)
        uniq, inv = np.unique(leaf_rc[k][:, err.axis], return_inverse=True)
        if uniq.size > _MAX_PARTS or uniq.size == 1:
            raise
        out: List[EltwiseLaunch] = []
        for u in range(uniq.size):
            sel = inv == u
            out += _plan_eltwise_parts(g, out_rc[sel], [x[sel] for x in leaf_rc], tensor_ref)  # no inlining in parts
            if len(out) > _MAX_PARTS:
                raise PlanError(f"a store site needs more than {_MAX_PARTS} launches: its "
                                "operands' tiles follow the output tiles in no affine way") from err
        return out


def _plan_reduce(g: _Group, out_rc, leaf_rc, order, tensor_ref,
                 inl: Optional["_Inliner"] = None) -> ReduceLaunch:
    """Iteration space: output tile coordinates along the kept axes, the tile
    coordinates of the first operand that varies along a reduced axis there.
    Every operand must be an affine image of it (as for eltwise), every
    output tile must collect one rectangle row / column of it."""
    _, kind, dims, inner, ishape, stree = g.tree
    n = out_rc.shape[0]
    out_t = g.out_tensor
    if getattr(out_t, "is_block_float", False) or any(
            getattr(t, "is_block_float", False) for t in g.leaf_tensors):
        raise PlanError("block-float tensors are supported as the B operand of a tile matmul only")
    it = np.empty((n, 2), dtype=np.int64)
    degenerate = [False, False]  # iteration axis of one element (size-1 tensor dimension)
    for ax in (0, 1):
        if ax not in dims:
            it[:, ax] = out_rc[:, ax]
            degenerate[ax] = out_t.shape[ax] == 1
            continue
        cands = [k for k in range(len(leaf_rc)) if g.leaf_tensors[k].shape[ax] > 1]
        varying = [k for k in cands if not np.all(leaf_rc[k][:, ax] == leaf_rc[k][0, ax])]
        prim = varying[0] if varying else (cands[0] if cands else 0)
        it[:, ax] = leaf_rc[prim][:, ax]
        degenerate[ax] = not cands
    key = it[:, 0] * (int(it[:, 1].max()) + 1) + it[:, 1]
    if np.unique(key).size != n:
        raise PlanError("a reduction reads an expression tile twice (every output tile must "
                        "reduce distinct tiles of its operands)")
    r0, r1, c0, c1 = _rect(it)
    if (r1 - r0) * (c1 - c0) != n:
        raise PlanError("the tiles a reduction reads do not form a rectangle")
    out_tile = [0, 0]
    for ax in (0, 1):
        o = out_rc[:, ax]
        if ax in dims:
            if not np.all(o == o[0]):
                raise PlanError("the reduced tiles of one store site land in more than one output "
                                "tile along the reduced dimension (only one run of tiles per "
                                "output tile is supported)")
            out_tile[ax] = int(o[0])
        else:
            d = o - it[:, ax]
            if not np.all(d == d[0]):
                raise PlanError("reduction output tiles are not an offset of the reduced tiles")
            out_tile[ax] = int(d[0]) + (r0 if ax == 0 else c0)
    # stores per output tile: several only when they accumulate a sum
    okey = out_rc[:, 0] * (int(out_rc[:, 1].max()) + 1) + out_rc[:, 1]
    pairs = np.unique(np.stack([okey, order], 1), axis=0)
    multi = np.unique(pairs[:, 0]).size != pairs.shape[0]
    if multi and not g.acc:
        raise PlanError("an output tile is stored more than once without acc=True")
    if multi and kind == "max":
        raise PlanError("reduce_max partial results accumulated with store(acc=True) would be "
                        "added (store acc semantics); reduce over one block per output tile")
    # operands
    specs, nodes, plain, subbed = _leaf_operands(g, it, leaf_rc, tensor_ref, inl)
    e = _to_expr(inner, nodes)
    if subbed and _program_size(e) == 0:
        e, subbed = _to_expr(inner, plain), set()
    if inl is not None:
        inl.note_reads(g.leaf_tensors, subbed)
        if g.scaler_tensor is not None:  # the scaler is read as it is
            inl.note_read(g.scaler_tensor, False)
    prog = X.compile_expr(e)
    operands = [specs[s.leaf.ref] if s.leaf is not None else None for s in prog.steps]
    y0, x0 = r0 * TILE, c0 * TILE
    h = 1 if degenerate[0] else (r1 - r0) * TILE
    w = 1 if degenerate[1] else (c1 - c0) * TILE
    # result placement: size-1 tensor dimensions take the value only, full
    # tiles the zero-padded result tile
    red_sizes = [out_t.shape[ax] for ax in dims]
    pads = {sz > 1 for sz in red_sizes}
    if len(pads) != 1:
        raise PlanError("a reduction over both dims needs an output that is size 1 in both or "
                        "whole tiles in both")
    out_pad = pads.pop()
    oy = 0 if (0 in dims and out_t.shape[0] == 1) else out_tile[0] * TILE
    ox = 0 if (1 in dims and out_t.shape[1] == 1) else out_tile[1] * TILE
    scaler_ref, scaler_at, scale = None, (0, 0), 1.0
    if stree[0] == "const":
        scale = float(stree[1])
    else:
        src = np.concatenate(g.scaler_rc, 0)
        if not np.all(src == src[0]):
            raise PlanError("a reduction's scaler must be the same tile for every store")
        st_ = g.scaler_tensor
        sr = int(src[0, 0]) * TILE if st_.shape[0] > 1 else 0
        sc = int(src[0, 1]) * TILE if st_.shape[1] > 1 else 0
        scaler_ref, scaler_at = tensor_ref(st_), (sr, sc)
    return ReduceLaunch(prog, operands, tensor_ref(out_t), kind, tuple(dims), (y0, x0, h, w),
                        (oy, ox), out_pad, scaler_ref, scaler_at, scale, n)


def _plan_matmul(g: _Group, out_rc, leaf_rc, tensor_ref) -> MatmulLaunch:
    a_t, b_t = g.leaf_tensors
    (ar, ac), (br, bc) = leaf_rc[0].T, leaf_rc[1].T
    orow, ocol = out_rc[:, 0], out_rc[:, 1]
    # A's rows and B's columns may sit at a fixed offset from the output's
    # (a product stored elsewhere, or split off a store expression)
    da, db = (int(ar[0] - orow[0]), int(bc[0] - ocol[0])) if ar.size else (0, 0)
    if not (np.array_equal(ar - orow, np.full_like(ar, da))
            and np.array_equal(bc - ocol, np.full_like(bc, db)) and np.array_equal(ac, br)):
        raise PlanError("tile matmul operands are not A(m + i, k) @ B(k, n + j) for output "
                        "tile (m, n) with fixed offsets i, j")
    if len(a_t.shape) != 2 or len(b_t.shape) != 2 or a_t.shape[1] != b_t.shape[0]:
        raise PlanError("tile matmul operand shapes do not chain")
    K = a_t.shape[1]
    kt = K // TILE
    n_out = _unique_tiles(out_rc)
    key = (orow * (int(ocol.max()) + 1) + ocol) * (kt + 1) + ac
    if np.unique(key).size != key.size:
        raise PlanError("a (output tile, k) product is accumulated twice")
    # every output tile sums the same k tiles: all of K, or (one round of an
    # accumulating store whose expression holds the product) one contiguous
    # part of it
    k0, k1 = (int(ac.min()), int(ac.max()) + 1) if ac.size else (0, kt)
    if key.size != n_out * (k1 - k0) or (not g.acc and k1 - k0 != 1):
        raise PlanError("every output tile must accumulate A(m,k) @ B(k,n) over all k "
                        "(store(acc=True) inside the K loop)")
    r0, r1, c0, c1 = _rect(out_rc)
    if (r1 - r0) * (c1 - c0) != n_out:
        raise PlanError("the matmul output tiles do not form a rectangle")
    if getattr(a_t, "is_block_float", False) or getattr(g.out_tensor, "is_block_float", False):
        raise PlanError("block-float tensors are supported as the B operand of a tile matmul only")
    b_block = getattr(b_t, "is_block_float", False)
    if b_block:
        if (c0, c1) != (0, b_t.shape[1] // TILE) or db != 0:
            raise PlanError(f"a {b_t.dtype.name} B operand must be used over all of its columns")
        if (k0, k1) != (0, kt):
            raise PlanError(f"a {b_t.dtype.name} B operand must be used over all of its rows")
        if a_t.dtype != torch.bfloat16 or g.out_tensor.dtype != torch.bfloat16:
            raise PlanError(f"the {b_t.dtype.name} matmul takes bfloat16 A and output tensors")
    part = (k0, k1) != (0, kt)
    return MatmulLaunch(tensor_ref(a_t), tensor_ref(b_t), tensor_ref(g.out_tensor),
                        (r0 * TILE, r1 * TILE), (c0 * TILE, c1 * TILE), (k1 - k0) * TILE, b_block,
                        a_rows=((r0 + da) * TILE, (r1 + da) * TILE) if da else None,
                        b_cols=((c0 + db) * TILE, (c1 + db) * TILE) if db else None,
                        k_range=(k0 * TILE, k1 * TILE) if part else None)


# ---------------------------------------------------------------------------
# execution


def execute(plan: Plan, args: Dict[Any, Any], stream=None, events=None) -> None:
    """Runs the plan's launches on the current (or given) stream.  With an
    `events` list, a pair of timing events is recorded around every launch."""
    from . import kernels as Kn
    from ._lib import require_device

    require_device()
    for l in plan.launches:
        if events is not None:
            # a short device spin ahead of the start event keeps the GPU busy
            # while the host enqueues the launch, so the events bracket device
            # time only (not the host's launch latency)
            with torch.cuda.stream(stream if stream is not None else torch.cuda.current_stream()):
                torch.cuda._sleep(200_000)
            e0 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
        _execute_one(l, args, stream, Kn)
        if events is not None:
            e1 = torch.cuda.Event(enable_timing=True)
            e1.record(stream)
            events.append((e0, e1))


def _execute_one(l, args, stream, Kn) -> None:
    if isinstance(l, EltwiseLaunch):
        ops = []
        for spec in l.operands:
            if spec is None:
                ops.append(None)
                continue
            ops.append(Kn.OperandMap(spec.ref.resolve(args), spec.row_mask, spec.col_mask,
                                     spec.row_off, spec.col_off))
        Kn.eltwise(l.prog, ops, l.out.resolve(args), region=l.region, stream=stream)
    elif isinstance(l, ReduceLaunch):
        ops = [None if spec is None else
               Kn.OperandMap(spec.ref.resolve(args), spec.row_mask, spec.col_mask, spec.row_off,
                             spec.col_off) for spec in l.operands]
        sc = None
        if l.scaler is not None:
            r, c = l.scaler_at
            sc = l.scaler.resolve(args)[r:r + 1, c:c + 1]
        Kn.reduce(l.prog, ops, l.kind, l.dims, l.out.resolve(args), l.region, l.out_origin,
                  l.out_pad, sc, l.scale, stream=stream)
    elif isinstance(l, FusedMatmulLaunch):
        if not _execute_fused(l, args, stream, Kn):
            _execute_one(l.mm, args, stream, Kn)
            _execute_one(l.ew, args, stream, Kn)
    elif isinstance(l, ReduceEltwiseLaunch):
        if not _execute_row_fused(l, args, stream, Kn):
            for r in l.reds:
                _execute_one(r, args, stream, Kn)
            _execute_one(l.ew, args, stream, Kn)
    elif isinstance(l, SdpaLaunch):
        q, kt, v, y = (r.resolve(args) for r in (l.q, l.kt, l.v, l.out))
        k = kt.t()
        if not k.is_contiguous():  # K^T stored as such: its rows transposed once more
            k = l.kbuf._tensor
            Kn.transpose(kt, k, stream=stream)
        if not (q.is_contiguous() and v.is_contiguous() and y.is_contiguous()):
            raise ValueError("fused attention takes contiguous Q, V and output tensors")
        lo, hi = y.data_ptr(), y.data_ptr() + y.numel() * y.element_size()
        for t in (q, k, v):
            if t.data_ptr() < hi and lo < t.data_ptr() + t.numel() * t.element_size():
                raise ValueError("fused attention output overlaps an input")
        shape = (1, l.heads, l.seq, q.shape[1])
        Kn.sdpa_fwd(q.view(shape), k.view(shape), v.view(shape), y.view(shape), l.scale,
                    stream=stream)
    else:
        a, b, c = l.a.resolve(args), l.b.resolve(args), l.c.resolve(args)
        if c.data_ptr() in (a.data_ptr(), b.data_ptr()):
            raise ValueError("matmul output aliases an input")
        r0, r1 = l.rows
        c0, c1 = l.cols
        (ar0, ar1), (bc0, bc1) = l.operand_ranges()
        ks = l.k_slice()
        if l.b_block:
            l.b.resolve_obj(args).dtype.matmul(a[ar0:ar1], b, c[r0:r1], stream=stream)
        else:
            Kn.matmul(a[ar0:ar1, ks], b[ks, bc0:bc1], c[r0:r1, c0:c1], accumulate=False,
                      stream=stream)


def _execute_fused(l: FusedMatmulLaunch, args, stream, Kn, force: bool = False) -> bool:
    """One ttlh_matmul_eltwise launch when it takes the problem and is
    expected to be the faster of the two forms (always when `force`); False
    (nothing launched) otherwise."""
    from . import _lib as L
    m, ew = l.mm, l.ew
    a, b, out = m.a.resolve(args), m.b.resolve(args), ew.out.resolve(args)
    (ar0, ar1), (bc0, bc1) = m.operand_ranges()
    ks = m.k_slice()
    aa, bb = a[ar0:ar1, ks], b[ks, bc0:bc1]
    M, K = aa.shape
    N = bb.shape[1]
    if aa.dtype != torch.bfloat16 or bb.dtype != torch.bfloat16:
        return False
    if not Kn.matmul_eltwise_supported(M, N, K, ew.prog):
        return False
    if not (force or Kn.matmul_eltwise_preferred(ew.prog)):
        return False
    lo, hi = out.data_ptr(), out.data_ptr() + out.numel() * out.element_size()
    for t in (a, b):
        if t.data_ptr() < hi and lo < t.data_ptr() + t.numel() * t.element_size():
            return False
    ops = []
    for k, spec in enumerate(ew.operands):
        if spec is None or k == l.prod_step:
            ops.append(None)
            continue
        t = spec.ref.resolve(args)
        if t.data_ptr() < hi and lo < t.data_ptr() + t.numel() * t.element_size():
            return False  # the fused kernel reads operands ahead of its stores
        ops.append(Kn.OperandMap(t, spec.row_mask, spec.col_mask, spec.row_off, spec.col_off))
    try:
        Kn.matmul_eltwise(aa, bb, ew.prog, ops, l.prod_step, out, ew.region, stream=stream)
    except L.TTLHError as err:
        if err.code != L.TTLH_EUNSUPPORTED:
            raise
        return False  # refused before launching (operand alignment): two launches
    return True


def _op_maps(operands, args, Kn):
    return [None if spec is None else
            Kn.OperandMap(spec.ref.resolve(args), spec.row_mask, spec.col_mask, spec.row_off,
                          spec.col_off) for spec in operands]


def _execute_row_fused(l: ReduceEltwiseLaunch, args, stream, Kn) -> bool:
    """One ttlh_reduce_rows_eltwise launch; False (nothing launched) where
    the library refuses the combination."""
    reds = []
    for r in l.reds:
        sc = None
        if r.scaler is not None:
            y, x = r.scaler_at
            sc = r.scaler.resolve(args)[y:y + 1, x:x + 1]
        reds.append(Kn.RowReduce(r.prog, _op_maps(r.operands, args, Kn), r.kind,
                                 r.out.resolve(args), r.out_origin, r.out_pad, sc, r.scale))
    return Kn.reduce_rows_eltwise(reds, l.ew.prog, _op_maps(l.ew.operands, args, Kn),
                                  l.ew.out.resolve(args), l.ew.region, stream=stream)
