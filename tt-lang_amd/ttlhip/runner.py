"""@ttl.kernel call path: body -> per-core traces -> plan -> GPU launches.

Mirrors the reference's two front doors: the simulator's kernel wrapper
(python/sim/kernel.py:202-291: run the body with `grid` injected, require one
compute and two data-movement threads, run every core) and the compiler's
pykernel_gen (python/ttl/ttl_api.py:1125-1249: compile once per argument
shapes / dtypes, then launch).  The plan for a given (shapes, dtypes, grid)
is cached, so repeated calls cost only the launches.
"""

from __future__ import annotations

import inspect
import os
import sys
import types
from typing import Any, Dict, List, Optional, Tuple

import numpy as np
import torch

import ttnn

from . import dsl
from . import profile
from . import plan as P
from . import trace as T


def _trace_print(*args, **kwargs):
    """Thread bodies run at trace time (once per core, loops vectorised);
    their prints are shown only with TTLH_TRACE_PRINT=1."""
    if os.environ.get("TTLH_TRACE_PRINT") == "1":
        print(*args, **kwargs)


def _refs(plan: P.Plan):
    for l in plan.launches:
        yield from P._launch_refs(l)


class KernelRunner:
    def __init__(self, func, grid: Tuple[int, ...], grid_spec, options: Dict[str, Any]):
        self.func = func
        self.grid = grid
        self.grid_spec = grid_spec
        self.options = options
        self.__name__ = func.__name__
        self.__doc__ = func.__doc__
        self.__wrapped__ = func
        self.__pykernel_config__ = {"grid": grid_spec}
        self._cache: Dict[Any, P.Plan] = {}
        self.last_plan: Optional[P.Plan] = None
        self.sync = options.get("sync", True)

    # -- cache key -----------------------------------------------------------
    @staticmethod
    def _key_of(v):
        if hasattr(v, "_tensor") and isinstance(v._tensor, torch.Tensor):
            return ("T", tuple(v.shape), str(v.dtype))
        if isinstance(v, torch.Tensor):
            return ("t", tuple(v.shape), str(v.dtype))
        try:
            hash(v)
            return ("v", v)
        except TypeError:
            return ("id", id(v))

    def _cache_key(self, args, kwargs):
        # The plan binds every tensor to the first argument position holding
        # it, so which positions hold the same object is part of the key:
        # k(a, a, out) and k(a, b, out) must not share a plan.
        first: Dict[int, Any] = {}
        alias = []
        for p, v in list(enumerate(args)) + sorted(kwargs.items()):
            alias.append(first.setdefault(id(v), p))
        return (tuple(self._key_of(a) for a in args),
                tuple(sorted((k, self._key_of(v)) for k, v in kwargs.items())),
                tuple(alias))

    @staticmethod
    def _check_layouts(args, kwargs) -> None:
        """Kernel tensors must be tilized (python/ttl/ttl_api.py:489-506)."""
        for i, a in enumerate(list(args) + list(kwargs.values())):
            lay = getattr(a, "layout", None)
            if isinstance(a, ttnn.Tensor) and "TILE" not in str(lay):
                raise ValueError(
                    f"TTNN interop requires tilized tensors, but tensor {i} has layout {lay}. "
                    "Use ttnn.to_layout(tensor, ttnn.TILE_LAYOUT) to convert.")

    # -- tracing ---------------------------------------------------------------
    def trace(self, *args, **kwargs) -> P.Plan:
        """Runs the kernel body and traces every core; returns the plan (no GPU)."""
        self._check_layouts(args, kwargs)
        g = dict(self.func.__globals__)
        g["grid"] = self.grid
        body = types.FunctionType(self.func.__code__, g, self.func.__name__,
                                  self.func.__defaults__, self.func.__closure__)
        prev = dsl._kstate
        dsl._kstate = dsl._KernelState(self.grid)
        dsl._last_grid = tuple(self.grid)
        prev_created, ttnn._created = ttnn._created, []
        try:
            body(*args, **kwargs)
            threads = list(dsl._kstate.threads)
            explicit = dsl._kstate.program_order
            created = ttnn._created
        finally:
            dsl._kstate = prev
            ttnn._created = prev_created
        if len(threads) != 3:
            raise ValueError(f"Kernel must define exactly 3 threads (compute, dm0, dm1), got "
                             f"{len(threads)}")
        comp = [t for t in threads if t.kind == "compute"]
        dms = [t for t in threads if t.kind == "dm"]
        if len(comp) != 1:
            raise ValueError(f"Kernel must define exactly 1 compute thread, got {len(comp)}")
        if len(dms) != 2:
            raise ValueError(f"Kernel must define exactly 2 datamovement threads, got {len(dms)}")
        ordered = [comp[0], dms[0], dms[1]]
        if explicit is not None:
            if [t.kind for t in explicit] != ["compute", "dm", "dm"]:
                raise ValueError("Program() expects (compute, dm0, dm1): one ttl.compute function "
                                 "followed by two ttl.datamovement functions")
            ordered = explicit
        ncores = int(np.prod(self.grid))
        core_traces = []
        for c in range(ncores):
            traced, errors, failed = [], [], []
            for t in ordered:
                try:
                    traced.append((t, self._trace_thread(t, c)))
                except Exception as e:  # noqa: BLE001 - re-raised below
                    root = getattr(e, "_ttlh_partial_root", None)
                    if root is None:
                        raise
                    failed.append(len(traced))
                    traced.append((t, root))
                    errors.append(e)
            if errors:
                # the simulator raises a thread's error only if that thread
                # gets there: when every thread blocks first (e.g. a store into
                # a waited block behind a wait nobody satisfies) the deadlock
                # is what it reports
                rep = P._deadlock_report({"core": c, "threads": traced}, failed)
                if rep is not None:
                    raise RuntimeError(rep) from None
                raise errors[0]
            core_traces.append({"core": c, "threads": traced})
        groups = P.resolve(core_traces)

        # tensors -> argument positions / names
        pos = {}
        for i, a in enumerate(args):
            pos.setdefault(id(a), i)
        for k, a in kwargs.items():
            pos.setdefault(id(a), k)

        made = {id(t): i for i, t in enumerate(created)}

        def tensor_ref(t):
            if id(t) in pos:
                return P.TensorRef(arg=pos[id(t)])
            if id(t) in made:
                return P.TensorRef(arg=("created", made[id(t)]), obj=t)
            return P.TensorRef(obj=t)

        plan = P.build_plan(groups, tensor_ref)
        plan.created = list(created)
        plan.uses_created = any(isinstance(r.arg, tuple) for r in _refs(plan))
        return plan

    def _created_tensors(self, *args, **kwargs) -> List[Any]:
        """Runs the kernel body again (no thread tracing) and returns the
        tensors it creates, in creation order."""
        g = dict(self.func.__globals__)
        g["grid"] = self.grid
        body = types.FunctionType(self.func.__code__, g, self.func.__name__,
                                  self.func.__defaults__, self.func.__closure__)
        prev = dsl._kstate
        dsl._kstate = dsl._KernelState(self.grid)
        prev_created, ttnn._created = ttnn._created, []
        try:
            body(*args, **kwargs)
            return ttnn._created
        finally:
            dsl._kstate = prev
            ttnn._created = prev_created

    def _trace_thread(self, t: dsl.ThreadTemplate, core: int):
        fn = t.rewritten()
        fn.__globals__["print"] = _trace_print
        first_err = None
        for scalar in (False, True):
            ctx = T.TraceContext(core, self.grid, t, scalar=scalar)
            prev = T._ctx
            T._ctx = ctx
            try:
                fn()
            except T.Devectorize:
                if scalar:
                    raise
                continue
            except Exception as e:
                if not scalar:
                    # a vectorised trace holds every iteration of the loops
                    # around the error; trace again with scalar loops so the
                    # operations before it are those of the simulator's run,
                    # which stops in the first iteration that fails
                    first_err = e
                    continue
                e._ttlh_partial_root = ctx.root  # the operations traced up to the error
                raise
            finally:
                T._ctx = prev
            if first_err is not None:  # the scalar run got through: keep the first error
                raise first_err
            if ctx.pending_reserve or ctx.pending_wait:
                err = RuntimeError(f"thread {t.__name__} on core {core} ended with a reserved or "
                                   "waited block that was never pushed / popped")
                err._ttlh_partial_root = ctx.root
                raise err
            return ctx.root
        raise AssertionError("unreachable")

    # -- call ------------------------------------------------------------------
    def __call__(self, *args, **kwargs):
        key = self._cache_key(args, kwargs)
        plan = self._cache.get(key)
        created = None
        if plan is None:
            plan = self.trace(*args, **kwargs)
            self._cache[key] = plan
            created = plan.created
        elif plan.uses_created:
            created = self._created_tensors(*args, **kwargs)
            if len(created) != len(plan.created):
                raise RuntimeError("the kernel body created a different number of tensors than "
                                   "when it was traced; cannot reuse the cached plan")
        self.last_plan = plan
        amap: Dict[Any, Any] = dict(enumerate(args))
        amap.update(kwargs)
        if created is not None:
            amap.update({("created", i): t for i, t in enumerate(created)})
        if profile.enabled():
            events: List[Any] = []
            P.execute(plan, amap, events=events)
            torch.cuda.synchronize()
            times = [a.elapsed_time(b) * 1e3 for a, b in events]
            print(profile.report(self.func.__name__, self.grid, plan, amap, times), flush=True)
            return None
        P.execute(plan, amap)
        if self.sync:
            torch.cuda.synchronize()
        return None
