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

from . import dsl
from . import plan as P
from . import trace as T


def _trace_print(*args, **kwargs):
    """Thread bodies run at trace time (once per core, loops vectorised);
    their prints are shown only with TTLH_TRACE_PRINT=1."""
    if os.environ.get("TTLH_TRACE_PRINT") == "1":
        print(*args, **kwargs)


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
        return (tuple(self._key_of(a) for a in args),
                tuple(sorted((k, self._key_of(v)) for k, v in kwargs.items())))

    # -- tracing ---------------------------------------------------------------
    def trace(self, *args, **kwargs) -> P.Plan:
        """Runs the kernel body and traces every core; returns the plan (no GPU)."""
        g = dict(self.func.__globals__)
        g["grid"] = self.grid
        body = types.FunctionType(self.func.__code__, g, self.func.__name__,
                                  self.func.__defaults__, self.func.__closure__)
        prev = dsl._kstate
        dsl._kstate = dsl._KernelState(self.grid)
        try:
            body(*args, **kwargs)
            threads = list(dsl._kstate.threads)
            explicit = dsl._kstate.program_order
        finally:
            dsl._kstate = prev
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
            traced = []
            for t in ordered:
                traced.append((t, self._trace_thread(t, c)))
            core_traces.append({"core": c, "threads": traced})
        groups = P.resolve(core_traces)

        # tensors -> argument positions / names
        pos = {}
        for i, a in enumerate(args):
            pos.setdefault(id(a), i)
        for k, a in kwargs.items():
            pos.setdefault(id(a), k)

        def tensor_ref(t):
            if id(t) in pos:
                return P.TensorRef(arg=pos[id(t)])
            return P.TensorRef(obj=t)

        return P.build_plan(groups, tensor_ref)

    def _trace_thread(self, t: dsl.ThreadTemplate, core: int):
        fn = t.rewritten()
        fn.__globals__["print"] = _trace_print
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
            finally:
                T._ctx = prev
            if ctx.pending_reserve or ctx.pending_wait:
                raise RuntimeError(f"thread {t.__name__} on core {core} ended with a reserved or "
                                   "waited block that was never pushed / popped")
            return ctx.root
        raise AssertionError("unreachable")

    # -- call ------------------------------------------------------------------
    def __call__(self, *args, **kwargs):
        key = self._cache_key(args, kwargs)
        plan = self._cache.get(key)
        if plan is None:
            plan = self.trace(*args, **kwargs)
            self._cache[key] = plan
        self.last_plan = plan
        amap: Dict[Any, Any] = dict(enumerate(args))
        amap.update(kwargs)
        P.execute(plan, amap)
        if self.sync:
            torch.cuda.synchronize()
        return None
