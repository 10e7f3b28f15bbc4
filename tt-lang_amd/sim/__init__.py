"""Drop-in for the reference simulator package's public names a tt-lang
script imports: `from sim import ttl, ttnn` (python/sim/__init__.py:9,66),
`sim.testing`, `sim.typedefs`.  `ttl` and `ttnn` are this backend's modules;
a script that resolves them from another tree is refused here rather than
silently run on that tree."""

import os as _os
import sys as _sys
import types as _types

import ttl  # noqa: F401
import ttnn  # noqa: F401

_PKG = _os.path.dirname(_os.path.dirname(_os.path.abspath(__file__)))
for _m in (ttl, ttnn):
    if not _os.path.abspath(_m.__file__).startswith(_PKG + _os.sep):
        raise ImportError(f"sim: {_m.__name__} resolved to {_m.__file__}, not this backend "
                          f"({_PKG}); run the script through ttlang_hip.py")

# `sim.typedefs` (python/sim/typedefs.py): the pipe and core-coordinate type
# names scripts import from it, bound to this build's `ttl`, plus the
# reference's shape / size / index aliases.
typedefs = _types.ModuleType(__name__ + ".typedefs", "sim.typedefs: ttl's pipe and core types")
for _n in ("CoreCoord", "CoreRange", "DstPipeIdentity", "Pipe", "SrcPipeIdentity"):
    setattr(typedefs, _n, getattr(ttl, _n))
typedefs.Shape, typedefs.Size, typedefs.Index = tuple, int, int
typedefs.__file__ = __file__  # defined here
_sys.modules[typedefs.__name__] = typedefs
