"""Drop-in for the reference simulator package's public names a tt-lang
script imports: `from sim import ttl, ttnn` (python/sim/__init__.py:9,66),
`sim.testing`, `sim.typedefs`.  `ttl` and `ttnn` are this backend's modules;
a script that resolves them from another tree is refused here rather than
silently run on that tree."""

import os as _os

import ttl  # noqa: F401
import ttnn  # noqa: F401

_PKG = _os.path.dirname(_os.path.dirname(_os.path.abspath(__file__)))
for _m in (ttl, ttnn):
    if not _os.path.abspath(_m.__file__).startswith(_PKG + _os.sep):
        raise ImportError(f"sim: {_m.__name__} resolved to {_m.__file__}, not this backend "
                          f"({_PKG}); run the script through ttlang_hip.py")
