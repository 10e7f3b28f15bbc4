"""ttlhip: the MI355X (gfx950) runtime behind the drop-in `ttl` / `ttnn` modules.

Layers:
  _lib     ctypes binding of libttlhip.so (C ABI: include/ttlhip.h)
  expr     elementwise tile-expression IR and stack-program compiler
  kernels  torch-tensor wrappers of the C entry points
  trace    vectorised tracer of @ttl.kernel thread bodies
  plan     tile-program extraction: CB dataflow -> kernel launches
"""

from . import _lib  # noqa: F401
