"""Drop-in `ttl` for tt-lang kernels on one MI355X (gfx950).

Same names as the reference's `ttl` namespace (python/sim/__init__.py:32-66,
python/ttl/__init__.py:10-50): kernel, grid_size, core, compute,
datamovement, make_circular_buffer_like, copy, Program, Pipe / PipeNet,
TILE_SHAPE, math.broadcast and the elementwise math ops, signpost.  Kernels
written against the reference run unchanged; their tile programs execute as
HIP kernels (tt-lang_amd/csrc).
"""

from ttlhip.dsl import (  # noqa: F401
    MAX_CBS,
    DstPipeIdentity,
    Pipe,
    PipeNet,
    Program,
    SrcPipeIdentity,
    TILE_SHAPE,
    Block,
    CircularBuffer,
    CopyTransaction,
    compute,
    copy,
    core,
    datamovement,
    flatten_core_index,
    grid_size,
    kernel,
    make_circular_buffer_like,
    math,
    signpost,
)

from ttnn import CoreCoord, CoreRange  # noqa: F401,E402

Shape = tuple
Size = int

# `from ttl import ttl` (the compiler package's python/ttl/ttl.py namespace
# module, used by its hardware tests) names this same namespace
import sys as _sys  # noqa: E402

ttl = _sys.modules[__name__]
