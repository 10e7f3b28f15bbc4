"""Drop-in `ttl` for tt-lang kernels on one MI355X (gfx950).

Same names as the reference's `ttl` namespace (python/sim/__init__.py:32-66,
python/ttl/__init__.py:10-50): kernel, grid_size, core, compute,
datamovement, make_circular_buffer_like, copy, TILE_SHAPE, math.broadcast and
the elementwise math ops, signpost.  Kernels written against the reference run
unchanged; their tile programs execute as HIP kernels (tt-lang_amd/csrc).
"""

from ttlhip.dsl import (  # noqa: F401
    MAX_CBS,
    Program,
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


class _Unsupported:
    def __init__(self, name: str):
        self._name = name

    def __call__(self, *a, **k):
        raise NotImplementedError(f"ttl.{self._name} (core-to-core pipes) is not supported by the "
                                  "MI355X backend")


Pipe = _Unsupported("Pipe")
PipeNet = _Unsupported("PipeNet")
SrcPipeIdentity = _Unsupported("SrcPipeIdentity")
DstPipeIdentity = _Unsupported("DstPipeIdentity")
