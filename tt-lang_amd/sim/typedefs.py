"""Type names scripts import from the reference simulator's `sim.typedefs`
(python/sim/typedefs.py): the pipe and core-coordinate types, bound to this
build's `ttl`."""

from ttl import CoreCoord, CoreRange, DstPipeIdentity, Pipe, SrcPipeIdentity  # noqa: F401

Shape = tuple
Size = int
Index = int
