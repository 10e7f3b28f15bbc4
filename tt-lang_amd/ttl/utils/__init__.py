"""`ttl.utils`: the reference installs its python/utils package here
(imported as ttl.utils.block_allocation by its hardware tests and metal
examples).  This package is that same module under a second name: the
import system finds `ttl.utils.block_allocation` in sys.modules."""

import sys as _sys

import utils.block_allocation as block_allocation

_sys.modules[__name__ + ".block_allocation"] = block_allocation
