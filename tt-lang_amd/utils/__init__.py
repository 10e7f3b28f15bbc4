"""Drop-in `utils` for tt-lang programs: the tolerance helpers
(`utils.correctness`) and the work-split helper (`utils.block_allocation`)
that the reference's example scripts import (python/utils/)."""
