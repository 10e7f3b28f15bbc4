#!/usr/bin/env python3
"""ttlang-hip: run an unmodified tt-lang script on the MI355X backend.

Like the reference's ttlang-sim launcher (python/sim/ttlang_sim.py:22-69), it
puts this package's `ttl`, `ttnn` and `sim` first on the import path and then
executes the script as __main__.

    python tt-lang_amd/ttlang_hip.py examples/eltwise_add.py [args...]
"""

import os
import runpy
import sys

PKG = os.path.dirname(os.path.abspath(__file__))


def main(argv=None) -> int:
    argv = list(sys.argv[1:] if argv is None else argv)
    if not argv:
        print(__doc__)
        return 2
    script = argv[0]
    sys.path.insert(0, PKG)
    for name in ("ttl", "ttnn", "sim", "sim.testing"):
        sys.modules.pop(name, None)
    sys.argv = argv
    runpy.run_path(script, run_name="__main__")
    return 0


if __name__ == "__main__":
    sys.exit(main())
