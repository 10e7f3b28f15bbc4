#!/usr/bin/env python3
"""ttlang-hip: run an unmodified tt-lang script on the MI355X backend.

Like the reference's ttlang-sim launcher (python/sim/ttlang_sim.py:22-69,
bin/ttlang-sim:10-13) it first installs this package's modules in
`sys.modules` (`ttl`, `ttnn`, `sim` with `sim.ttl` / `sim.ttnn`,
`sim.testing`, `sim.typedefs`, `utils`, `utils.correctness`,
`utils.block_allocation`, `ttlang_test_utils`), then executes the script as
__main__ with the script's directory on the import path.  Because the
modules are already imported, a script that puts another tree first on
sys.path and then does `import ttl` or `from sim import ttl, ttnn`
(examples/broadcast_demo.py:16-20) still binds to this backend.

    python tt-lang_amd/ttlang_hip.py examples/eltwise_add.py [args...]
    python tt-lang_amd/ttlang_hip.py -m package.module [args...]
"""

import importlib
import os
import runpy
import sys

PKG = os.path.dirname(os.path.abspath(__file__))

# the modules a tt-lang script may import, in dependency order
MODULES = ("ttnn", "ttl", "sim", "sim.testing", "sim.typedefs", "utils", "utils.correctness",
           "utils.block_allocation", "ttl.utils", "ttl.utils.block_allocation",
           "ttlang_test_utils")


def _ours(mod) -> bool:
    f = getattr(mod, "__file__", None) or ""
    return os.path.abspath(f).startswith(PKG + os.sep)


def install() -> None:
    """Puts this backend's modules in sys.modules (idempotent).  Modules of
    the same names imported earlier from another tree are dropped first;
    raises ImportError if a name still resolves outside this package."""
    if PKG in sys.path:
        sys.path.remove(PKG)
    sys.path.insert(0, PKG)
    roots = {m.split(".")[0] for m in MODULES}
    for name in list(sys.modules):
        if name.split(".")[0] in roots and not _ours(sys.modules[name]):
            del sys.modules[name]
    for name in MODULES:
        mod = importlib.import_module(name)
        if not _ours(mod):
            raise ImportError(f"ttlang-hip: module {name!r} resolved to {mod.__file__}, "
                              f"outside {PKG}")
    sim = sys.modules["sim"]
    sim.ttl = sys.modules["ttl"]
    sim.ttnn = sys.modules["ttnn"]


def run_file(path: str, argv) -> None:
    """Executes `path` as __main__ (the script's directory first on sys.path,
    as ttlang_sim.run_file does)."""
    if not os.path.exists(path):
        print(f"Error: File not found: {path}", file=sys.stderr)
        sys.exit(1)
    sys.path.insert(0, os.path.dirname(os.path.abspath(path)))
    sys.argv = [path] + list(argv)
    runpy.run_path(path, run_name="__main__")


def run_module(name: str, argv) -> None:
    sys.argv = [name] + list(argv)
    runpy.run_module(name, run_name="__main__", alter_sys=True)


def main(argv=None) -> int:
    argv = list(sys.argv[1:] if argv is None else argv)
    if not argv or argv[0] in ("-h", "--help"):
        print(__doc__)
        return 2
    install()
    if argv[0] == "-m":
        if len(argv) < 2:
            print(__doc__)
            return 2
        run_module(argv[1], argv[2:])
    else:
        run_file(argv[0], argv[1:])
    return 0


if __name__ == "__main__":
    sys.exit(main())
