"""pytest plugin that runs tt-lang's own hardware test files against this
build (test infrastructure).

Loaded with `-p refsuite_plugin --noconftest` in a child pytest: the
launcher's module injection (ttlang_hip.install: the drop-in `ttl`, `ttnn`,
`sim`, `utils`, `ttlang_test_utils` in sys.modules, as the reference's
ttlang-sim does for its simulator) runs first, the `device` fixture opens
the drop-in device, and every kernel call is traced and planned by the
drop-in, then executed by the CPU plan interpreter (`plan_interp`), so the
test's own torch golden and tolerance judge the tracer + planner without a
GPU.  At the end, any module imported from the reference tree other than the
test file or script being run fails the run (exit status 3): the results
must come from this build.  Nothing is written next to the test files: no
bytecode, no cache.
"""

import os
import sys
import types

sys.dont_write_bytecode = True
_HERE = os.path.dirname(os.path.abspath(__file__))
_ROOT = os.path.dirname(_HERE)
for _p in (_HERE, _ROOT, os.path.join(_ROOT, "tt-lang_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import pytest  # noqa: E402

import ttlang_hip  # noqa: E402

ttlang_hip.install()

REFERENCE = "/root/reference"


def foreign_modules(allowed=()):
    """Modules loaded from the reference tree, other than the files in
    `allowed` (the test file or script being run)."""
    allowed = {os.path.abspath(a) for a in allowed}
    bad = []
    for name, m in list(sys.modules.items()):
        f = getattr(m, "__file__", None) or ""
        if f and os.path.abspath(f).startswith(REFERENCE + os.sep) and os.path.abspath(f) not in allowed:
            bad.append(f"{name} ({f})")
    return bad

# the hardware tests import their conftest's list of generated kernel files
_conftest = types.ModuleType("conftest")
_conftest.temp_kernel_files = []
sys.modules.setdefault("conftest", _conftest)


def install_cpu_exec():
    """Kernel calls trace + plan on the drop-in and run on the CPU plan
    interpreter; the drop-in ttnn's elementwise ops run on its CPU stand-in
    of the eltwise launch."""
    import plan_interp
    from ttlhip import _lib, kernels, runner

    def call(self, *args):
        plan = self.trace(*args)
        plan_interp.run(plan, {i: a for i, a in enumerate(args)})
    runner.KernelRunner.__call__ = call
    kernels.eltwise = plan_interp.eltwise_cpu
    _lib.require_device = lambda: None


def pytest_configure(config):
    config.addinivalue_line("markers", "requires_device: runs on the drop-in device")
    install_cpu_exec()


def pytest_sessionfinish(session, exitstatus):
    bad = foreign_modules(str(item.fspath) for item in session.items)
    if bad:
        print("refsuite_plugin: reference modules imported: " + ", ".join(bad), file=sys.stderr)
        session.exitstatus = 3


def pytest_unconfigure(config):
    for path in _conftest.temp_kernel_files:
        try:
            os.unlink(path)
        except OSError:
            pass


@pytest.fixture
def ttnn_device():
    import ttnn

    dev = ttnn.open_device(device_id=0)
    yield dev
    ttnn.close_device(dev)


@pytest.fixture
def device(ttnn_device):
    return ttnn_device


if __name__ == "__main__":
    # `python refsuite_plugin.py script.py`: run one of the lit-style script
    # tests (kernel + driver code at module level) the same way
    import runpy

    install_cpu_exec()
    script = os.path.abspath(sys.argv[1])
    sys.argv = sys.argv[1:]
    try:
        runpy.run_path(script, run_name="__main__")
    finally:
        bad = foreign_modules([script])
        if bad:
            print("refsuite_plugin: reference modules imported: " + ", ".join(bad),
                  file=sys.stderr)
            sys.exit(3)
