"""The reference's hardware test suite (test/python of tt-lang), unmodified,
against this build's drop-in `ttl` / `ttnn` / `ttlang_test_utils`.

Each pytest-style file runs in a child pytest with `refsuite_plugin` (the
`device` fixture, kernel calls traced and planned by the drop-in and executed
by the CPU plan interpreter); the lit-style scripts run as programs and must
print their PASS line.  The tests' own torch goldens and tolerances judge the
results, so this checks the front end (tracer, planner, broadcast and CB
semantics) against the reference's expectations for its compiled path.  The
kernels the plans launch on the GPU are covered by the GPU tests.  The runner
installs the drop-in modules the way the launcher does and fails a run that
imported any module of the reference tree besides the file under test.  Nothing is
written under the reference tree (no bytecode, no pytest cache).
"""

import os
import re
import subprocess
import sys

import pytest

SUITE = "/root/reference/test/python"
HERE = os.path.dirname(os.path.abspath(__file__))

needs_ref = pytest.mark.skipif(not os.path.isdir(SUITE), reason="reference tree not present")

# file -> number of tests it holds (all must pass)
PYTEST_FILES = {
    "test_adversarial_multicore.py": 1,
    "test_axby.py": 1,
    "test_bcast_multicore.py": 1,
    "test_bcast_ops.py": 15,
    "test_bcast_shape_expansion.py": 6,
    "test_block_allocation.py": 33,
    "test_comprehensive_multicore.py": 1,
    "test_dst_multi_consumer.py": 5,
    "test_elementwise_ops.py": 13,
    "test_elementwise_shapes.py": 208,
    "test_grid_auto.py": 1,
    "test_intermediate_cb.py": 1,
    "test_multicore.py": 49,
    "test_sanity.py": 3,
    "test_tensor_slice.py": 241,
    "test_uneven_grids.py": 14,
}
# lit-style scripts that check their result and print PASS
SCRIPT_FILES = ["test_ttnn_interop_add.py", "test_dram_interleaved_add.py",
                "test_large_dram_streaming.py", "many_fused_ops.py", "simple_bcast.py",
                "mixed_l1_dram.py", "program_cache_lit.py"]
# lit-style compile checks (their FileCheck patterns are MLIR / C++ of the
# reference compiler): the kernels must trace, plan and run cleanly
CLEAN_FILES = ["simple_add.py", "simple_add_dram.py", "simple_add_f32.py",
               "simple_add_loop.py", "simple_add_multitile.py", "simple_add_with_stmt.py",
               "simple_fused.py", "simple_multicore.py", "debug_locations.py",
               "auto_profile_signposts.py"]


def _env():
    env = dict(os.environ)
    env["PYTHONDONTWRITEBYTECODE"] = "1"
    env["PYTHONPATH"] = HERE + os.pathsep + env.get("PYTHONPATH", "")
    return env


@needs_ref
@pytest.mark.parametrize("name", sorted(PYTEST_FILES))
def test_reference_pytest_file(name, tmp_path):
    cmd = [sys.executable, "-m", "pytest", "--noconftest", "-p", "refsuite_plugin",
           "-p", "no:cacheprovider", "-c", os.devnull, "--rootdir", str(tmp_path), "-q",
           os.path.join(SUITE, name)]
    r = subprocess.run(cmd, cwd=tmp_path, env=_env(), capture_output=True, text=True,
                       timeout=600)
    tail = r.stdout[-3000:] + r.stderr[-2000:]
    assert r.returncode == 0, tail
    m = re.search(r"(\d+) passed", r.stdout)
    assert m and int(m.group(1)) == PYTEST_FILES[name], tail
    assert "failed" not in r.stdout.splitlines()[-1], tail


@needs_ref
@pytest.mark.parametrize("name", SCRIPT_FILES)
def test_reference_script(name, tmp_path):
    cmd = [sys.executable, os.path.join(HERE, "refsuite_plugin.py"), os.path.join(SUITE, name)]
    r = subprocess.run(cmd, cwd=tmp_path, env=_env(), capture_output=True, text=True,
                       timeout=600)
    tail = r.stdout[-3000:] + r.stderr[-2000:]
    assert r.returncode == 0, tail
    assert "PASS" in r.stdout and "FAIL" not in r.stdout, tail


@needs_ref
@pytest.mark.parametrize("name", CLEAN_FILES)
def test_reference_compile_script_runs(name, tmp_path):
    cmd = [sys.executable, os.path.join(HERE, "refsuite_plugin.py"), os.path.join(SUITE, name)]
    r = subprocess.run(cmd, cwd=tmp_path, env=_env(), capture_output=True, text=True,
                       timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-2000:]


EXAMPLES = "/root/reference/examples"


def _run_example(name, tmp_path):
    cmd = [sys.executable, os.path.join(HERE, "refsuite_plugin.py"), os.path.join(EXAMPLES, name)]
    return subprocess.run(cmd, cwd=tmp_path, env=_env(), capture_output=True, text=True,
                          timeout=600)


@needs_ref
def test_reference_error_examples(tmp_path):
    # the simulator's errors for the reference's two broken examples
    # (test/sim/test_examples.py:125-193): the copy lock error (not a
    # deadlock: the failing thread reaches its error before anything blocks)
    # and the block / slice shape mismatch with its source line
    r = _run_example("copy_lock_error.py", tmp_path)
    assert r.returncode != 0 and "reference modules imported" not in r.stderr
    assert "locked as copy destination until tx.wait() completes (copy lock error)" in r.stderr
    assert "Deadlock" not in r.stderr
    r = _run_example("eltwise_add_error.py", tmp_path)
    assert r.returncode != 0 and "reference modules imported" not in r.stderr
    assert ("Tensor shape (32, 32) (=(1, 1) tiles) does not match Block shape (2, 2) tiles"
            in r.stderr)
    assert 'eltwise_add_error.py", line 37' in r.stderr
