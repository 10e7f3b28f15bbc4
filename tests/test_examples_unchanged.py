"""The north-star examples, unmodified, through this build's drop-in.

1. The launcher's module injection (tt-lang_amd/ttlang_hip.py, after the
   reference's python/sim/ttlang_sim.py:22-34): with the drop-in modules in
   sys.modules, a script that puts another tree first on sys.path and then
   does `from sim import ttl, ttnn` still binds to this build.
2. examples/eltwise_add.py, broadcast.py, singlecore_matmul.py,
   multicore_matmul.py and broadcast_demo.py run whole (their own main() /
   module-level driver and golden check decide) with kernel calls traced and
   planned by the drop-in and executed by the CPU plan interpreter; the
   runner fails the run if any module from the reference tree other than
   the script itself was imported.
3. Each unmodified example kernel plans to exactly the launches (stack
   program, operand maps, regions, argument bindings) of the restatement in
   tests/kernel_lib.py that the GPU tests run on the MI355X at the same
   shapes, so those GPU parity results carry over to the unmodified files.
"""

import os
import subprocess
import sys

import pytest
import torch

import kernel_lib as KL
import ttl
import ttnn
from ttlhip import plan as P

REF = "/root/reference/examples"
HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(os.path.dirname(HERE), "tt-lang_amd")
needs_ref = pytest.mark.skipif(not os.path.isdir(REF), reason="reference tree not present")


def _env():
    env = dict(os.environ)
    env["PYTHONDONTWRITEBYTECODE"] = "1"
    env["PYTHONPATH"] = HERE + os.pathsep + env.get("PYTHONPATH", "")
    return env


def test_launcher_injection_beats_a_prepended_tree(tmp_path):
    # a decoy tree with its own sim / ttl / ttnn, put first on sys.path by the
    # script (as broadcast_demo.py does with ../python): importing any of its
    # modules fails the run
    decoy = tmp_path / "decoy"
    for name in ("sim", "ttl", "ttnn", "utils"):
        (decoy / name).mkdir(parents=True)
        (decoy / name / "__init__.py").write_text("raise RuntimeError('decoy imported')\n")
    script = tmp_path / "script.py"
    script.write_text(
        "import sys\n"
        f"sys.path.insert(0, {str(decoy)!r})\n"
        "from sim import ttl, ttnn\n"
        "import ttl as ttl2, ttnn as ttnn2, sim.testing, sim.typedefs\n"
        "from utils.correctness import assert_allclose\n"
        "assert ttl is ttl2 and ttnn is ttnn2\n"
        "for m in (ttl, ttnn, sim.testing, sim.typedefs, sys.modules['utils.correctness']):\n"
        "    print(m.__file__)\n"
        "print('ARGV', sys.argv[1:])\n")
    r = subprocess.run([sys.executable, os.path.join(PKG, "ttlang_hip.py"), str(script), "x", "y"],
                       cwd=tmp_path, env=_env(), capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    files = [l for l in r.stdout.splitlines() if l.endswith(".py")]
    assert len(files) == 5 and all(f.startswith(PKG + os.sep) for f in files), r.stdout
    assert "ARGV ['x', 'y']" in r.stdout


def test_sim_package_refuses_a_foreign_ttl(tmp_path):
    # without the launcher, a `sim` import that would pair this package with
    # another tree's ttl fails loudly instead of running that tree
    other = tmp_path / "other"
    (other / "ttl").mkdir(parents=True)
    (other / "ttl" / "__init__.py").write_text("")
    code = (f"import sys; sys.path[:0] = [{str(other)!r}, {PKG!r}]\n"
            "try:\n    import sim\nexcept ImportError as e:\n    print('REFUSED', e)\n")
    r = subprocess.run([sys.executable, "-c", code], cwd=tmp_path, env=_env(),
                       capture_output=True, text=True, timeout=300)
    assert "REFUSED" in r.stdout, r.stdout + r.stderr[-2000:]


@needs_ref
@pytest.mark.parametrize("name,marker", [
    ("eltwise_add.py", None),
    ("broadcast.py", None),
    ("singlecore_matmul.py", "Matrix multiplication: (128, 256) @ (256, 64)"),
    ("multicore_matmul.py", "Grid: 8x8 = 64 cores"),
    ("broadcast_demo.py", "Result matches expected output"),
])
def test_example_runs_whole_unmodified(name, marker, tmp_path):
    cmd = [sys.executable, os.path.join(HERE, "refsuite_plugin.py"), os.path.join(REF, name)]
    r = subprocess.run(cmd, cwd=tmp_path, env=_env(), capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-3000:]
    assert "reference modules imported" not in r.stderr
    if marker:
        assert marker in r.stdout


# ---------------------------------------------------------------------------
# plan equality: unmodified example kernel vs. the GPU-tested restatement


def _ref_sig(r: P.TensorRef):
    if r.arg is not None:
        return ("arg", r.arg)
    return ("obj", type(r.obj).__name__, tuple(getattr(r.obj, "shape", ())))


def _spec_sig(s):
    if s is None:
        return None
    return (_ref_sig(s.ref), s.row_mask, s.col_mask, s.row_off, s.col_off)


def plan_signature(plan: P.Plan):
    """Everything a plan's launches do (not where in the source they came
    from): launch kinds, stack programs, operand maps, regions, bindings."""
    sig = []
    flat = []
    for l in plan.launches:
        flat += (l.reds + [l.ew]) if isinstance(l, P.ReduceEltwiseLaunch) else [l]
    for l in flat:
        if isinstance(l, (P.EltwiseLaunch, P.ReduceLaunch)):
            steps = [(s.op, s.form, s.rnd, s.imm, s.imm2) for s in l.prog.steps]
            item = [type(l).__name__, tuple(l.region), steps,
                    [_spec_sig(s) for s in l.operands], _ref_sig(l.out)]
            if isinstance(l, P.ReduceLaunch):
                item += [l.kind, tuple(l.dims), tuple(l.out_origin), l.out_pad,
                         None if l.scaler is None else _ref_sig(l.scaler), l.scaler_at, l.scale]
        else:
            item = ["MatmulLaunch", _ref_sig(l.a), _ref_sig(l.b), _ref_sig(l.c), tuple(l.rows),
                    tuple(l.cols), l.k, l.b_block]
        sig.append(item)
    return sig


def _load_example(name):
    path = os.path.join(REF, name)
    src = open(path).read().replace('if __name__ == "__main__":', "if False:")
    if name == "broadcast.py":  # module-level driver: keep the kernel definitions
        src = src.split("torch.manual_seed(42)")[0]
    g = {"__name__": "example"}
    exec(compile(src, path, "exec"), g)
    return g


def _t(shape, dtype):
    return ttnn.Tensor(torch.zeros(shape, dtype=dtype))


# (example file, kernel name, restatement factory + kwargs as the GPU tests
# call it, argument shapes / dtype at which the GPU tests run the restatement)
CASES = [
    ("eltwise_add.py", "eltwise_add", lambda: KL.make_eltwise_add(ttl),
     [(256, 256)] * 3, torch.float32),              # test_eltwise_add_kernel_bitexact
    ("eltwise_add.py", "eltwise_add", lambda: KL.make_eltwise_add(ttl),
     [(2048, 2048)] * 3, torch.bfloat16),           # test_eltwise_add_bf16_2048_config1
    ("broadcast.py", "__demo_kernel", lambda: KL.make_bcast_fma(ttl),
     [(2048, 2048), (2048, 2048), (2048, 1), (2048, 2048)], torch.bfloat16),
    # test_bcast_fma_example_config
    ("singlecore_matmul.py", "tt_lang_singlecore_matmul", lambda: KL.make_matmul_single(ttl),
     [(128, 256), (256, 64), (128, 64)], torch.float32),  # test_matmul_kernels_fp32_like_examples
    ("multicore_matmul.py", "tt_lang_multicore_matmul", lambda: KL.make_matmul_multi(ttl, ttnn),
     [(128, 256), (256, 64), (128, 64)], torch.float32),
]


@needs_ref
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[3][0][0]}")
def test_example_plan_equals_gpu_tested_restatement(case):
    name, fn, restated, shapes, dtype = case
    example = _load_example(name)[fn]
    pe = example.trace(*[_t(s, dtype) for s in shapes])
    pr = restated().trace(*[_t(s, dtype) for s in shapes])
    assert len(pe.launches) >= 1
    assert plan_signature(pe) == plan_signature(pr)
