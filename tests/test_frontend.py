"""CPU tests of the drop-in front-end: tracing, planning, DSL rules.

Each kernel of kernel_lib is traced by this build's `ttl` (no GPU needed: the
plan is built, not launched), the plan is executed by the CPU plan
interpreter, and the result is compared with the oracle's eager tile-by-tile
executor running the same kernel source.  This checks the tracer's
vectorised index arithmetic, the CB FIFO matching and the launch
classification end to end.
"""

import math
import traceback
import os

import numpy as np
import pytest
import torch

import kernel_lib as KL
import plan_interp
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O
from ttlhip import plan as P
from ttlhip import trace as T

REF = "/root/reference/examples"


def _tt(t):
    return ttnn.Tensor(t.clone())


def _run_both(factory, tensors, out_index, **kw):
    """Returns (front-end result via CPU plan interpreter, oracle result, plan)."""
    k = factory(ttl, **kw) if "ttnn" not in factory.__code__.co_varnames else factory(ttl, ttnn, **kw)
    args = [_tt(t) for t in tensors]
    plan = k.trace(*args)
    plan_interp.run(plan, {i: a for i, a in enumerate(args)})
    ons = sim_exec.make_ttl()
    ko = factory(ons, **kw) if "ttnn" not in factory.__code__.co_varnames else factory(ons, ttnn, **kw)
    oargs = [sim_exec.OracleTensor(t.clone()) for t in tensors]
    ko(*oargs)
    return args[out_index]._tensor, oargs[out_index].t, plan


def test_eltwise_add_plan_and_parity():
    a = O.seeded((128, 256), "uniform", 1, torch.float32, lo=0, hi=1)
    b = O.seeded((128, 256), "uniform", 2, torch.float32, lo=0, hi=1)
    got, ref, plan = _run_both(KL.make_eltwise_add, [a, b, torch.zeros(128, 256)], 2)
    assert len(plan.launches) == 1 and isinstance(plan.launches[0], P.EltwiseLaunch)
    assert plan.launches[0].region == (0, 0, 128, 256)
    assert torch.equal(got, ref)
    assert torch.equal(ref, a + b)


def test_bcast_fma_column_vector():
    n = 256
    a, b = (O.seeded((n, n), "uniform", s) for s in (3, 4))
    c = O.seeded((n, 1), "uniform", 5)
    got, ref, plan = _run_both(KL.make_bcast_fma, [a, b, c, torch.zeros(n, n, dtype=torch.bfloat16)],
                               3, g=2, grid=(2, 2))
    (l,) = plan.launches
    spec_c = [s for s in l.operands if s is not None and s.ref.arg == 2][0]
    assert spec_c.col_mask == 31  # size-1 column broadcast across tiles
    assert torch.equal(got, ref)
    assert torch.equal(ref, a * b + c)  # per-op bf16 rounding == torch bf16 ops


def test_outer_fma_three_arg_broadcast():
    n = 256
    a, b, c = O.seeded((n, 1), "uniform", 6), O.seeded((1, n), "uniform", 7), O.seeded((1, 1), "uniform", 8)
    got, ref, plan = _run_both(KL.make_outer_fma, [a, b, c, torch.zeros(n, n, dtype=torch.bfloat16)],
                               3, grid=(2, 2))
    assert len(plan.launches) == 1
    assert torch.equal(got, ref)
    assert torch.equal(ref, a * b + c)


@pytest.mark.parametrize("bshape,cshape", [((512, 512), (512, 1)), ((1, 512), (1, 1))])
def test_shape_dispatch_fma(bshape, cshape):
    n = 512
    a, b, c = O.seeded((n, n), "uniform", 9), O.seeded(bshape, "uniform", 10), O.seeded(cshape, "uniform", 11)
    got, ref, plan = _run_both(KL.make_shape_dispatch_fma,
                               [a, b, c, torch.zeros(n, n, dtype=torch.bfloat16)], 3)
    assert len(plan.launches) == 1
    assert torch.equal(got, ref)


def test_exp_row_pipe_config2_semantics():
    n = 256
    a, c = O.seeded((n, n), "uniform", 6, lo=-2, hi=2), O.seeded((n, n), "uniform", 7, lo=-2, hi=2)
    b = O.seeded((1, n), "uniform", 8, lo=-2, hi=2)
    got, ref, plan = _run_both(KL.make_exp_row_pipe,
                               [a, b, c, torch.zeros(n, n, dtype=torch.bfloat16)], 3, g=2,
                               grid=(2, 2))
    assert len(plan.launches) == 1
    assert int(O.bf16_ulp_diff(got, ref).max()) <= 1
    assert torch.equal(ref, torch.exp(a + b) * c)


@pytest.mark.parametrize("M,K,N", [(64, 96, 128), (128, 256, 64)])
def test_matmul_single_plan(M, K, N):
    a = O.seeded((M, K), "uniform", 9, torch.float32, lo=0, hi=1)
    b = O.seeded((K, N), "uniform", 10, torch.float32, lo=0, hi=1)
    got, ref, plan = _run_both(KL.make_matmul_single, [a, b, torch.zeros(M, N)], 2)
    (l,) = plan.launches
    assert isinstance(l, P.MatmulLaunch) and l.k == K and l.rows == (0, M) and l.cols == (0, N)
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-5)


def test_matmul_multi_split_work_plan():
    M, K, N = 128, 256, 96
    a = O.seeded((M, K), "uniform", 11, torch.float32, lo=0, hi=1)
    b = O.seeded((K, N), "uniform", 12, torch.float32, lo=0, hi=1)
    got, ref, plan = _run_both(KL.make_matmul_multi, [a, b, torch.zeros(M, N)], 2)
    (l,) = plan.launches
    assert isinstance(l, P.MatmulLaunch) and l.k == K
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-5)


def test_tile_reuse_mask_mode():
    a = O.seeded((256, 256), "uniform", 13)
    t = O.seeded((32, 32), "uniform", 14)
    got, ref, plan = _run_both(KL.make_tile_reuse, [a, t, torch.zeros(256, 256, dtype=torch.bfloat16)], 2)
    (l,) = plan.launches
    spec_t = [s for s in l.operands if s is not None and s.ref.arg == 1][0]
    assert (spec_t.row_mask, spec_t.col_mask) == (31, 31)
    assert torch.equal(got, ref)


def test_branch_on_loop_variable_falls_back_to_scalar_trace():
    a = O.seeded((64, 128), "uniform", 15)
    b = O.seeded((64, 128), "uniform", 16)
    got, ref, plan = _run_both(KL.make_branchy_add, [a, b, torch.zeros(64, 128, dtype=torch.bfloat16)], 2)
    assert len(plan.launches) == 1
    assert torch.equal(got, ref)


def test_large_matmul_traces_fast():
    import time
    k = KL.make_matmul_single(ttl)
    a, b, c = (ttnn.Tensor(torch.empty(s, dtype=torch.bfloat16)) for s in
               ((2048, 2048), (2048, 2048), (2048, 2048)))
    t0 = time.time()
    plan = k.trace(a, b, c)
    assert time.time() - t0 < 20.0  # 262,144 tile-steps, vectorised
    assert plan.launches[0].k == 2048


# ---------------------------------------------------------------------------
# vectorised integers and the loop rewrite


def test_vint_arithmetic_and_guards():
    v = T.VInt(np.arange(6).reshape(6, 1, 1, 1, 1, 1, 1, 1), frozenset([1]))
    w = (v * 3 + 2) // 4 % 5
    assert w.v.ravel().tolist() == [((i * 3 + 2) // 4) % 5 for i in range(6)]
    with pytest.raises(T.Devectorize):
        bool(v < 3)
    with pytest.raises(T.Devectorize):
        range(v)


def test_loop_carried_variables_are_not_vectorised():
    import ast
    src = "for i in range(4):\n    x = x + i\n"
    loop = ast.parse(src).body[0]
    assert not T._vectorisable_body(loop)
    src2 = "for i in range(4):\n    y = i * 2\n    z = y + 1\n"
    assert T._vectorisable_body(ast.parse(src2).body[0])
    src3 = "for i in range(4):\n    acc += i\n"
    assert not T._vectorisable_body(ast.parse(src3).body[0])


# ---------------------------------------------------------------------------
# DSL rules (messages follow the simulator's)


def _bad_kernel(nthreads):
    @ttl.kernel(grid=(1, 1))
    def k(a):
        cb = ttl.make_circular_buffer_like(a, shape=(1, 1))

        @ttl.compute()
        def c():
            pass

        for _ in range(nthreads - 1):
            @ttl.datamovement()
            def d():
                pass
    return k


def test_thread_count_validation():
    a = ttnn.Tensor(torch.zeros(32, 32))
    with pytest.raises(ValueError, match="exactly 3 threads"):
        _bad_kernel(2).trace(a)


def test_copy_shape_mismatch_is_rejected():
    @ttl.kernel(grid=(1, 1))
    def k(a, out):
        cb = ttl.make_circular_buffer_like(a, shape=(1, 1))

        @ttl.compute()
        def c():
            pass

        @ttl.datamovement()
        def r():
            with cb.reserve() as blk:
                ttl.copy(a[0:2, 0:1], blk).wait()

        @ttl.datamovement()
        def w():
            pass

    with pytest.raises(ValueError, match="does not match Block shape"):
        k.trace(ttnn.Tensor(torch.zeros(64, 32)), ttnn.Tensor(torch.zeros(64, 32)))


def _copy_lock_kernel(mistake):
    @ttl.kernel(grid=(1, 1))
    def k(a, out):
        a_cb = ttl.make_circular_buffer_like(a, shape=(1, 1))
        o_cb = ttl.make_circular_buffer_like(out, shape=(1, 1))

        @ttl.compute()
        def c():
            with a_cb.wait() as ab, o_cb.reserve() as ob:
                ob.store(ab)

        @ttl.datamovement()
        def r():
            blk = a_cb.reserve()
            tx = ttl.copy(a[0, 0], blk)
            if mistake == "store":
                blk.store(blk)  # written before tx.wait() (examples/copy_lock_error.py:86-88)
            elif mistake == "push":
                a_cb.push()  # pushed before tx.wait()
            elif mistake == "copy":
                ttl.copy(a[0, 0], blk)  # second copy into a locked block
            tx.wait()
            a_cb.push()

        @ttl.datamovement()
        def w():
            with o_cb.wait() as ob:
                tx = ttl.copy(ob, out[0, 0])
                if mistake == "pop":
                    o_cb.pop()  # popped while still the source of a copy
                tx.wait()
    return k


@pytest.mark.parametrize("mistake,msg", [
    ("store", r"locked as copy destination until tx.wait\(\) completes \(copy lock error\)"),
    ("push", r"Cannot perform push\(\): Expected one of \[TX_WAIT\]"),
    ("copy", r"Cannot perform copy \(as destination\): Expected one of \[TX_WAIT\]"),
    ("pop", r"Cannot perform pop\(\): Expected one of \[TX_WAIT\]"),
])
def test_copy_lock_errors(mistake, msg):
    # simulator block state machine: a block is locked from copy() to tx.wait()
    # (python/sim/block.py:263-343, 656-694; test/sim/test_examples.py:160-190)
    a = ttnn.Tensor(torch.zeros(32, 32))
    with pytest.raises(RuntimeError, match=msg) as ei:
        _copy_lock_kernel(mistake).trace(a, ttnn.Tensor(torch.zeros(32, 32)))
    # the traceback names the offending line of the kernel source
    here = [f for f in traceback.extract_tb(ei.tb) if f.filename == __file__]
    assert here and {"store": "blk.store", "push": "a_cb.push()", "copy": "ttl.copy(a[0, 0], blk)",
                     "pop": "o_cb.pop()"}[mistake] in here[-1].line


def test_copy_lock_released_by_wait():
    a = ttnn.Tensor(torch.zeros(32, 32))
    plan = _copy_lock_kernel(None).trace(a, ttnn.Tensor(torch.zeros(32, 32)))
    assert len(plan.launches) == 1


def test_unbalanced_cb_is_reported_as_deadlock():
    @ttl.kernel(grid=(1, 1))
    def k(a, out):
        cb = ttl.make_circular_buffer_like(a, shape=(1, 1))
        ocb = ttl.make_circular_buffer_like(out, shape=(1, 1))

        @ttl.compute()
        def c():
            for _ in range(2):
                with cb.wait() as x, ocb.reserve() as o:
                    o.store(x)

        @ttl.datamovement()
        def r():
            with cb.reserve() as blk:
                ttl.copy(a[0, 0], blk).wait()

        @ttl.datamovement()
        def w():
            for i in range(2):
                with ocb.wait() as o:
                    ttl.copy(o, out[i, 0]).wait()

    with pytest.raises(RuntimeError, match="Deadlock"):
        k.trace(ttnn.Tensor(torch.zeros(64, 32)), ttnn.Tensor(torch.zeros(64, 32)))


def test_broadcast_validation():
    @ttl.kernel(grid=(1, 1))
    def k(a, out):
        cb = ttl.make_circular_buffer_like(a, shape=(2, 2))
        ocb = ttl.make_circular_buffer_like(out, shape=(2, 2))

        @ttl.compute()
        def c():
            with cb.wait() as x, ocb.reserve() as o:
                o.store(ttl.math.broadcast(x, dims=[1]))

        @ttl.datamovement()
        def r():
            with cb.reserve() as blk:
                ttl.copy(a[0:2, 0:2], blk).wait()

        @ttl.datamovement()
        def w():
            with ocb.wait() as o:
                ttl.copy(o, out[0:2, 0:2]).wait()

    with pytest.raises(ValueError, match="dimension must have size 1"):
        k.trace(ttnn.Tensor(torch.zeros(64, 64)), ttnn.Tensor(torch.zeros(64, 64)))


def test_grid_size_and_core_semantics():
    # python/sim/kernel.py:89-199: flatten trailing / pad with 1s; row-major ids
    from ttlhip import dsl
    ctx = T.TraceContext(core=19, grid=(8, 8), thread=None, scalar=True)
    T._ctx = ctx
    try:
        assert dsl.grid_size(1) == 64
        assert dsl.grid_size(2) == (8, 8)
        assert dsl.grid_size(3) == (8, 8, 1)
        assert dsl.core(2) == (2, 3)
        assert dsl.core(1) == 19
        assert dsl.core(3) == (2, 3, 0)
    finally:
        T._ctx = None


def test_split_work_to_cores_assignment():
    n, allc, g1, g2, w1, w2 = ttnn.split_work_to_cores(ttnn.CoreCoord(10, 13), 16384, row_wise=True)
    assert (n, w1, w2, g1.num_cores(), g2.num_cores()) == (130, 127, 126, 4, 126)
    first = [(r.start.x, r.start.y) for r in g1.ranges()]
    assert first == [(0, 0), (1, 0), (2, 0), (3, 0)]
    assert ttnn.split_work_to_cores(ttnn.CoreCoord(8, 8), 0)[0] == 0


# ---------------------------------------------------------------------------
# the reference's own example kernels (read from /root/reference when present)


def _load_example(name):
    path = os.path.join(REF, name)
    src = open(path).read()
    src = src.replace('if __name__ == "__main__":', "if False:")
    if name == "broadcast.py":  # module-level driver code: keep the kernel definitions only
        src = src.split("torch.manual_seed(42)")[0]
    g = {"__name__": "example"}
    exec(compile(src, path, "exec"), g)
    return g


needs_ref = pytest.mark.skipif(not os.path.isdir(REF), reason="reference tree not present")


@needs_ref
def test_reference_example_eltwise_add_plans_one_launch():
    g = _load_example("eltwise_add.py")
    a, b, o = (ttnn.Tensor(torch.rand(256, 256)) for _ in range(3))
    plan = g["eltwise_add"].trace(a, b, o)
    assert len(plan.launches) == 1 and plan.launches[0].region == (0, 0, 256, 256)


@needs_ref
def test_reference_example_broadcast_plans_one_launch():
    g = _load_example("broadcast.py")
    k = g["__demo_kernel"]
    a, b = ttnn.Tensor(torch.rand(2048, 2048).bfloat16()), ttnn.Tensor(torch.rand(2048, 2048).bfloat16())
    c = ttnn.Tensor(torch.rand(2048, 1).bfloat16())
    y = ttnn.Tensor(torch.zeros(2048, 2048).bfloat16())
    plan = k.trace(a, b, c, y)
    assert len(plan.launches) == 1 and isinstance(plan.launches[0], P.EltwiseLaunch)


@needs_ref
@pytest.mark.parametrize("name,fn", [("singlecore_matmul.py", "tt_lang_singlecore_matmul"),
                                     ("multicore_matmul.py", "tt_lang_multicore_matmul")])
def test_reference_example_matmuls_plan_one_gemm(name, fn):
    g = _load_example(name)
    a, b, o = ttnn.Tensor(torch.rand(128, 256)), ttnn.Tensor(torch.rand(256, 64)), \
        ttnn.Tensor(torch.zeros(128, 64))
    plan = g[fn].trace(a, b, o)
    (l,) = plan.launches
    assert isinstance(l, P.MatmulLaunch) and l.k == 256


# The tutorials and general_broadcast.py: kernel definitions read from the
# reference tree (source cut before the driver code, which is re-stated here
# with smaller shapes), traced by the drop-in and executed by the CPU plan
# interpreter; results bit-exact against the oracle's per-op-rounded formula.

def _load_defs(path):
    src = open(os.path.join(REF, path)).read().split("torch.manual_seed(42)")[0]
    g = {"__name__": "example", "device": None}
    exec(compile(src, os.path.join(REF, path), "exec"), g)
    return g


@pytest.fixture
def cpu_exec(monkeypatch):
    """Kernel calls trace and run on the CPU plan interpreter (tests only)."""
    from ttlhip import runner

    def call(self, *args):
        plan = self.trace(*args)
        plan_interp.run(plan, {i: a for i, a in enumerate(args)})
        call.plans.append(plan)
    call.plans = []
    monkeypatch.setattr(runner.KernelRunner, "__call__", call)
    return call


def _bf(shape, seed):
    return O.seeded(shape, "uniform", seed, torch.bfloat16, lo=0, hi=1)


@needs_ref
@pytest.mark.parametrize("name,n,bcast", [
    ("tutorial/single_core_single_tile_block.py", 128, False),
    ("tutorial/single_core_multitile_block.py", 256, False),
    ("tutorial/single_core_broadcast_single_tile_block.py", 128, True),
    ("tutorial/single_core_broadcast_multitile_blocks.py", 256, True),
    ("tutorial/multicore.py", 512, False),
    ("tutorial/multicore_grid_auto.py", 1024, False),
])
def test_reference_tutorials(cpu_exec, name, n, bcast):
    g = _load_defs(name)
    if bcast:
        a, b, c = _bf((n, 1), 1), _bf((1, n), 2), _bf((1, 1), 3)
    else:
        a, b, c = _bf((n, n), 1), _bf((n, n), 2), _bf((n, n), 3)
    y = g["demo_kernel"](ttnn.from_torch(a), ttnn.from_torch(b), ttnn.from_torch(c))
    expect = O.eval_expr(("add", ("mul", ("leaf", "a"), ("leaf", "b")), ("leaf", "c")),
                         {"a": a, "b": b, "c": c})
    assert torch.equal(ttnn.to_torch(y), expect.expand(n, n))
    assert len(cpu_exec.plans[-1].launches) == 1


@needs_ref
def test_reference_deadlock_report(cpu_exec, tmp_path):
    # the reference's own deadlock check (test/sim/test_examples.py:194-300):
    # tutorial/multicore_grid_auto.py with the compute thread's y_cb.reserve()
    # turned into y_cb.wait() must report every blocked thread, its
    # operation, the CB and the source line of the blocking call
    import re
    src = open(os.path.join(REF, "tutorial/multicore_grid_auto.py")).read()
    bad = src.replace("y_cb.reserve() as y_blk,", "y_cb.wait() as y_blk,")
    assert bad != src
    path = tmp_path / "multicore_grid_auto_deadlock.py"
    path.write_text(bad)
    g = {"__name__": "example", "device": None}
    exec(compile(bad.split("torch.manual_seed(42)")[0], str(path), "exec"), g)
    n = 2048  # the script's own size: the reader fills a_cb before compute blocks
    with pytest.raises(RuntimeError) as ei:
        g["demo_kernel"](ttnn.from_torch(_bf((n, n), 1)), ttnn.from_torch(_bf((n, n), 2)),
                         ttnn.from_torch(_bf((n, n), 3)))
    out = str(ei.value)
    assert "Deadlock detected: all generators blocked" in out
    assert "CircularBuffer(y_cb)" in out
    assert "blocked on wait()" in out and "blocked on reserve()" in out
    for t in ("core0-compute:", "core0-dm0:", "core0-dm1:"):
        assert t in out
    lines = bad.splitlines()
    for thread, line in re.findall(r"core0-(\w+).*? at .*?:(\d+)", out):
        text = lines[int(line) - 1]
        assert (".wait()" if thread in ("compute", "dm1") else ".reserve()") in text, (thread, text)
    assert "y_cb.wait()" in lines[int(re.search(r"core0-compute.*?:(\d+)", out).group(1)) - 1]


@needs_ref
@pytest.mark.parametrize("bshape,cshape", [((1024, 1024), (1024, 1024)), ((1024, 1), (1, 1024)),
                                           ((1, 1024), (1, 1)), ((1, 1), (1024, 1))])
def test_reference_general_broadcast(cpu_exec, bshape, cshape):
    g = _load_defs("general_broadcast.py")
    a, b, c = _bf((1024, 1024), 4), _bf(bshape, 5), _bf(cshape, 6)
    y = ttnn.from_torch(torch.zeros(1024, 1024, dtype=torch.bfloat16))
    g["__demo_kernel"](ttnn.from_torch(a), ttnn.from_torch(b), ttnn.from_torch(c), y)
    expect = O.eval_expr(("add", ("mul", ("leaf", "a"), ("leaf", "b")), ("leaf", "c")),
                         {"a": a, "b": b, "c": c})
    assert torch.equal(ttnn.to_torch(y), expect)
