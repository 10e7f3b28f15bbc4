"""The drop-in `utils` (tolerance helpers and work split the reference's
example scripts import, python/utils/) and the explicit `ttl.Program` form.

ulp() is pinned against torch.nextafter (the definition the reference uses,
correctness.py:142-165); the ULP / allclose / PCC assertions against hand
cases; split_work_to_cores against hand-derived assignments and the
work-conservation property.  The reference's metal-example tt-lang scripts
run unmodified through the drop-in on the CPU plan interpreter (skipped
without /root/reference).
"""

import math
import os
import sys

import pytest
import torch

import plan_interp
import ttl
import ttnn
from utils import block_allocation as BA
from utils import correctness as C

REF = "/root/reference/examples/metal_examples"
needs_ref = pytest.mark.skipif(not os.path.isdir(REF), reason="reference examples not present")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_ulp_matches_nextafter(dtype):
    fi = torch.finfo(dtype)
    g = torch.Generator().manual_seed(3)
    x = torch.cat([
        torch.randn(2000, generator=g) * 10.0 ** torch.randint(-6, 6, (2000,), generator=g),
        torch.tensor([0.0, 1.0, 2.0, 0.75, fi.tiny, fi.tiny / 8, -fi.tiny * 3, fi.max / 2]),
    ]).to(dtype)
    x = x[torch.isfinite(x)]
    ax = x.abs().to(torch.float64)
    nxt = torch.nextafter(x.abs().to(torch.float32), torch.tensor(math.inf)).to(torch.float64) \
        if dtype == torch.float32 else None
    got = C.ulp(x).to(torch.float64)
    if nxt is not None:
        assert torch.equal(got, nxt - ax)
    else:
        # 16-bit formats: the next value above |x| is |x| + ulp, and nothing
        # representable lies strictly between them
        up = (ax + got).to(dtype).to(torch.float64)
        mid = (ax + got / 2).to(dtype).to(torch.float64)
        assert torch.equal(up, ax + got)
        assert bool(((mid == ax) | (mid == ax + got)).all())
    # at the format maximum: the gap below it
    m = torch.tensor([fi.max], dtype=dtype)
    assert float(C.ulp(m)) == 2.0 ** (math.floor(math.log2(fi.max)) - {torch.float32: 23, torch.float16: 10, torch.bfloat16: 7}[dtype])


def test_comp_ulp_cases():
    g = torch.tensor([1.0, 2.0, -3.0, 0.5], dtype=torch.bfloat16)
    ok, msg = C.comp_ulp(g, g.clone(), 0)
    assert ok and "Max ULP Delta: 0" in msg
    one_up = g.to(torch.float32) + C.ulp(g).to(torch.float32)
    assert C.comp_ulp(g, one_up.to(torch.bfloat16), 1)[0]
    assert not C.comp_ulp(g, one_up.to(torch.bfloat16), 0.5)[0]
    # a float64 golden measures sub-ULP errors of a bf16 result
    ok, msg = C.comp_ulp(torch.tensor([1.0 + 2 ** -9], dtype=torch.float64),
                         torch.tensor([1.0], dtype=torch.bfloat16), 0.3)
    assert ok and "0.25" in msg
    nan = torch.tensor([1.0, float("nan")])
    assert C.comp_ulp(nan, nan.clone(), 0)[0]
    assert not C.comp_ulp(nan, torch.tensor([1.0, 1.0]), 1e9)[0]
    assert not C.comp_ulp(torch.tensor([math.inf]), torch.tensor([-math.inf]), 1e9)[0]
    assert not C.comp_ulp(nan, nan.clone(), 0, allow_nonfinite=False)[0]
    assert C.comp_ulp(torch.tensor([]), torch.tensor([]), 0) == (True, "Both tensors are empty")


def test_assertions_raise_with_reports():
    a = torch.linspace(-1, 1, 64)
    C.assert_with_ulp(a.bfloat16(), a.bfloat16())
    with pytest.raises(AssertionError, match="Max ULP Delta"):
        C.assert_with_ulp(a.bfloat16(), (a + 0.5).bfloat16())
    with pytest.raises(AssertionError, match="shape"):
        C.assert_with_ulp(a, a[:10])
    C.assert_allclose(a, a + 1e-9, rtol=1e-5, atol=1e-8)
    with pytest.raises(AssertionError, match="Mismatched elements: 64 / 64"):
        C.assert_allclose(a + 1.0, a)
    with pytest.raises(AssertionError, match="Shape mismatch"):
        C.assert_allclose(a, a[:3])
    C.assert_pcc(a, 2 * a + 1)
    with pytest.raises(AssertionError, match="Expected pcc"):
        C.assert_pcc(a, -a)


@pytest.mark.parametrize("grid,units,row_wise,expect", [
    # 640^3 tiles on the multicore example's 13 x 10 grid: 400 = 10 x 4 + 120 x 3
    ((13, 10), 400, True, (130, ((0, 0), (0, 9)), ((1, 0), (12, 9)), 4, 3)),
    # fewer units than cores: 6 full rows of 10, then 4 cores of row 6
    ((13, 10), 64, True, (64, ((0, 0), (6, 3)), (), 1, 0)),
    ((13, 10), 260, True, (130, ((0, 0), (12, 9)), (), 2, 0)),
    # column-wise fill: 7 extra units -> cores (0..6, 0), the rest from (7, 0)
    ((13, 10), 137, False, (130, ((0, 0), (6, 0)), ((7, 0), (12, 9)), 2, 1)),
    ((1, 8), 5, True, (5, ((0, 0), (0, 4)), (), 1, 0)),
    ((4, 4), 0, True, (0, (), (), 0, 0)),
])
def test_split_work_to_cores_known_answers(grid, units, row_wise, expect):
    assert BA.split_work_to_cores(grid, units, row_wise=row_wise) == expect


def test_split_work_conserves_units_on_full_rows():
    # whenever both groups are whole rows (x fastest), box sizes x units/core add up
    for ny, nx in ((13, 10), (8, 8), (3, 7)):
        for units in range(1, 5 * ny * nx):
            n, g1, g2, u1, u2 = BA.split_work_to_cores((ny, nx), units)
            boxes = [g for g in (g1, g2) if g]
            cnt = [(e[0] - s[0] + 1) * (e[1] - s[1] + 1) for s, e in boxes]
            full = all(s[1] == 0 and e[1] == nx - 1 for s, e in boxes)
            if full:
                assert sum(c * u for c, u in zip(cnt, (u1, u2))) == units
            assert n == min(units, ny * nx)


def test_split_rows_kernel_plans_one_gemm():
    import kernel_lib as KL
    a, b = torch.rand(640, 640).bfloat16(), torch.rand(640, 640).bfloat16()
    c = torch.zeros(640, 640, dtype=torch.bfloat16)
    plan = KL.make_matmul_split_rows(ttl).trace(ttnn.Tensor(a), ttnn.Tensor(b), ttnn.Tensor(c))
    assert len(plan.launches) == 1
    plan_interp.run(plan, {0: ttnn.Tensor(a), 1: ttnn.Tensor(b), 2: ttnn.Tensor(c)})
    C.assert_with_ulp(a @ b, c)


def test_program_explicit_thread_order():
    def make(order):
        @ttl.kernel(grid=(1, 1))
        def k(a, out):
            a_cb = ttl.make_circular_buffer_like(a, shape=(1, 1))
            o_cb = ttl.make_circular_buffer_like(out, shape=(1, 1))

            @ttl.compute()
            def comp():
                with a_cb.wait() as ab, o_cb.reserve() as ob:
                    ob.store(ab + ab)

            @ttl.datamovement()
            def rd():
                with a_cb.reserve() as ab:
                    ttl.copy(a[0, 0], ab).wait()

            @ttl.datamovement()
            def wr():
                with o_cb.wait() as ob:
                    ttl.copy(ob, out[0, 0]).wait()

            threads = {"c": comp, "r": rd, "w": wr}
            return ttl.Program(*[threads[x] for x in order], grid=grid)()
        return k

    a = torch.full((32, 32), 3.0)
    out = torch.zeros(32, 32)
    plan = make("crw").trace(ttnn.Tensor(a), ttnn.Tensor(out))
    plan_interp.run(plan, {0: ttnn.Tensor(a), 1: ttnn.Tensor(out)})
    assert torch.equal(out, torch.full((32, 32), 6.0))
    with pytest.raises(ValueError, match="compute, dm0, dm1"):
        make("rcw").trace(ttnn.Tensor(a), ttnn.Tensor(out))


@pytest.fixture
def cpu_exec(monkeypatch):
    from ttlhip import runner

    def call(self, *args):
        plan_interp.run(self.trace(*args), {i: x for i, x in enumerate(args)})
    monkeypatch.setattr(runner.KernelRunner, "__call__", call)


@needs_ref
@pytest.mark.parametrize("path,test,args", [
    ("singlecore_matmul/ttlang/singlecore_matmul.py", "test_singlecore_matmul_tt_lang", ()),
    ("multicore_matmul/ttlang/multicore_matmul.py", "test_multicore_matmul_tt_lang", (640, 640, 640)),
])
def test_reference_metal_ttlang_scripts_run_unmodified(cpu_exec, path, test, args):
    # the scripts' own test functions, with their own assert_with_ulp bar (10
    # bf16 ULP against torch's bf16 matmul); only this build's ttl / ttnn /
    # utils may be imported (never the reference's python package)
    assert not any(p.startswith("/root/reference") for p in sys.path)
    src = open(os.path.join(REF, path)).read()
    g = {"__name__": "metal_example"}
    exec(compile(src, os.path.join(REF, path), "exec"), g)
    g[test](*args)
    import utils
    assert os.path.dirname(utils.__file__).endswith("tt-lang_amd/utils")
    for m in list(sys.modules.values()):
        f = getattr(m, "__file__", None) or ""
        assert not f.startswith("/root/reference"), f"reference module imported: {f}"
