"""Whole tt-lang kernels on the MI355X through the drop-in `ttl`, checked
against the CPU oracle's eager tile-by-tile executor (same kernel source).

Bars: elementwise/broadcast kernels bit-exact (exp: <= 1 bf16 ulp); matmul
kernels within the tolerance the reference's own examples assert
(assert_pcc rtol = atol = 1e-4 for fp32, singlecore_matmul.py:84-88) and, for
bf16, within the stated bf16 bound and no worse than the simulator.
Full-size configs are checked against the vectorised oracle (whole-tensor
torch ops with the same per-op rounding) and float64 products.
"""

import math

import pytest
import torch

import kernel_lib as KL
import ttl
import ttnn
from oracle import sim_exec, tile_ops as O

pytestmark = pytest.mark.gpu


def _oracle(factory, tensors, out_index, **kw):
    ons = sim_exec.make_ttl()
    k = factory(ons, ttnn, **kw) if "ttnn" in factory.__code__.co_varnames else factory(ons, **kw)
    oargs = [sim_exec.OracleTensor(t.clone()) for t in tensors]
    k(*oargs)
    return oargs[out_index].t


def _gpu(factory, tensors, out_index, **kw):
    k = factory(ttl, ttnn, **kw) if "ttnn" in factory.__code__.co_varnames else factory(ttl, **kw)
    args = [ttnn.from_torch(t) for t in tensors]
    k(*args)
    return ttnn.to_torch(args[out_index]), k


def test_eltwise_add_kernel_bitexact():
    a = O.seeded((256, 256), "uniform", 1, torch.float32, lo=0, hi=1)
    b = O.seeded((256, 256), "uniform", 2, torch.float32, lo=0, hi=1)
    out = torch.zeros(256, 256)
    got, _ = _gpu(KL.make_eltwise_add, [a, b, out], 2)
    assert torch.equal(got, _oracle(KL.make_eltwise_add, [a, b, out], 2))


def test_eltwise_add_bf16_2048_config1():
    # bf16 2048x2048, U[-1, 1]
    a = O.seeded((2048, 2048), "uniform", 3, lo=-1, hi=1)
    b = O.seeded((2048, 2048), "uniform", 4, lo=-1, hi=1)
    got, k = _gpu(KL.make_eltwise_add, [a, b, torch.zeros(2048, 2048, dtype=torch.bfloat16)], 2)
    assert len(k.last_plan.launches) == 1
    assert torch.equal(got, a + b)  # the simulator's per-tile bf16 add, vectorised


def test_bcast_fma_kernel_bitexact():
    n = 512
    a, b = O.seeded((n, n), "uniform", 5), O.seeded((n, n), "uniform", 6)
    c = O.seeded((n, 1), "uniform", 7)
    ts = [a, b, c, torch.zeros(n, n, dtype=torch.bfloat16)]
    got, _ = _gpu(KL.make_bcast_fma, ts, 3, g=2, grid=(4, 4))
    assert torch.equal(got, _oracle(KL.make_bcast_fma, ts, 3, g=2, grid=(4, 4)))


def test_exp_row_pipe_kernel():
    n = 256
    a, c = O.seeded((n, n), "uniform", 8, lo=-2, hi=2), O.seeded((n, n), "uniform", 9, lo=-2, hi=2)
    b = O.seeded((1, n), "uniform", 10, lo=-2, hi=2)
    ts = [a, b, c, torch.zeros(n, n, dtype=torch.bfloat16)]
    got, _ = _gpu(KL.make_exp_row_pipe, ts, 3, g=2, grid=(2, 2))
    ref = _oracle(KL.make_exp_row_pipe, ts, 3, g=2, grid=(2, 2))
    assert int(O.bf16_ulp_diff(got, ref).max()) <= 1


def test_exp_row_pipe_4096_config2():
    # BASELINE configs[1] at full size through the unmodified-style kernel
    n = 4096
    a, c = O.seeded((n, n), "uniform", 11, lo=-2, hi=2), O.seeded((n, n), "uniform", 12, lo=-2, hi=2)
    b = O.seeded((1, n), "uniform", 13, lo=-2, hi=2)
    got, k = _gpu(KL.make_exp_row_pipe, [a, b, c, torch.zeros(n, n, dtype=torch.bfloat16)], 3)
    ref = torch.exp(a + b) * c
    ulp = O.bf16_ulp_diff(got, ref)
    assert int(ulp.max()) <= 1
    assert float((ulp > 0).float().mean()) < 1e-3


def test_tile_reuse_kernel_bitexact():
    a = O.seeded((256, 256), "uniform", 14)
    t = O.seeded((32, 32), "uniform", 15)
    ts = [a, t, torch.zeros(256, 256, dtype=torch.bfloat16)]
    got, _ = _gpu(KL.make_tile_reuse, ts, 2)
    assert torch.equal(got, _oracle(KL.make_tile_reuse, ts, 2))


def test_branchy_kernel_scalar_fallback():
    a, b = O.seeded((64, 128), "uniform", 16), O.seeded((64, 128), "uniform", 17)
    ts = [a, b, torch.zeros(64, 128, dtype=torch.bfloat16)]
    got, _ = _gpu(KL.make_branchy_add, ts, 2)
    assert torch.equal(got, _oracle(KL.make_branchy_add, ts, 2))


@pytest.mark.parametrize("factory", [KL.make_matmul_single, KL.make_matmul_multi])
def test_matmul_kernels_fp32_like_examples(factory):
    # the reference examples' case: fp32 128x256 @ 256x64, assert_pcc rtol=atol=1e-4
    a = O.seeded((128, 256), "uniform", 18, torch.float32, lo=0, hi=1)
    b = O.seeded((256, 64), "uniform", 19, torch.float32, lo=0, hi=1)
    ts = [a, b, torch.zeros(128, 64)]
    got, _ = _gpu(factory, ts, 2)
    ref = _oracle(factory, ts, 2)
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4)


def test_matmul_kernel_bf16_vs_sim_error():
    M = K = N = 256
    a = O.seeded((M, K), "normal", 20, std=1 / math.sqrt(K))
    b = O.seeded((K, N), "normal", 21, std=1 / math.sqrt(K))
    ts = [a, b, torch.zeros(M, N, dtype=torch.bfloat16)]
    got, _ = _gpu(KL.make_matmul_single, ts, 2)
    sim = _oracle(KL.make_matmul_single, ts, 2)
    exact = O.matmul_fp64(a, b)
    e_gpu = float((got.double() - exact).abs().max())
    e_sim = float((sim.double() - exact).abs().max())
    assert e_gpu <= e_sim
    assert e_gpu <= 1e-2 * float(exact.abs().max())


def test_matmul_multi_4096_config3():
    n = 4096
    a = O.seeded((n, n), "normal", 22, std=1 / math.sqrt(n))
    b = O.seeded((n, n), "normal", 23, std=1 / math.sqrt(n))
    got, k = _gpu(KL.make_matmul_multi, [a, b, torch.zeros(n, n, dtype=torch.bfloat16)], 2)
    rows = torch.arange(0, n, 64)
    exact = a[rows].double() @ b.double()
    err = (got[rows].double() - exact).abs()
    assert float(err.max()) <= 1e-2 * float(exact.abs().max())
    assert bool((err <= exact.abs() * 2 ** -8 + 1e-6 * 64 * float(exact.abs().max())).all())


def test_ttnn_multiply_runs_on_device():
    a = O.seeded((256, 256), "uniform", 24)
    b = O.seeded((256, 256), "uniform", 25)
    got = ttnn.to_torch(ttnn.multiply(ttnn.from_torch(a), ttnn.from_torch(b)))
    assert torch.equal(got, a * b)


def test_outer_fma_three_arg_broadcast_bitexact():
    # the broadcast tutorials' pattern: (H,1) x (1,W) + (1,1), scalar block held
    # by compute for the whole kernel, multicore
    n = 512
    a, b, c = O.seeded((n, 1), "uniform", 21), O.seeded((1, n), "uniform", 22), O.seeded((1, 1), "uniform", 23)
    ts = [a, b, c, torch.zeros(n, n, dtype=torch.bfloat16)]
    got, k = _gpu(KL.make_outer_fma, ts, 3)
    assert len(k.last_plan.launches) == 1
    assert torch.equal(got, _oracle(KL.make_outer_fma, ts, 3))


@pytest.mark.parametrize("bshape,cshape", [((1024, 1024), (1024, 1024)), ((1024, 1), (1, 1024)),
                                           ((1, 1024), (1, 1)), ((1, 1), (1024, 1))])
def test_shape_dispatch_fma_bitexact(bshape, cshape):
    # general_broadcast.py's pattern: CB shapes / slices / broadcast dims picked
    # from the operand shapes, auto grid
    n = 1024
    a, b, c = O.seeded((n, n), "uniform", 24), O.seeded(bshape, "uniform", 25), O.seeded(cshape, "uniform", 26)
    ts = [a, b, c, torch.zeros(n, n, dtype=torch.bfloat16)]
    got, k = _gpu(KL.make_shape_dispatch_fma, ts, 3)
    assert len(k.last_plan.launches) == 1
    expect = O.eval_expr(("add", ("mul", ("leaf", "a"), ("leaf", "b")), ("leaf", "c")),
                         {"a": a, "b": b, "c": c})
    assert torch.equal(got, expect)


def test_matmul_split_rows_meets_metal_examples_ulp_bar():
    # the metal examples' tt-lang versions check 10 bf16 ULP against torch's
    # bf16 matmul (examples/metal_examples/*/ttlang/*.py, utils/correctness.py)
    from utils.correctness import assert_with_ulp
    n = 640
    a = ttnn.rand((n, n), dtype=ttnn.bfloat16, layout=ttnn.TILE_LAYOUT)
    b = ttnn.rand((n, n), dtype=ttnn.bfloat16, layout=ttnn.TILE_LAYOUT)
    c = ttnn.empty((n, n), dtype=ttnn.bfloat16, layout=ttnn.TILE_LAYOUT)
    k = KL.make_matmul_split_rows(ttl)
    k(a, b, c)
    assert len(k.last_plan.launches) == 1
    golden = torch.matmul(ttnn.to_torch(a).to(torch.bfloat16), ttnn.to_torch(b).to(torch.bfloat16))
    assert_with_ulp(golden, ttnn.to_torch(c).to(torch.bfloat16))


def test_row_bias_multicast_pipe_kernel_bitexact():
    # blocks multicast over pipes become direct tile reads of the sent block's
    # origin; per-op bf16 rounding = torch's bf16 add (pinned in test_oracle)
    a = O.seeded((512, 256), "uniform", 31)
    bias = O.seeded((1, 256), "uniform", 32)
    got, k = _gpu(KL.make_row_bias_multicast, [a, bias, torch.zeros(512, 256, dtype=torch.bfloat16)], 2)
    assert len(k.last_plan.launches) == 1
    assert torch.equal(got, a + bias)


def test_forwarded_pipe_block_kernel_bitexact():
    # core 1 forwards on a second pipe the block it received from core 0:
    # core 2's launch reads the tile core 0 copied (closed form: one bf16 add)
    a = O.seeded((32, 64), "uniform", 33)
    b = O.seeded((64, 96), "uniform", 34)
    got, k = _gpu(KL.make_pipe_chain, [a, b, torch.zeros(64, 96, dtype=torch.bfloat16)], 2)
    want = torch.cat([torch.cat([a[:, 32 * j:32 * (j + 1)] + b[32 * j:32 * (j + 1),
                                                               32 * c:32 * (c + 1)]
                                 for c in range(3)], 1) for j in range(2)], 0)
    assert torch.equal(got, want)


def test_body_created_tensor_rebound_across_calls():
    # the kernel body expands c to a tile with ttnn ops; a second call with a
    # new c reuses the cached plan but must read the new expansion
    k = KL.make_scalar_expand_add(ttl, ttnn)
    a = O.seeded((64, 128), "uniform", 33)
    y = ttnn.from_torch(torch.zeros(64, 128, dtype=torch.bfloat16))
    for cval in (1.5, -2.0, 0.25):
        k(ttnn.from_torch(a), ttnn.from_torch(torch.full((1, 1), cval, dtype=torch.bfloat16)), y)
        assert torch.equal(ttnn.to_torch(y), a + torch.tensor(cval, dtype=torch.bfloat16))
    assert len(k._cache) == 1


def test_bcast_fma_example_config():
    # examples/broadcast.py's own configuration (GRANULARITY 4, grid (8, 8),
    # bf16 2048x2048, c of shape (2048, 1)); the unmodified example plans to
    # these launches (test_examples_unchanged.py)
    n = 2048
    a, b = O.seeded((n, n), "uniform", 40, lo=0, hi=1), O.seeded((n, n), "uniform", 41, lo=0, hi=1)
    c = O.seeded((n, 1), "uniform", 42, lo=0, hi=1)
    got, k = _gpu(KL.make_bcast_fma, [a, b, c, torch.zeros(n, n, dtype=torch.bfloat16)], 3)
    assert len(k.last_plan.launches) == 1
    assert torch.equal(got, a * b + c)  # per-op bf16 rounding, vectorised


@pytest.mark.parametrize("bm,bk,bn,R,C", [(1, 3, 4, 2, 1), (2, 4, 2, 2, 3)])
def test_block_matmul_kernel_gpu(bm, bk, bn, R, C):
    # the spec's (M, K) @ (K, N) block matmul planned onto one tile matmul
    # launch: within one bf16 ulp of the oracle and of the float64 product
    a = O.seeded((bm * 32 * R, bk * 32), "normal", 3 * bm + bk)
    b = O.seeded((bk * 32, bn * 32 * C), "normal", 5 * bn + C)
    out = torch.zeros(a.shape[0], b.shape[1], dtype=torch.bfloat16)
    got, k = _gpu(KL.make_block_matmul, [a, b, out], 2, bm=bm, bk=bk, bn=bn)
    assert len(k.last_plan.launches) == 1
    orc = _oracle(KL.make_block_matmul, [a, b, out], 2, bm=bm, bk=bk, bn=bn)
    exact = (a.double() @ b.double()).to(torch.bfloat16)
    assert int(O.bf16_ulp_diff(got, orc).abs().max()) <= 1
    assert int(O.bf16_ulp_diff(got, exact).abs().max()) <= 1


@pytest.mark.parametrize("K", [96, 1024])
def test_dma_gemm_with_slow_operand_loads(K):
    # A and B in pinned host memory: every operand load of the 256x256 DMA
    # GEMM crosses PCIe and takes far longer than a stage, so a wait that let
    # a stage be read before its loads landed would show as wrong products
    # (K = 96: the three-stage tail path only; K = 1024: the steady loop)
    from ttlhip import _lib as L
    M = N = 4096
    g = torch.Generator().manual_seed(K)
    a = (torch.randn(M, K, generator=g) / K ** 0.5).bfloat16()
    b = (torch.randn(K, N, generator=g) / K ** 0.5).bfloat16()
    ah, bh = a.pin_memory(), b.pin_memory()
    c = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
    L.call("ttlh_matmul", ah.data_ptr(), L.dtype_code(a.dtype), K, bh.data_ptr(),
           L.dtype_code(b.dtype), N, c.data_ptr(), L.dtype_code(c.dtype), N, M, N, K, 0,
           L.stream_ptr())
    torch.cuda.synchronize()
    rows = torch.arange(0, M, 61)
    exact = a[rows].double() @ b.double()
    err = float((c.cpu()[rows].double() - exact).abs().max())
    assert err <= 1e-2 * float(exact.abs().max()), err
