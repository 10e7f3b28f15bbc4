"""GPU parity of the tile matmul (ttlh_matmul) against the CPU oracle.

The simulator multiplies 32x32 tiles in the input dtype and accumulates the K
tile products with store(acc=True) in the output block's dtype
(oracle.tile_ops.tile_matmul_sim); the MI355X kernel accumulates the full K
in fp32 and rounds once.  Parity bar (stated by the north star for bf16):
  - |gpu - exact| <= 1 bf16 ulp of |exact| + 1e-6 * sqrt(K) * max|exact|
    (one final rounding plus fp32 accumulation error), i.e. max-abs well
    inside 1e-2 relative to the fp32/fp64 reference, and
  - the GPU's max error is no worse than the simulator restatement's.
fp32 inputs: torch.testing.assert_close against float64 with rtol = atol = 1e-5
(the examples' own assert_pcc uses rtol = atol = 1e-4).
"""

import math

import pytest
import torch

from oracle import tile_ops as O

pytestmark = pytest.mark.gpu


def _mm(a, b, out_dtype, accumulate=False, c0=None):
    from ttlhip import kernels as K

    da, db = a.cuda(), b.cuda()
    c = (c0.cuda().clone() if c0 is not None
         else torch.zeros((a.shape[0], b.shape[1]), dtype=out_dtype, device="cuda"))
    K.matmul(da, db, c, accumulate=accumulate)
    torch.cuda.synchronize()
    return c.cpu()


def _inputs(M, K, N, seed, dtype=torch.bfloat16):
    a = O.seeded((M, K), "normal", seed, dtype, std=1.0 / math.sqrt(K) ** 0.5)
    b = O.seeded((K, N), "normal", seed + 1, dtype, std=1.0 / math.sqrt(K) ** 0.5)
    return a, b


@pytest.mark.parametrize("M,K,N", [(128, 128, 128), (256, 384, 192), (96, 160, 224),
                                   (32, 32, 32), (512, 1024, 256)])
def test_bf16_matmul_vs_exact_and_sim(M, K, N):
    a, b = _inputs(M, K, N, 7)
    got = _mm(a, b, torch.bfloat16).double()
    exact = O.matmul_fp64(a, b)
    sim = O.tile_matmul_sim(a, b).double()
    err_gpu = (got - exact).abs()
    err_sim = (sim - exact).abs()
    bound = exact.abs() * 2.0 ** -8 + 1e-6 * math.sqrt(K) * float(exact.abs().max())
    assert bool((err_gpu <= bound).all()), f"max err {float(err_gpu.max())}"
    assert float(err_gpu.max()) <= float(err_sim.max()) + 1e-12
    assert float(err_gpu.max()) <= 1e-2 * float(exact.abs().max())


def test_bf16_matmul_accumulate_and_f32_out():
    a, b = _inputs(128, 256, 160, 11)
    c0 = O.seeded((128, 160), "normal", 13, torch.float32)
    got = _mm(a, b, torch.float32, accumulate=True, c0=c0).double()
    exact = O.matmul_fp64(a, b) + c0.double()
    torch.testing.assert_close(got, exact, rtol=1e-5, atol=1e-5)


def test_bf16_matmul_layout_known_answer():
    # A = identity-like permutation, B = distinct integers: every output element
    # is an exact small integer, so any lane-layout mistake shows up exactly.
    M = K = N = 128
    perm = torch.randperm(K, generator=torch.Generator().manual_seed(3))
    a = torch.zeros(M, K)
    a[torch.arange(M), perm] = 1.0
    b = (torch.arange(K * N).reshape(K, N) % 251).float()
    got = _mm(a.bfloat16(), b.bfloat16(), torch.float32)
    assert torch.equal(got, b[perm])


@pytest.mark.parametrize("M,K,N", [(64, 64, 64), (128, 256, 64), (96, 160, 224)])
def test_f32_matmul(M, K, N):
    a = O.seeded((M, K), "uniform", 21, torch.float32, lo=0, hi=1)
    b = O.seeded((K, N), "uniform", 22, torch.float32, lo=0, hi=1)
    got = _mm(a, b, torch.float32).double()
    torch.testing.assert_close(got, O.matmul_fp64(a, b), rtol=1e-5, atol=1e-5)


def test_bf16_matmul_4096_sampled_rows():
    # the benchmark shape: check 64 sampled rows against float64
    M = K = N = 4096
    a = O.seeded((M, K), "normal", 31, torch.bfloat16, std=1.0 / math.sqrt(K))
    b = O.seeded((K, N), "normal", 32, torch.bfloat16, std=1.0 / math.sqrt(K))
    got = _mm(a, b, torch.bfloat16).double()
    rows = torch.arange(0, M, M // 64)
    exact = a[rows].double() @ b.double()
    err = (got[rows] - exact).abs()
    bound = exact.abs() * 2.0 ** -8 + 1e-6 * math.sqrt(K) * float(exact.abs().max())
    assert bool((err <= bound).all()), f"max err {float(err.max())}"


# Problems with >= 192 output blocks of 256x256 take the large-block kernel
# (mm256_kernel); the shapes below are ragged on purpose: M and N not
# multiples of 256, K not a multiple of its 64-deep staging step.

def test_bf16_large_block_kernel_ragged_sampled():
    M, K, N = 4000, 1056, 3104  # 16 x 13 = 208 blocks
    a, b = _inputs(M, K, N, 41)
    got = _mm(a, b, torch.bfloat16).double()
    rows = torch.cat([torch.arange(0, M, 37), torch.arange(M - 40, M)])
    exact = a[rows].double() @ b.double()
    err = (got[rows] - exact).abs()
    bound = exact.abs() * 2.0 ** -8 + 1e-6 * math.sqrt(K) * float(exact.abs().max())
    assert bool((err <= bound).all()), f"max err {float(err.max())}"
    sim_rows = O.tile_matmul_sim(a[-32:], b).double()  # last tile row through the simulator rule
    assert float((got[-32:] - exact[-32:]).abs().max()) <= float((sim_rows - exact[-32:]).abs().max()) + 1e-12


def test_bf16_large_block_kernel_layout_known_answer():
    # permutation rows x small integers: every output is exact, so any
    # fragment / accumulator layout mistake in the 256x256 kernel is visible
    M = K = N = 3584  # 14 x 14 = 196 blocks
    perm = torch.randperm(K, generator=torch.Generator().manual_seed(5))
    a = torch.zeros(M, K, dtype=torch.bfloat16)
    a[torch.arange(M), perm] = 1.0
    b = (torch.arange(K * N).reshape(K, N) % 251).to(torch.bfloat16)
    got = _mm(a, b, torch.float32)
    assert torch.equal(got, b[perm].float())


def test_bf16_large_block_kernel_accumulate_f32():
    M, K, N = 3584, 96, 3616  # 14 x 15 = 210 blocks, K shorter than one 64-step pair
    a, b = _inputs(M, K, N, 43)
    c0 = O.seeded((M, N), "normal", 44, torch.float32)
    got = _mm(a, b, torch.float32, accumulate=True, c0=c0).double()
    exact = O.matmul_fp64(a, b) + c0.double()
    torch.testing.assert_close(got, exact, rtol=1e-5, atol=1e-5)


# Large problems whose 256x256 block count does not fill whole rounds of the
# 256 CUs, some with N ragged against 256: every output tile is the same MFMA
# sequence over k whatever the grid, so the result equals, bit for bit, the
# same product with B padded by zero columns to a block count the CUs divide
# evenly (and stays within the float64 bound).
@pytest.mark.parametrize("M,N,K", [(4096, 5120, 256), (4096, 6144, 256), (2048, 11008, 256),
                                   (4096, 11008, 128), (4096, 5216, 256)])
def test_large_gemm_independent_of_padding(M, N, K):
    print(f"padding invariance M={M} N={N} K={K}", flush=True)
    from ttlhip import kernels as Kn
    a, b = _inputs(M, K, N, 71)
    # padded width: whole rounds of blocks (256 per round, M / 256 per column)
    unit = 256 * 256 // (M // 256)
    npad = -(-N // unit) * unit
    bp = torch.zeros(K, npad, dtype=torch.bfloat16)
    bp[:, :N] = b
    c = torch.full((M, N), 3.0, dtype=torch.bfloat16, device="cuda")
    cp = torch.empty((M, npad), dtype=torch.bfloat16, device="cuda")
    Kn.matmul(a.cuda(), b.cuda(), c, accumulate=False)
    Kn.matmul(a.cuda(), bp.cuda(), cp, accumulate=False)
    torch.cuda.synchronize()
    assert torch.equal(c.cpu().view(torch.int16), cp.cpu()[:, :N].view(torch.int16))
    rows = torch.arange(0, M, 97)
    exact = a[rows].double() @ b.double()
    err = (c.cpu()[rows].double() - exact).abs()
    bound = exact.abs() * 2.0 ** -8 + 1e-6 * math.sqrt(K) * float(exact.abs().max())
    assert bool((err <= bound).all()), float(err.max())
