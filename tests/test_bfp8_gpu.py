"""bfloat8_b on the MI355X: device dequantisation (bit-exact against the
oracle for every (exponent, byte) pair) and the bf16 x bfp8-weight matmul on
both paths (fused: dequantised in LDS ahead of the MFMA; two-pass: dequantised
once into a bf16 workspace, then the bf16 GEMM), checked against float64
products of the oracle-dequantised weights."""

import math

import numpy as np
import pytest
import torch

from oracle import bfp8 as OB
from oracle import tile_ops as O

pytestmark = pytest.mark.gpu


def _all_pairs_tiles():
    q = np.zeros((64, 1088), dtype=np.uint8)
    for t in range(64):
        for r in range(32):
            for c in range(32):
                f = (r // 16) * 2 + c // 16
                q[t, 16 * f + r % 16] = (t * 4 + f) % 256
                q[t, 64 + 256 * f + 16 * (r % 16) + c % 16] = ((r % 16) * 16 + c % 16) % 256
    return torch.from_numpy(q.ravel().copy())


def test_device_dequant_all_pairs_bitexact():
    from ttlhip import kernels as K
    q = _all_pairs_tiles()
    got = K.bfp8_unpack(q.cuda(), 32, 2048).cpu()
    ref = OB.unpack_c(q, 32, 2048)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_device_dequant_random_weights():
    from ttlhip import kernels as K
    w = O.seeded((256, 512), "normal", 3, torch.float32, std=0.02)
    q = OB.pack_c(w)
    got = K.bfp8_unpack(q.cuda(), 256, 512).cpu()
    assert torch.equal(got.view(torch.int16), OB.unpack_c(q, 256, 512).view(torch.int16))


@pytest.mark.parametrize("rows,cols", [(96, 1440), (32, 32), (64, 2080)])
def test_device_dequant_ragged_tile_runs(rows, cols):
    # ragged tile grids (odd tile counts per row, a single tile, partial last workgroup)
    from ttlhip import kernels as K
    w = O.seeded((rows, cols), "normal", 4, torch.float32, std=0.5)
    q = OB.pack_c(w)
    got = K.bfp8_unpack(q.cuda(), rows, cols).cpu()
    assert torch.equal(got.view(torch.int16), OB.unpack_c(q, rows, cols).view(torch.int16))


@pytest.mark.parametrize("two_pass", [False, True])
@pytest.mark.parametrize("M,K,N", [(128, 256, 128), (96, 160, 224), (256, 512, 352)])
def test_matmul_bfp8w_small(M, K, N, two_pass):
    from ttlhip import kernels as Kn
    a = O.seeded((M, K), "normal", 5)
    w = O.seeded((K, N), "normal", 6, torch.float32, std=0.02)
    q = OB.pack_c(w)
    c = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    Kn.matmul_bfp8w(a.cuda(), q.cuda(), c, two_pass=two_pass)
    torch.cuda.synchronize()
    wd = OB.unpack_c(q, K, N)
    exact = a.double() @ wd.double()
    err = (c.cpu().double() - exact).abs()
    bound = exact.abs() * 2.0 ** -8 + 1e-6 * math.sqrt(K) * float(exact.abs().max())
    assert bool((err <= bound).all()), float(err.max())


@pytest.mark.parametrize("two_pass", [False, True])
def test_matmul_bfp8w_config4_sampled(two_pass):
    from ttlhip import kernels as Kn
    M, K, N = 4096, 4096, 11008
    a = O.seeded((M, K), "normal", 7)
    w = O.seeded((K, N), "normal", 8, torch.float32, std=0.02)
    q = OB.pack_c(w)
    c = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    Kn.matmul_bfp8w(a.cuda(), q.cuda(), c, two_pass=two_pass)
    torch.cuda.synchronize()
    rows = torch.arange(0, M, 128)
    wd = OB.unpack_c(q, K, N).double()
    exact = a[rows].double() @ wd
    err = (c.cpu()[rows].double() - exact).abs()
    bound = exact.abs() * 2.0 ** -8 + 1e-6 * 64 * float(exact.abs().max())
    assert bool((err <= bound).all()), float(err.max())


@pytest.mark.parametrize("two_pass", [False, True])
def test_matmul_bfp8w_large_block_ragged(two_pass):
    # >= 192 output blocks of 256x256 -> the large-block kernel; M, N ragged
    # against 256 and K against its 64-deep staging step
    from ttlhip import kernels as Kn
    M, K, N = 2080, 544, 5408
    a = O.seeded((M, K), "normal", 9)
    w = O.seeded((K, N), "normal", 10, torch.float32, std=0.02)
    q = OB.pack_c(w)
    c = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    Kn.matmul_bfp8w(a.cuda(), q.cuda(), c, two_pass=two_pass)
    torch.cuda.synchronize()
    rows = torch.cat([torch.arange(0, M, 41), torch.arange(M - 32, M)])
    wd = OB.unpack_c(q, K, N).double()
    exact = a[rows].double() @ wd
    err = (c.cpu()[rows].double() - exact).abs()
    bound = exact.abs() * 2.0 ** -8 + 1e-6 * math.sqrt(K) * float(exact.abs().max())
    assert bool((err <= bound).all()), float(err.max())


def test_two_pass_matches_fused_path():
    # both paths multiply the same bf16 values with fp32 accumulation in
    # ascending k: results agree to within one bf16 rounding of the sum
    from ttlhip import kernels as Kn
    M, K, N = 1024, 1024, 2048
    a = O.seeded((M, K), "normal", 11).cuda()
    q = OB.pack_c(O.seeded((K, N), "normal", 12, torch.float32, std=0.02)).cuda()
    c1 = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    c2 = torch.empty_like(c1)
    Kn.matmul_bfp8w(a, q, c1, two_pass=False)
    Kn.matmul_bfp8w(a, q, c2, two_pass=True)
    torch.cuda.synchronize()
    assert int(O.bf16_ulp_diff(c1.cpu(), c2.cpu()).max()) <= 1


def _bound_check(got, exact, K):
    err = (got.double() - exact).abs()
    bound = exact.abs() * 2.0 ** -8 + 1e-6 * math.sqrt(K) * float(exact.abs().max())
    assert bool((err <= bound).all()), float(err.max())


@pytest.mark.parametrize("M,K,N", [(96, 256, 160), (512, 384, 640)])
def test_ttnn_matmul_with_bfloat8_b_weights(M, K, N):
    # ttnn-level use of the format: from_torch(dtype=bfloat8_b) packs, matmul
    # runs the fused (small M) or two-pass (M >= 512) bf16 x bfloat8_b GEMM
    import ttnn
    a = O.seeded((M, K), "normal", 61)
    w = O.seeded((K, N), "normal", 62, torch.float32, std=0.02)
    wq = ttnn.from_torch(w, dtype=ttnn.bfloat8_b, layout=ttnn.TILE_LAYOUT)
    back = ttnn.to_torch(wq)  # device dequantisation
    assert torch.equal(back, OB.unpack_c(OB.pack_c(w), K, N).float())
    c = ttnn.to_torch(ttnn.matmul(ttnn.from_torch(a), wq))
    _bound_check(c, a.double() @ back.double(), K)


@pytest.mark.parametrize("M,K,N", [(256, 256, 320), (1024, 512, 1024)])
def test_ttl_kernel_with_bfloat8_b_weights(M, K, N):
    # a tt-lang multicore matmul kernel whose B tensor is bfloat8_b: the plan
    # is one bf16 x bfloat8_b GEMM launch
    import kernel_lib as KL
    import ttl
    import ttnn
    a = O.seeded((M, K), "normal", 63)
    w = O.seeded((K, N), "normal", 64, torch.float32, std=0.02)
    wq = ttnn.from_torch(w, dtype=ttnn.bfloat8_b)
    c = ttnn.empty((M, N), dtype=ttnn.bfloat16)
    k = KL.make_matmul_multi(ttl, ttnn)
    k(ttnn.from_torch(a), wq, c)
    (l,) = k.last_plan.launches
    assert l.b_block
    exact = a.double() @ OB.unpack_c(OB.pack_c(w), K, N).double()
    _bound_check(ttnn.to_torch(c), exact, K)


def test_fused_bfp8_gemm_with_slow_loads():
    # the fused path (weights decoded between MFMAs) with A and the packed
    # weights in pinned host memory: every load far slower than a k step
    from ttlhip import _lib as L
    from ttlhip import kernels as K
    M, N, Kd = 256, 1024, 512
    g = torch.Generator().manual_seed(8)
    a = torch.randn(M, Kd, generator=g).bfloat16()
    w = torch.randn(Kd, N, generator=g) * 0.02
    bq = K.bfp8_pack_host(w)
    ah, bqh = a.pin_memory(), bq.pin_memory()
    c = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
    L.call("ttlh_matmul_bfp8w", ah.data_ptr(), Kd, bqh.data_ptr(), c.data_ptr(), N, M, N, Kd,
           L.stream_ptr())
    torch.cuda.synchronize()
    _bound_check(c.cpu(), a.double() @ OB.unpack_c(bq, Kd, N).double(), Kd)
