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


def test_tile_array_at_an_8_byte_offset():
    # the device decode reads tiles in 16-byte words: a tile array that is
    # only 8-byte aligned is refused there, and the matmul wrapper sends it to
    # the fused path, whose result it must equal
    from ttlhip import kernels as Kn
    M, K, N = 512, 256, 256
    a = O.seeded((M, K), "normal", 13).cuda()
    q = OB.pack_c(O.seeded((K, N), "normal", 14, torch.float32, std=0.02))
    buf = torch.zeros(q.numel() + 8, dtype=torch.uint8, device="cuda")
    qm = buf[8:]
    qm.copy_(q.cuda())
    assert qm.data_ptr() % 16 == 8
    with pytest.raises(ValueError, match="16-byte aligned"):
        Kn.bfp8_unpack(qm, K, N)
    c1 = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    c2 = torch.empty_like(c1)
    Kn.matmul_bfp8w(a, qm, c1)                            # M >= 512: fused for this Bq
    Kn.matmul_bfp8w(a, q.cuda(), c2, two_pass=False)      # the fused path, aligned Bq
    torch.cuda.synchronize()
    assert torch.equal(c1.cpu().view(torch.int16), c2.cpu().view(torch.int16))


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


# --- the fused entry's large-problem kernel: weights dequantised in LDS -----
# (ttlh_matmul_bfp8w with >= 192 output blocks of 256 x 256, N a multiple of
# 256 and K of 128).  It runs the DMA GEMM's MFMAs in the same k order on the
# same bf16 values as the two-pass path (bfp8_unpack_kernel, itself bit-exact
# against the oracle, then the DMA GEMM), so the two agree bit for bit.


def _lds_decode_vs_two_pass(a, q, M, K, N):
    from ttlhip import kernels as Kn
    c1 = torch.full((M, N), 7.0, dtype=torch.bfloat16, device="cuda")
    c2 = torch.full((M, N), 5.0, dtype=torch.bfloat16, device="cuda")
    Kn.matmul_bfp8w(a, q, c1, two_pass=False)
    Kn.matmul_bfp8w(a, q, c2, two_pass=True)
    torch.cuda.synchronize()
    return c1, c2


@pytest.mark.parametrize("M,K,N", [(4096, 4096, 11008), (2048, 128, 6144), (3072, 512, 4096)])
def test_lds_decode_gemm_equals_two_pass(M, K, N):
    print(f"lds-decode gemm vs two-pass M={M} K={K} N={N}", flush=True)
    a = O.seeded((M, K), "normal", 21).cuda()
    q = OB.pack_c(O.seeded((K, N), "normal", 22, torch.float32, std=0.02)).cuda()
    c1, c2 = _lds_decode_vs_two_pass(a, q, M, K, N)
    assert torch.equal(c1.view(torch.int16), c2.view(torch.int16))


def _all_pairs_weights(K, N, e_lo, e_hi):
    """bfloat8_b tiles of a K x N matrix whose face rows take every exponent in
    [e_lo, e_hi] with every element byte 0..255 (16 face rows per exponent)."""
    nt = (K // 32) * (N // 32)
    q = np.zeros((nt, 1088), dtype=np.uint8)
    ne = e_hi - e_lo + 1
    g = 0
    for t in range(nt):
        for x in range(64):
            q[t, x] = e_lo + g % ne
            q[t, 64 + 16 * x:64 + 16 * x + 16] = 16 * ((g // ne) % 16) + np.arange(16)
            g += 1
    assert g >= 16 * ne
    return torch.from_numpy(q.ravel().copy())


def test_lds_decode_gemm_all_pairs_equals_two_pass():
    # every (exponent, byte) pair the packer can produce (e <= 254), subnormal
    # products included, through the in-LDS decode: equal to the two-pass path
    M, K, N = 4096, 128, 3072
    q = _all_pairs_weights(K, N, 0, 254).cuda()
    a = O.seeded((M, K), "normal", 23).cuda()
    c1, c2 = _lds_decode_vs_two_pass(a, q, M, K, N)
    assert torch.equal(c1.view(torch.int16), c2.view(torch.int16))


def test_lds_decode_gemm_selects_decoded_rows_exactly():
    # A row i is the unit vector e_(i mod K), so C row i is weight row i mod K
    # itself: exact against the oracle's dequantisation (normal values only,
    # e >= 7, so no subnormal operand is involved; -0 reads as +0)
    M, K, N = 4096, 128, 3072
    q = _all_pairs_weights(K, N, 7, 254)
    a = torch.zeros(M, K, dtype=torch.bfloat16)
    a[torch.arange(M), torch.arange(M) % K] = 1.0
    from ttlhip import kernels as Kn
    c = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    Kn.matmul_bfp8w(a.cuda(), q.cuda(), c, two_pass=False)
    torch.cuda.synchronize()
    wd = OB.unpack_c(q, K, N)
    assert torch.equal(c.cpu(), wd[torch.arange(M) % K])


def test_lds_decode_gemm_with_slow_loads():
    # A and the packed weights in pinned host memory: every load of a stage
    # far slower than a stage's MFMAs; the waits must still cover them
    from ttlhip import _lib as L
    from ttlhip import kernels as Kn
    M, K, N = 2048, 256, 6144
    a = O.seeded((M, K), "normal", 24)
    q = OB.pack_c(O.seeded((K, N), "normal", 25, torch.float32, std=0.02))
    ah, qh = a.pin_memory(), q.pin_memory()
    c = torch.zeros(M, N, dtype=torch.bfloat16, device="cuda")
    L.call("ttlh_matmul_bfp8w", ah.data_ptr(), K, qh.data_ptr(), c.data_ptr(), N, M, N, K,
           L.stream_ptr())
    ref = torch.empty_like(c)
    Kn.matmul_bfp8w(a.cuda(), q.cuda(), ref, two_pass=True)
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int16), ref.view(torch.int16))
