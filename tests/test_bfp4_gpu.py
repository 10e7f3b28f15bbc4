"""bfloat4_b on the MI355X: device dequantisation bit-exact against the
oracle for every (exponent, nibble) pair, and matmuls with bfloat4_b weights
(dequantisation pass + bf16 GEMM) through the C ABI, ttnn and a tt-lang
kernel, against float64 products of the oracle-dequantised weights."""

import math

import numpy as np
import pytest
import torch

from oracle import bfp8 as OB
from oracle import tile_ops as O

pytestmark = pytest.mark.gpu


def test_device_dequant_all_pairs_bitexact():
    from test_bfp4 import _all_pairs_tiles, _expected_all_pairs
    from ttlhip import kernels as K
    got = K.bfp4_unpack(_all_pairs_tiles().cuda(), 32, 512).cpu().double().numpy()
    assert np.array_equal(got, _expected_all_pairs())


@pytest.mark.parametrize("rows,cols", [(96, 1440), (32, 32), (64, 2080), (32, 2048)])
def test_device_dequant_random(rows, cols):
    from ttlhip import kernels as K
    w = O.seeded((rows, cols), "normal", 71, torch.float32, std=0.3)
    q = OB.pack4_c(w)
    assert torch.equal(K.bfp4_unpack(q.cuda(), rows, cols).cpu().view(torch.int16),
                       OB.unpack4_c(q, rows, cols).view(torch.int16))


def test_device_dequant_tile_array_at_an_8_byte_offset():
    # the decode stages tiles in 8-byte loads: an array that is 8- but not
    # 16-byte aligned decodes to the same bits
    from ttlhip import kernels as K
    rows, cols = 64, 800
    q = OB.pack4_c(O.seeded((rows, cols), "normal", 72, torch.float32, std=0.3))
    buf = torch.zeros(q.numel() + 8, dtype=torch.uint8, device="cuda")
    qm = buf[8:]
    qm.copy_(q.cuda())
    assert qm.data_ptr() % 16 == 8
    assert torch.equal(K.bfp4_unpack(qm, rows, cols).cpu().view(torch.int16),
                       OB.unpack4_c(q, rows, cols).view(torch.int16))


def _bound_check(got, exact, K):
    err = (got.double() - exact).abs()
    bound = exact.abs() * 2.0 ** -8 + 1e-6 * math.sqrt(K) * float(exact.abs().max())
    assert bool((err <= bound).all()), float(err.max())


@pytest.mark.parametrize("M,K,N", [(96, 256, 160), (512, 384, 640)])
def test_matmul_with_bfloat4_b_weights(M, K, N):
    import ttnn
    from ttlhip import kernels as Kn
    a = O.seeded((M, K), "normal", 72)
    w = O.seeded((K, N), "normal", 73, torch.float32, std=0.02)
    wd = OB.unpack4_c(OB.pack4_c(w), K, N).double()
    c = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    Kn.matmul_bfp4w(a.cuda(), OB.pack4_c(w).cuda(), c)
    torch.cuda.synchronize()
    _bound_check(c.cpu(), a.double() @ wd, K)
    wq = ttnn.from_torch(w, dtype=ttnn.bfloat4_b)
    _bound_check(ttnn.to_torch(ttnn.matmul(ttnn.from_torch(a), wq)), a.double() @ wd, K)


def test_ttl_kernel_with_bfloat4_b_weights():
    import kernel_lib as KL
    import ttl
    import ttnn
    M, K, N = 1024, 512, 1024
    a = O.seeded((M, K), "normal", 74)
    w = O.seeded((K, N), "normal", 75, torch.float32, std=0.02)
    c = ttnn.empty((M, N), dtype=ttnn.bfloat16)
    k = KL.make_matmul_multi(ttl, ttnn)
    k(ttnn.from_torch(a), ttnn.from_torch(w, dtype=ttnn.bfloat4_b), c)
    (l,) = k.last_plan.launches
    assert l.b_block
    _bound_check(ttnn.to_torch(c), a.double() @ OB.unpack4_c(OB.pack4_c(w), K, N).double(), K)
