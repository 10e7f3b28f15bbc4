"""bfloat4_b codec: oracle pins, the library's host codec and ttnn / tt-lang
integration on the CPU.

The reference defines only the tile size (576 B, python/ttl/dtype_utils.py:
176-177), so the format is this build's (include/ttlhip.h); parity with
tt-metal's packer is unpinned.  Pins:
  - every (exponent, nibble) pair decodes to the exact float64 value
    (-1)^s m 2^(e-129) (brute force, 4,096 cases) in the C oracle and in the
    library's host decoder;
  - the C (integer-only), numpy (float64) and library packers agree bit for bit;
  - hand-computed vectors: the shared exponent, RNE ties, saturation at 7,
    signed zeros, sub-half values.
"""

import numpy as np
import pytest
import torch

import kernel_lib as KL
import plan_interp
import ttl
import ttnn
from oracle import bfp8 as OB
from oracle import tile_ops as O
from ttlhip import kernels as K
from ttlhip import plan as P


def _all_pairs_tiles():
    """16 tiles; tile t, face f has exponent 16 t + 4 f + (face row) ... chosen
    so that the 64 exponent bytes x 16 nibbles cover all 256 x 16 pairs."""
    q = np.zeros((16, 576), dtype=np.uint8)
    for t in range(16):
        for f in range(4):
            for r in range(16):
                q[t, 16 * f + r] = (t * 64 + f * 16 + r) % 256
                for c in range(16):
                    nib = c  # every nibble in every face row
                    q[t, 64 + 128 * f + 8 * r + c // 2] |= nib << (4 * (c & 1))
    return torch.from_numpy(q.ravel().copy())


def _expected_all_pairs():
    tab = OB.decode4_table()
    out = np.zeros((32, 16 * 32))
    for t in range(16):
        for f in range(4):
            for r in range(16):
                e = (t * 64 + f * 16 + r) % 256
                for c in range(16):
                    out[(f >> 1) * 16 + r, t * 32 + (f & 1) * 16 + c] = tab[e, c]
    return out


def test_oracle_decode_brute_force():
    L = OB.lib()
    tab = OB.decode4_table()
    got = np.array([[L.oracle_bfp4_decode(e, n) for n in range(16)] for e in range(256)],
                   dtype=np.uint32)
    vals = (got << 16).astype(np.uint32).view(np.float32).astype(np.float64)
    assert np.array_equal(vals, tab)


def test_library_host_decoder_all_pairs():
    q = _all_pairs_tiles()
    got = K.bfp4_unpack_host(q, 32, 16 * 32).double().numpy()
    assert np.array_equal(got, _expected_all_pairs())
    assert np.array_equal(OB.unpack4_c(q, 32, 512).double().numpy(), _expected_all_pairs())


def test_packers_agree():
    for seed, scale in ((0, 0.02), (1, 1.0), (2, 1e-30), (3, 3e30)):
        x = torch.randn(96, 64, generator=torch.Generator().manual_seed(seed)) * scale
        x[5, :16] = 0.0
        lib = K.bfp4_pack_host(x)
        assert torch.equal(lib, OB.pack4_c(x))
        assert np.array_equal(lib.numpy(), OB.pack4_np(x.numpy()))


def test_hand_vectors():
    x = torch.zeros(32, 32)
    # face row 0 of face 0: max 1.75 (biased exponent 127): m = RNE(4 |x|)
    row = torch.tensor([1.0, -1.0, 0.5, 0.25, 1.75, 1.875, 0.125, 0.375,
                        0.625, -0.0, 0.0, 0.875, 1.5, 0.1, 1.25, -0.25])
    x[0, :16] = row
    q = OB.pack4_c(x).numpy()
    assert q[0] == 127
    nib = [(q[64 + c // 2] >> (4 * (c & 1))) & 15 for c in range(16)]
    mags = [n & 7 for n in nib]
    signs = [n >> 3 for n in nib]
    # 1.875*4 = 7.5 -> 8 -> saturates at 7; 0.125*4 = 0.5 -> 0 (tie to even);
    # 0.375*4 = 1.5 -> 2; 0.625*4 = 2.5 -> 2; 0.875*4 = 3.5 -> 4; 0.1*4 -> 0
    assert mags == [4, 4, 2, 1, 7, 7, 0, 2, 2, 0, 0, 4, 6, 0, 5, 1]
    assert signs == [0, 1, 0, 0, 0, 0, 0, 0, 0, 1, 0, 0, 0, 0, 0, 1]
    assert torch.equal(K.bfp4_pack_host(x), torch.from_numpy(q))
    back = OB.unpack4_np(q, 32, 32)[0, :16]
    assert back[4] == 1.75 and back[5] == 1.75 and back[14] == 1.25


def test_ttnn_bfloat4_b_tensors_and_matmul_plan():
    w = O.seeded((128, 96), "normal", 8, torch.float32, std=0.5)
    t = ttnn.from_torch(w, dtype=ttnn.bfloat4_b)
    assert t.dtype is ttnn.bfloat4_b and t.shape == (128, 96)
    assert torch.equal(t._tensor.cpu(), OB.pack4_c(w))
    assert torch.equal(ttnn.to_torch(t), OB.unpack4_c(OB.pack4_c(w), 128, 96).float())
    a = O.seeded((64, 128), "normal", 9)
    c = ttnn.Tensor(torch.zeros(64, 96, dtype=torch.bfloat16))
    args = [ttnn.Tensor(a.clone()), t, c]
    plan = KL.make_matmul_multi(ttl, ttnn).trace(*args)
    (l,) = plan.launches
    assert isinstance(l, P.MatmulLaunch) and l.b_block
    plan_interp.run(plan, {i: x for i, x in enumerate(args)})
    exact = (a.double() @ OB.unpack4_c(OB.pack4_c(w), 128, 96).double()).bfloat16()
    assert torch.equal(c._tensor, exact)
