"""bfloat8_b codec: oracle pins and the library's host codec (CPU).

The reference defines only the tile size (1088 B, python/ttl/dtype_utils.py:
174-175), so the format is this build's (include/ttlhip.h).  Pins:
  - every (exponent, byte) pair decodes to the exact float64 value
    (-1)^s m 2^(e-133) (brute force, 65,536 cases), in the C oracle and in
    the library's host decoder;
  - the C (integer-only) and numpy (float64) packers agree bit for bit;
  - hand-computed vectors: powers of two, a face row's max, ties, zeros,
    subnormal inputs, saturation;
  - round trip: decode(encode(x)) is within half a step of the shared scale,
    encode(decode(q)) == q for canonical blocks.
"""

import numpy as np
import pytest
import torch

from oracle import bfp8 as OB


def test_oracle_decode_brute_force():
    L = OB.lib()
    tab = OB.decode_table()
    got = np.array([[L.oracle_bfp8_decode(e, b) for b in range(256)] for e in range(256)],
                   dtype=np.uint32)
    vals = (got << 16).astype(np.uint32).view(np.float32).astype(np.float64)
    assert np.array_equal(vals, tab)


def test_oracle_c_and_numpy_packers_agree():
    for seed, scale in ((0, 0.02), (1, 1.0), (2, 1e-30), (3, 3e30)):
        x = torch.randn(96, 64, generator=torch.Generator().manual_seed(seed)) * scale
        x[5, :16] = 0.0  # an all-zero face row
        assert np.array_equal(OB.pack_c(x).numpy(), OB.pack_np(x.numpy()))
        q = OB.pack_c(x)
        assert np.array_equal(OB.unpack_c(q, 96, 64).double().numpy(), OB.unpack_np(q.numpy(), 96, 64))


def test_hand_vectors():
    x = torch.zeros(32, 32)
    row = torch.tensor([1.0, -1.0, 0.5, 0.25, 1.5, 1.984375, 2.0 ** -6, 3 * 2.0 ** -8,
                        0.0, -0.0, 1.0 + 2 ** -7, 1.0 + 3 * 2 ** -7, 2 ** -7, 1e-45, 0.75, -0.5])
    x[0, :16] = row
    q = OB.pack_c(x).numpy()
    assert q[0] == 127  # max exponent: 1.984375 has biased exponent 127
    mags = q[64:80] & 0x7F
    signs = q[64:80] >> 7
    # m = RNE(|x| * 2^(133 - 127)) = RNE(64 |x|), saturated at 127
    expect = [64, 64, 32, 16, 96, 127, 1, 0, 0, 0, 64, 66, 0, 0, 48, 32]
    # 3*2^-8 * 64 = 0.75 -> 1 (RNE); 1 + 2^-7 -> 64.5 -> 64 (tie to even); 1 + 3*2^-7 -> 65.5 -> 66
    expect[7] = 1
    assert mags.tolist() == expect
    assert signs.tolist() == [0, 1, 0, 0, 0, 0, 0, 0, 0, 1, 0, 0, 0, 0, 0, 1]
    back = OB.unpack_np(q, 32, 32)[0, :16]
    assert back[0] == 1.0 and back[5] == 127 / 64 and back[11] == 66 / 64


def test_round_trip_bounds():
    x = torch.randn(64, 64, generator=torch.Generator().manual_seed(7)) * 0.02
    q = OB.pack_np(x.numpy())
    y = OB.unpack_np(q, 64, 64)
    # per face row, error <= half a quantum 2^(e-133), or the saturation gap
    tile_e = q.reshape(-1, 1088)[:, :64]
    assert np.abs(y - x.numpy()).max() <= 2.0 ** (int(tile_e.max()) - 133)
    # canonical blocks re-encode to themselves
    assert np.array_equal(OB.pack_np(y.astype(np.float32)), q)


# ---------------------------------------------------------------------------
# the library's host codec (no GPU needed: host functions of libttlhip.so)


def _lib_available():
    try:
        from ttlhip import _lib
        _lib.load()
        return True
    except Exception:
        return False


needs_lib = pytest.mark.skipif(not _lib_available(), reason="libttlhip.so not built")


@needs_lib
def test_library_host_codec_matches_oracle():
    from ttlhip import kernels as K
    for seed, scale in ((0, 0.02), (1, 1.0), (2, 1e-33), (3, 1e35)):
        x = torch.randn(64, 96, generator=torch.Generator().manual_seed(seed)) * scale
        q = K.bfp8_pack_host(x)
        assert torch.equal(q, OB.pack_c(x))
        assert torch.equal(K.bfp8_unpack_host(q, 64, 96).view(torch.int16),
                           OB.unpack_c(q, 64, 96).view(torch.int16))


@needs_lib
def test_library_host_decode_brute_force():
    from ttlhip import kernels as K
    # a 32 x 2048 matrix whose 64 tiles enumerate every (exponent, byte) pair
    q = np.zeros(64 * 1088, dtype=np.uint8).reshape(64, 1088)
    for t in range(64):
        for r in range(32):
            for c in range(32):
                f = (r // 16) * 2 + c // 16
                e = (t * 4 + f) % 256
                q[t, 16 * f + r % 16] = e
                q[t, 64 + 256 * f + 16 * (r % 16) + c % 16] = ((r % 16) * 16 + c % 16) % 256
    qt = torch.from_numpy(q.ravel().copy())
    got = K.bfp8_unpack_host(qt, 32, 64 * 32).float().double().numpy()
    assert np.array_equal(got, OB.unpack_np(q.ravel(), 32, 64 * 32))


@needs_lib
def test_library_pack_rejects_non_finite():
    from ttlhip import kernels as K
    x = torch.zeros(32, 32)
    x[3, 4] = float("inf")
    with pytest.raises(ValueError, match="inf or NaN"):
        K.bfp8_pack_host(x)
