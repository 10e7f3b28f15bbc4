"""Tilized element order (TILE_LAYOUT storage) on the CPU: the oracle's
reshape / permute restatement pinned by the scalar position formula of
include/ttlhip.h and by the bfloat8_b codec's byte layout (an independent
formulation of the same face order), plus the layout rules of the drop-in
`ttnn` (the reference's compiled path rejects non-tilized tensors,
python/ttl/ttl_api.py:489-506).

The face order itself comes from tt-metal (not vendored in the reference):
"parity unpinned" against it beyond the 16x16 face split the bfloat8_b size
implies (python/ttl/dtype_utils.py:174-175: 64 shared exponents = 4 faces x
16 rows).
"""

import pytest
import torch

import kernel_lib as KL
import ttl
import ttnn
from oracle import bfp8 as OB, tile_ops as O


def _pos(i, j, cols):
    t = (i // 32) * (cols // 32) + j // 32
    return 1024 * t + 256 * (2 * ((i % 32) // 16) + (j % 32) // 16) + 16 * (i % 16) + j % 16


def test_tilize_ref_matches_position_formula():
    rows, cols = 96, 64
    x = torch.arange(rows * cols, dtype=torch.float32).reshape(rows, cols)
    d = O.tilize_ref(x)
    for i in range(rows):
        for j in range(cols):
            assert d[_pos(i, j, cols)] == x[i, j]
    assert torch.equal(O.untilize_ref(d, rows, cols), x)


def test_tilize_ref_matches_bfloat8_b_byte_order():
    # every face row of values 64..127 shares exponent 133, so each element
    # byte of a bfloat8_b tile is the value itself, stored in face order
    rows, cols = 64, 96
    i = torch.arange(rows).view(-1, 1)
    j = torch.arange(cols).view(1, -1)
    x = (64 + (i * 7 + j * 3) % 64).float()
    q = OB.pack_np(x.numpy())
    tiles = torch.from_numpy(q.reshape(-1, 1088)[:, 64:].copy()).reshape(-1).float()
    assert torch.equal(tiles, O.tilize_ref(x))


def test_layout_tags_and_kernel_check():
    t = ttnn.from_torch(torch.zeros(64, 64), layout=ttnn.ROW_MAJOR_LAYOUT)
    assert t.layout is ttnn.ROW_MAJOR_LAYOUT
    tt = ttnn.to_layout(t, ttnn.TILE_LAYOUT)
    assert tt.layout is ttnn.TILE_LAYOUT and tt._tensor is t._tensor
    assert ttnn.untilize(tt).layout is ttnn.ROW_MAJOR_LAYOUT
    assert ttnn.rand((32, 32), layout=ttnn.ROW_MAJOR_LAYOUT).layout is ttnn.ROW_MAJOR_LAYOUT
    k = KL.make_eltwise_add(ttl)
    a = ttnn.Tensor(torch.zeros(64, 64))
    b = ttnn.Tensor(torch.zeros(64, 64), layout=ttnn.ROW_MAJOR_LAYOUT)
    with pytest.raises(ValueError, match="TTNN interop requires tilized tensors, but tensor 1"):
        k.trace(a, b, ttnn.Tensor(torch.zeros(64, 64)))
