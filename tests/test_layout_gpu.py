"""ttlh_tilize / ttlh_untilize on the MI355X against the oracle's
restatement (tilize_ref / untilize_ref): bit-exact for bf16 and f32, round
trips, strided row-major sides, the drop-in ttnn interop helpers, and the
argument checks."""

import pytest
import torch

import ttnn
from oracle import tile_ops as O
from ttlhip import kernels as K

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(32, 32), (96, 64), (4096, 4096), (64, 4160)])
def test_tilize_matches_oracle(dtype, shape):
    x = O.seeded(shape, "normal", 71, dtype)
    d = K.tilize(x.cuda())
    torch.cuda.synchronize()
    assert torch.equal(d.cpu(), O.tilize_ref(x))
    back = K.untilize(d, *shape)
    torch.cuda.synchronize()
    assert torch.equal(back.cpu(), x)


def test_strided_row_major_sides():
    base = O.seeded((128, 200), "normal", 72)  # row pitch 200 (400 bytes, 16-byte aligned)
    x = base[:, :160].cuda()
    full = base.cuda()
    d = K.tilize(full[:, :160])
    assert torch.equal(d.cpu(), O.tilize_ref(base[:, :160].contiguous()))
    out = torch.zeros(128, 200, dtype=torch.bfloat16, device="cuda")
    K.untilize(d, 128, 160, out=out[:, :160])
    torch.cuda.synchronize()
    assert torch.equal(out[:, :160].cpu(), base[:, :160]) and not out[:, 160:].any()
    assert x.shape == (128, 160)


def test_ttnn_tiled_data_round_trip():
    x = O.seeded((256, 128), "uniform", 73)
    t = ttnn.from_torch(x, layout=ttnn.TILE_LAYOUT)
    d = t.tiled_data()
    assert torch.equal(d.cpu(), O.tilize_ref(x))
    back = ttnn.from_tiled_data(d.cpu(), (256, 128))
    assert torch.equal(back.to_torch(), x) and back.layout is ttnn.TILE_LAYOUT
    q = ttnn.from_torch(x.float(), dtype=ttnn.bfloat8_b)
    assert q.tiled_data().dtype == torch.uint8 and q.tiled_data().numel() == 32 * 1088


def test_layout_argument_checks():
    with pytest.raises(ValueError, match="multiples of 32"):
        K.tilize(torch.zeros(48, 32, dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(ValueError, match="elements"):
        K.untilize(torch.zeros(100, dtype=torch.bfloat16, device="cuda"), 32, 32)
