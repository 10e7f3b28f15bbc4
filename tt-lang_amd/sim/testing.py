"""sim.testing.assert_pcc for tt-lang examples (python/sim/testing.py:11-21)."""

from ttnn import Tensor, isclose


def assert_pcc(tensor_a: Tensor, tensor_b: Tensor, rtol: float = 1e-5, atol: float = 1e-8) -> None:
    assert tensor_a.shape == tensor_b.shape, "Tensors must have the same shape"
    assert tensor_a.dtype == tensor_b.dtype, "Tensors must have the same dtype"
    close = isclose(tensor_a, tensor_b, rtol=rtol, atol=atol)
    assert close.to_torch().all().item(), "Tensor values are not close enough"
