"""Drop-in for the helpers tt-lang's hardware tests import
(`test/ttlang_test_utils.py` in the reference): feature probes, device tensor
creation in "DRAM" / "L1", and tensor comparisons with the same names,
arguments and error behaviour, backed by this build's `ttnn`.

On the MI355X there is one memory (HBM) for every tensor: `to_dram` and
`to_l1` both return a TILE_LAYOUT bf16 device tensor.  "Hardware available"
means a GPU is visible and the kernel library is built; without one, tests
that need the device skip, as the reference's do without a Tenstorrent card.
"""

from __future__ import annotations

import sys

import torch


def is_ttnn_available() -> bool:
    """The drop-in ttnn is always importable (test/ttlang_test_utils.py:68-78)."""
    try:
        import ttnn  # noqa: F401
    except ImportError:
        return False
    return True


def is_hardware_available() -> bool:
    """A GPU to run kernels on (test/ttlang_test_utils.py:81-93)."""
    return bool(torch.cuda.is_available())


def require_ttnn() -> None:
    """Exit the script quietly when ttnn is missing (test/ttlang_test_utils.py:96-100)."""
    if not is_ttnn_available():
        print("TTNN not available - exiting")
        sys.exit(0)


def require_hardware(message: str = "Skipping test - no hardware available") -> None:
    """Exit the script quietly without a device (test/ttlang_test_utils.py:103-114)."""
    if not is_hardware_available():
        print(message)
        sys.exit(0)


def to_dram(torch_tensor: torch.Tensor, device=None):
    """bf16 TILE_LAYOUT device tensor (test/ttlang_test_utils.py:122-141)."""
    import ttnn

    return ttnn.from_torch(torch_tensor, dtype=ttnn.bfloat16, layout=ttnn.TILE_LAYOUT,
                           device=device, memory_config=ttnn.DRAM_MEMORY_CONFIG)


def to_l1(torch_tensor: torch.Tensor, device=None):
    """Same as to_dram: the MI355X has no separate L1 tensor placement
    (test/ttlang_test_utils.py:144-171)."""
    import ttnn

    t = to_dram(torch_tensor, device)
    return ttnn.to_memory_config(t, memory_config=ttnn.L1_MEMORY_CONFIG)


def _flat(t) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) and hasattr(t, "to_torch"):
        t = t.to_torch()
    return t.detach().cpu().flatten().to(torch.float64)


def assert_pcc(golden, actual, threshold: float = 0.99) -> float:
    """Pearson correlation >= threshold; two constant tensors pass when equal
    (test/ttlang_test_utils.py:174-223).  Returns the correlation."""
    g, a = _flat(golden), _flat(actual)
    gs, as_ = float(g.std()), float(a.std())
    if gs == 0 and as_ == 0:
        if torch.allclose(g, a):
            return 1.0
        raise AssertionError(f"Both tensors are constant but differ: golden={float(g[0])}, "
                             f"actual={float(a[0])}")
    if gs == 0 or as_ == 0:
        raise AssertionError(f"Cannot compute PCC: one tensor is constant "
                             f"(golden std={gs}, actual std={as_})")
    gc, ac = g - g.mean(), a - a.mean()
    pcc = float((gc * ac).sum() / torch.sqrt((gc * gc).sum() * (ac * ac).sum()))
    if pcc < threshold:
        raise AssertionError(f"PCC {pcc:.6f} is below threshold {threshold}. "
                             f"Golden: mean={float(g.mean()):.4f}, std={gs:.4f}. "
                             f"Actual: mean={float(a.mean()):.4f}, std={as_:.4f}.")
    return pcc


def assert_allclose(actual, expected, rtol: float = 1e-5, atol: float = 1e-8,
                    verbose: bool = True) -> None:
    """torch.allclose with a report of the largest difference
    (test/ttlang_test_utils.py:226-262)."""
    if not isinstance(actual, torch.Tensor):
        actual = actual.to_torch()
    if not isinstance(expected, torch.Tensor):
        expected = expected.to_torch()
    if torch.allclose(actual, expected, rtol=rtol, atol=atol):
        return
    diff = (actual - expected).abs()
    msg = (f"Tensors not close: max_diff={float(diff.max()):.6e}, "
           f"mean_diff={float(diff.float().mean()):.6e}, rtol={rtol}, atol={atol}")
    if verbose:
        i = int(diff.argmax())
        msg += (f"\nMax diff at flat index {i}: actual={float(actual.flatten()[i]):.6e}, "
                f"expected={float(expected.flatten()[i]):.6e}")
    raise AssertionError(msg)
