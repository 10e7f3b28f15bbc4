"""Tensor comparison helpers with the names and behaviour of the reference's
python/utils/correctness.py: Pearson correlation, allclose with a report, and
distances in units of least precision (ULP, Goldberg's definition).

All comparisons run on host tensors; ttnn tensors are converted first.
"""

from __future__ import annotations

from typing import Tuple

import torch

# significand bits (excluding the implicit one) and minimum normal exponent
_FORMAT = {
    torch.float64: (52, -1022),
    torch.float32: (23, -126),
    torch.float16: (10, -14),
    torch.bfloat16: (7, -126),
}
# largest ULP distance that still means "same order of magnitude"
_MEANINGFUL_ULP = {torch.float64: 2 ** 52, torch.float32: 2 ** 23, torch.float16: 2 ** 10,
                   torch.bfloat16: 2 ** 7}


def _host(t) -> torch.Tensor:
    if hasattr(t, "to_torch") and not isinstance(t, torch.Tensor):
        t = t.to_torch()
    return t.detach().cpu()


def assert_pcc(golden, actual, threshold: float = 0.99) -> None:
    """Raises AssertionError unless the Pearson correlation of the flattened
    tensors is at least `threshold` (correctness.py:12-28)."""
    g = _host(golden).flatten().to(torch.float64)
    a = _host(actual).flatten().to(torch.float64)
    pcc = float(torch.corrcoef(torch.stack([g, a]))[0, 1])
    assert pcc >= threshold, f"Expected pcc {pcc} >= {threshold}\ngolden:\n{golden}\nactual:\n{actual}"


def assert_allclose(actual, expected, rtol: float = 1e-5, atol: float = 1e-8,
                    verbose: bool = True) -> None:
    """torch.allclose with an error report: shape mismatch, then |a - e| <=
    atol + rtol |e| elementwise; the failure text gives max / mean absolute
    and relative errors and where the worst ones are (correctness.py:31-117)."""
    a, e = _host(actual), _host(expected)
    if a.shape != e.shape:
        raise AssertionError(f"Shape mismatch: actual {a.shape} vs expected {e.shape}")
    if torch.allclose(a, e, rtol=rtol, atol=atol):
        return
    diff = (a - e).abs()
    rel = diff / (e.abs() + 1e-10)
    max_abs, max_rel = float(diff.max()), float(rel.max())
    if not verbose:
        raise AssertionError(f"Tensors not close: max_abs_error={max_abs:.6e}, "
                             f"max_rel_error={max_rel:.6e}, rtol={rtol}, atol={atol}")
    ia = torch.unravel_index(diff.flatten().argmax(), a.shape)
    ir = torch.unravel_index(rel.flatten().argmax(), a.shape)
    at = tuple(int(c) for c in ia)
    rt = tuple(int(c) for c in ir)
    bad = int((diff > atol + rtol * e.abs()).sum())
    raise AssertionError(
        "\nTensor comparison failed!\n\nError Statistics:\n"
        f"  Absolute Error:\n    Mean: {float(diff.mean()):.6e}\n    Max:  {max_abs:.6e} at {at}\n"
        f"          actual={float(a[ia]):.6f}, expected={float(e[ia]):.6f}\n\n"
        f"  Relative Error:\n    Mean: {float(rel.mean()):.6e}\n    Max:  {max_rel:.6e} at {rt}\n"
        f"          actual={float(a[ir]):.6f}, expected={float(e[ir]):.6f}\n\n"
        f"Thresholds:\n  rtol: {rtol}\n  atol: {atol}\n\nShape: {a.shape}\n"
        f"Mismatched elements: {bad} / {a.numel()}\n")


def ulp(x: torch.Tensor) -> torch.Tensor:
    """Unit of least precision of every element, in x's dtype: the distance
    from |x| to the next representable number above it (so for a power of two
    the gap above, and at the format's maximum the gap below it, which is the
    same size) (correctness.py:142-165)."""
    if x.dtype not in _FORMAT:
        raise TypeError(f"ulp() takes a floating-point tensor, got {x.dtype}")
    p, emin = _FORMAT[x.dtype]
    ax = x.abs().to(torch.float64)
    _, exp = torch.frexp(ax)  # |x| = m 2^exp, m in [0.5, 1)
    # zero and subnormals: the spacing of the subnormal range
    e = torch.where(ax == 0, torch.full_like(exp, emin, dtype=torch.int64),
                    torch.clamp(exp.to(torch.int64) - 1, min=emin))
    out = torch.ldexp(torch.ones_like(e, dtype=torch.float64), (e - p).to(torch.float64))
    out = torch.where(torch.isfinite(x), out, torch.full_like(out, float("nan")))
    return out.to(x.dtype)


def _same_nonfinite(golden: torch.Tensor, calculated: torch.Tensor) -> bool:
    """NaNs at the same places and infinities at the same places with the
    same signs (correctness.py:120-139)."""
    if not torch.equal(torch.isnan(golden), torch.isnan(calculated)):
        return False
    gi, ci = torch.isinf(golden), torch.isinf(calculated)
    if not torch.equal(gi, ci):
        return False
    return torch.equal(golden[gi], calculated[ci])


def comp_ulp(golden, calculated, ulp_threshold, allow_nonfinite: bool = True) -> Tuple[bool, str]:
    """(passed, message): the largest |calculated - golden| / ULP(golden),
    with ULP taken in calculated's dtype (so a higher-precision golden can
    measure sub-ULP errors), against `ulp_threshold` (correctness.py:168-210)."""
    golden, calculated = _host(golden), _host(calculated)
    if golden.numel() == 0 and calculated.numel() == 0:
        return True, "Both tensors are empty"
    if not allow_nonfinite and not bool(torch.isfinite(calculated).all()):
        return False, "Calculated tensor contains non-finite values"
    if not _same_nonfinite(golden, calculated):
        return False, "Tensors are not finite at the same positions"
    keep = torch.isfinite(golden)
    golden = torch.where(keep, golden, torch.zeros_like(golden))
    calculated = torch.where(keep, calculated, torch.zeros_like(calculated))
    u = ulp(golden.to(calculated.dtype))
    if golden.dtype != calculated.dtype:
        calculated = calculated.to(golden.dtype)
        u = u.to(golden.dtype)
    delta = torch.max((calculated - golden).abs() / u)
    return bool(delta <= ulp_threshold), f"Max ULP Delta: {delta}"


def assert_with_ulp(expected_result, actual_result, ulp_threshold=10, allow_nonfinite=False):
    """Asserts that the tensors are within `ulp_threshold` ULP of each other
    (ULP of the expected values); returns (passed, message)
    (correctness.py:213-293)."""
    expected_result, actual_result = _host(expected_result), _host(actual_result)
    assert list(expected_result.shape) == list(actual_result.shape), (
        f"list(expected_result.shape)={list(expected_result.shape)} vs "
        f"list(actual_result.shape)={list(actual_result.shape)}")
    meaningful = _MEANINGFUL_ULP.get(expected_result.dtype, _MEANINGFUL_ULP[torch.float32])
    if ulp_threshold > meaningful:
        print(f"ULP threshold {ulp_threshold} is greater than the maximum meaningful ULP threshold "
              f"of {meaningful} for dtype {expected_result.dtype}")
    passed, message = comp_ulp(expected_result, actual_result, ulp_threshold, allow_nonfinite)
    assert passed, message
    return passed, message
