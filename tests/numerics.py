"""Tolerance helpers shared by the parity tests."""

import os

import torch


def errors(actual: torch.Tensor, expected: torch.Tensor) -> tuple[float, float, float]:
    """(max-abs error, relative L2 error, max |expected|) in float64."""
    a, e = actual.double().cpu(), expected.double().cpu()
    diff = a - e
    max_abs = diff.abs().max().item() if diff.numel() else 0.0
    norm = e.norm().item()
    rel_l2 = diff.norm().item() / norm if norm > 0 else diff.norm().item()
    scale = e.abs().max().item() if e.numel() else 0.0
    return max_abs, rel_l2, scale


def assert_bf16_close(actual, expected, *, max_abs=1e-2, rel_l2=5e-3, what=""):
    """bf16 result against the float64/fp32 oracle on the same inputs.

    Bar: relative L2 error <= rel_l2 and max-abs error <= max_abs * max(1, max|expected|)
    (the max-abs bar scales with the tensor's magnitude because a bf16 result
    carries a relative rounding of 2^-9 per element).
    """
    assert torch.isfinite(actual.float()).all(), f"{what}: non-finite values"
    m, r, s = errors(actual, expected)
    bound = max_abs * max(1.0, s)
    log = os.environ.get("WMX_NUMERICS_LOG")
    if log:
        with open(log, "a") as f:
            f.write(f"{os.environ.get('PYTEST_CURRENT_TEST', '?').split(' ')[0]} {what} max_abs={m:.3e} rel_l2={r:.3e} scale={s:.2e}\n")
    assert m <= bound and r <= rel_l2, f"{what}: max_abs={m:.3e} (bound {bound:.3e}), rel_l2={r:.3e} (bound {rel_l2:.1e})"
