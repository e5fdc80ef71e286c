"""Shared helpers for the test-suite (seeded CPU inputs, tolerance checks)."""

from __future__ import annotations

import torch


def randn(shape, dtype=torch.float32, seed=0, mean=0.0, std=1.0, gen=None):
    """Seeded CPU normal draw (identical on every host), cast to dtype."""
    g = gen if gen is not None else torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std + mean).to(dtype)


def bf16_flip_check(actual: torch.Tensor, expected: torch.Tensor, max_flip_frac: float = 1e-6,
                    atol: float = 1e-2):
    """bf16 RMSNorm parity against the oracle's bf16 result.

    Elements equal bit for bit except at most ``max_flip_frac`` of them (at
    least one element is never granted: a 10-element tensor with cap 2e-5
    must match exactly).  A differing element comes from the fp32 summation
    order of the sum of squares: ``inv`` one fp32 ulp away flips the first
    rounding point dt(x*inv) by one bf16 ulp, which the weight multiply and
    the second rounding can carry to two ulps of y, so every differing
    element must lie within 2^-6 |e| (two bf16 ulps) of the oracle.  Elements
    that agree meet the north-star ``atol`` trivially; it is asserted over
    all elements with |e| < 0.5, where two ulps are below it.
    Returns (max_abs_err, n_diff)."""
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    assert a.shape == e.shape
    diff = (a - e).abs()
    flipped = diff > 0
    n_diff = int(flipped.sum())
    assert n_diff <= max_flip_frac * a.numel(), f"{n_diff} of {a.numel()} elements differ"
    assert bool((diff[flipped] <= 2.0 ** -6 * e.abs()[flipped] + 1e-30).all()), "a flip exceeds two ulps"
    small = e.abs() < 0.5
    assert float(diff[small].max()) <= atol if bool(small.any()) else True
    return float(diff.max()) if a.numel() else 0.0, n_diff
