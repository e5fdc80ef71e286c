"""Shared helpers for the test-suite (seeded CPU inputs, tolerance checks)."""

from __future__ import annotations

import torch


def randn(shape, dtype=torch.float32, seed=0, mean=0.0, std=1.0, gen=None):
    """Seeded CPU normal draw (identical on every host), cast to dtype."""
    g = gen if gen is not None else torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std + mean).to(dtype)


def bf16_flip_check(actual: torch.Tensor, expected: torch.Tensor, rate: float = 1e-5, atol: float = 1e-2):
    """bf16 RMSNorm parity against the oracle's bf16 result.

    Elements must be equal bit for bit except for summation-order flips.  The
    kernel sums x^2 in another order than torch's CPU sum, so `inv` can land
    an fp32 ulp or two away; an element then flips when x*inv sits that close
    to a bf16 rounding midpoint (~2^-16 relative), one bf16 ulp of the first
    rounding point dt(x*inv), which the weight multiply and the second
    rounding can carry to two ulps of y.  Measured: 185 of 33.5M elements
    (5.5e-6) at [16384, 2048].  Allowed: at most rate*numel flips plus a
    Poisson margin of 4 standard deviations and 3 (so small tensors are not
    failed by one or two flips), each within 2^-6 |e| of the oracle.  A
    systematically wrong inv (an approximate rsqrt in every row) flips
    several times more often; the inverse square root itself is pinned bit for
    bit by the rmsnorm_inv golden rows.  Elements with |e| < 0.5, where two
    ulps are below it, also meet the north-star `atol`.
    Returns (max_abs_err, n_diff)."""
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    assert a.shape == e.shape
    diff = (a - e).abs()
    flipped = diff > 0
    n_diff = int(flipped.sum())
    lam = rate * a.numel()
    assert n_diff <= lam + 4.0 * lam ** 0.5 + 3, f"{n_diff} of {a.numel()} elements differ"
    assert bool((diff[flipped] <= 2.0 ** -6 * e.abs()[flipped] + 1e-30).all()), "a flip exceeds two ulps"
    small = e.abs() < 0.5
    if bool(small.any()):
        assert float(diff[small].max()) <= atol
    return float(diff.max()) if a.numel() else 0.0, n_diff
