"""Shared helpers for the test-suite (seeded CPU inputs, tolerance checks)."""

from __future__ import annotations

import torch


def randn(shape, dtype=torch.float32, seed=0, mean=0.0, std=1.0, gen=None):
    """Seeded CPU normal draw (identical on every host), cast to dtype."""
    g = gen if gen is not None else torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g, dtype=torch.float32) * std + mean).to(dtype)


def bf16_flip_check(actual: torch.Tensor, expected: torch.Tensor, atol=1e-2, max_flip_frac=1e-3):
    """bf16 RMSNorm parity: |a-e| <= atol + 2^-6 |e| everywhere, and at most
    `max_flip_frac` of the elements differ at all.

    A differing element comes from the fp32 summation order of the sum of
    squares: `inv` one fp32 ulp away flips the first rounding point dt(x*inv)
    by one bf16 ulp (2^-7 relative at most), which the weight multiply and the
    second rounding can carry to two ulps of y, i.e. 2^-6 |y|.
    Returns (max_abs_err, n_diff)."""
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    torch.testing.assert_close(a, e, atol=atol, rtol=2.0 ** -6)
    n_diff = int((a != e).sum())
    assert n_diff <= max_flip_frac * a.numel(), f"{n_diff} of {a.numel()} elements differ"
    return float((a - e).abs().max()) if a.numel() else 0.0, n_diff
