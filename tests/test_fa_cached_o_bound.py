"""CPU check of the bound behind the standalone JVP's use of the cached O.

The JVP-from-LSE kernel (csrc/fa_jvp.hip) writes tO = G/l - (r/l) O with the
cached 16-bit O only for rows where |r/l| * max(max|O|, 1) <= kCachedOBound
(1.0, csrc/fa_common.h); other rows are redone with U = P v recomputed, whose
tO is tO6 = G/l - (r/l) (U/l).  This emulates every rounding point of both
formulas in fp64 (16-bit E and H in the products and in l and r, the cached O
as the forward kernel makes it: 16-bit E relative to the first 32 keys' max
over the fp32 sum, rounded to 16 bits) and checks that on rows under the bound
the cached-O formula moves tO by well under the bf16/fp16 tolerances of the
GPU tests, while peaked softmaxes do produce rows past the bound (so the
recompute path is exercised, and the bound is not vacuous).
"""

import pytest
import torch

BOUND = 1.0  # kCachedOBound
TOL = {torch.bfloat16: (3e-2, 3e-2), torch.float16: (3e-3, 1e-2)}


def rnd(x, dtype):
    return x.to(dtype).to(torch.float64)


def emulate(n, d, scale, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v, tq, tk, tv = (rnd(torch.randn(n, d, generator=g, dtype=torch.float64), dtype) for _ in range(6))
    s = scale * q @ k.T
    lse = torch.logsumexp(s, -1, keepdim=True)
    ts = scale * (tq @ k.T + q @ tk.T)
    p = torch.exp(s - lse)
    exact = p @ tv + (p * ts) @ v - (p * ts).sum(-1, keepdim=True) * (p @ v)
    e = rnd(p, dtype)
    h = rnd(p * ts, dtype)
    l, r = e.sum(-1, keepdim=True), h.sum(-1, keepdim=True)
    gacc = e @ tv + h @ v
    m32 = s[:, :32].max(-1, keepdim=True).values
    ef = torch.exp(s - m32)
    o_cached = rnd((rnd(ef, dtype) @ v) / ef.sum(-1, keepdim=True), dtype)
    t5 = gacc / l - (r / l) * o_cached
    t6 = gacc / l - (r / l) * ((e @ v) / l)
    crit = (r / l).abs().squeeze(-1) * o_cached.abs().max(-1).values.clamp(min=1.0)
    return exact, t5, t6, crit


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_rows_under_the_bound_stay_well_inside_the_tolerance(dtype):
    atol, rtol = TOL[dtype]
    worst, fast = 0.0, 0
    for seed, (n, d, scale) in enumerate(((256, 64, 64 ** -0.5), (512, 128, 128 ** -0.5), (256, 32, 0.3),
                                          (256, 128, 0.2), (128, 64, 0.5), (512, 32, 1.0))):
        exact, t5, t6, crit = emulate(n, d, scale, dtype, seed)
        under = crit <= BOUND
        fast += int(under.sum())
        if under.any():
            added = ((t5 - t6).abs() / (atol + rtol * exact.abs()))[under]
            worst = max(worst, added.max().item())
    assert fast > 0
    assert worst < 0.3, worst


def test_scale_one_over_sqrt_d_never_reaches_the_bound():
    # Fewer keys average less: the largest products are ~0.8 at 256-512 keys
    # with D = 32-64 and ~0.4 at 4096 keys with D = 128.
    for seed, (n, d) in enumerate(((512, 64), (512, 128), (256, 32), (2048, 128))):
        *_, crit = emulate(n, d, d ** -0.5, torch.bfloat16, seed)
        assert crit.max().item() < BOUND


def test_peaked_softmax_rows_exceed_the_bound_and_need_the_recompute():
    exact, t5, t6, crit = emulate(64, 32, 1.0, torch.bfloat16, 7)
    over = crit > BOUND
    assert over.float().mean().item() > 0.5
    atol, rtol = TOL[torch.bfloat16]
    err5 = ((t5 - exact).abs() / (atol + rtol * exact.abs()))[over].max().item()
    err6 = ((t6 - exact).abs() / (atol + rtol * exact.abs()))[over].max().item()
    assert err6 < err5
