"""RMSNorm CPU oracle -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates ``RMSNorm._norm`` / ``RMSNorm.forward`` (rmsnorm/original.py:38,
51-52) and the weight-free two-scan kernel (rmsnorm/original.py:55-78).
"""

from __future__ import annotations

import torch


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``(x.float() * rsqrt(mean(x^2) + eps)).type_as(x) * weight`` on the CPU.

    rmsnorm/original.py:38 (``_norm``) and :51-52 (``forward``): the
    normalised value is rounded to x's dtype before the weight multiply, and
    the product is rounded again (torch promotes bf16*bf16 through fp32).
    ``rsqrt`` is evaluated as a correctly rounded ``1/sqrt`` in fp32.
    """
    x = x.detach().cpu()
    weight = weight.detach().cpu()
    xf = x.float()
    ms = xf.pow(2).mean(-1, keepdim=True)
    inv = 1.0 / torch.sqrt(ms + eps)
    normed = (xf * inv).to(x.dtype)
    return (normed.float() * weight.float()).to(torch.promote_types(x.dtype, weight.dtype))


def rmsnorm_grads(x: torch.Tensor, weight: torch.Tensor, dy: torch.Tensor, eps: float = 1e-6):
    """``(dx, dweight)`` of ``rmsnorm`` for the output gradient ``dy``, by torch
    autograd on the CPU through the same operations (rmsnorm/original.py:38,
    51-52), as the reference module's backward computes them."""
    x = x.detach().cpu().clone().requires_grad_(True)
    weight = weight.detach().cpu().clone().requires_grad_(True)
    xf = x.float() if x.dtype != torch.float64 else x
    normed = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).type_as(x)
    out = normed * weight
    out.backward(dy.detach().cpu().to(out.dtype))
    return x.grad, weight.grad


def rmsnorm_fp64(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """The same formula with every step in fp64 and no intermediate rounding."""
    xd = x.detach().cpu().double()
    inv = 1.0 / torch.sqrt(xd.pow(2).mean(-1, keepdim=True) + eps)
    return xd * inv * weight.detach().cpu().double()


def rmsnorm_noweight(a: torch.Tensor, eps: float = 1e-12) -> torch.Tensor:
    """fp32 ``A * rsqrt(sum(A^2)/N + eps)`` (rmsnorm/original.py:69-75, eps 1e-12 at :73)."""
    a = a.detach().cpu().float()
    inv = 1.0 / torch.sqrt(a.pow(2).sum(-1, keepdim=True) / a.shape[-1] + eps)
    return a * inv
