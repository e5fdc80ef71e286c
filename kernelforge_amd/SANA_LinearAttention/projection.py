"""SANA projection GEMMs on the hand-written gfx950 kernel (``kf_proj_gemm``).

- ``linear(x, weight, bias=None)`` -- ``y = x W^T (+ b)`` with
  ``torch.nn.Linear``'s ``weight[N, K]``; the modules call it for both
  projections, straight on their parameters (no transposed copies).
- ``qkv_projection(batch, seq_len, channels, dtype)`` -- the no-bias QKV
  projection factory taking the prepacked ``WeightT[C, 3C]``
  (SANA_LinearAttention/custom.py:23-85).
- ``output_projection(batch, seq_len, channels, dtype)`` -- the bias-fused
  output projection factory taking ``WeightT[C, C]`` and ``Bias[C]``
  (SANA_LinearAttention/custom.py:457-523).

Arithmetic: 16-bit (or fp32) operands, fp32 products and sums on the MFMA
pipe, the bias added in fp32, one round-to-nearest-even to the input dtype --
the reference's ``T.gemm`` into an fp32 fragment followed by
``T.Cast(dtype, acc + float(bias))``.  There is no CPU path: CPU tensors are
rejected.
"""

from __future__ import annotations

from typing import Optional

import torch

from .. import _lib

_DTYPES = (torch.bfloat16, torch.float16, torch.float32)

# torch dtype <-> reference dtype string (SANA_LinearAttention/custom.py:16-20).
TORCH_DTYPES = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float"}


def _rows(x: torch.Tensor, k: int) -> tuple[torch.Tensor, int]:
    """x as a [rows, k] matrix with unit column stride and a uniform row stride
    that keeps 16-byte row alignment; copies only when no such view exists."""
    x2 = x.reshape(-1, k)
    esize = x.element_size()
    ok = (x2.stride(1) == 1 and (x2.shape[0] <= 1 or x2.stride(0) >= k)
          and (x2.stride(0) * esize) % 16 == 0 and x2.data_ptr() % 16 == 0)
    if not ok:
        x2 = x2.contiguous()
        if x2.data_ptr() % 16:
            x2 = x2.clone()
    return x2, (x2.stride(0) if x2.shape[0] > 1 else k)


def _launch(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], layout: int, n: int,
            out: Optional[torch.Tensor]) -> torch.Tensor:
    k = x.shape[-1]
    if x.dtype not in _DTYPES:
        raise ValueError(f"projection dtype must be one of {_DTYPES}, got {x.dtype}")
    if weight.dtype != x.dtype or (bias is not None and bias.dtype != x.dtype):
        raise ValueError(f"weight and bias must have x's dtype {x.dtype}")
    _lib.require_gpu(x, weight, bias)
    if bias is not None and bias.shape != (n,):
        raise ValueError(f"bias must be [{n}], got {tuple(bias.shape)}")
    if n % 8 or k % 8:
        return _launch_padded(x, weight, bias, layout, n, out)
    weight = weight.contiguous()
    if weight.data_ptr() % 16:
        weight = weight.clone()
    if bias is not None:
        bias = bias.contiguous()
    x2, ldx = _rows(x, k)
    if out is None:
        out = torch.empty(*x.shape[:-1], n, device=x.device, dtype=x.dtype)
    elif out.shape != (*x.shape[:-1], n) or out.dtype != x.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of the result's shape and dtype")
    m = x2.shape[0]
    rc = _lib.load().kf_proj_gemm(_lib.ptr(x2), _lib.ptr(weight), _lib.ptr(bias), _lib.ptr(out), m, n, k, ldx, n,
                                  layout, _lib.kf_dtype(x.dtype), _lib.stream_of(x))
    _lib.check(rc, "kf_proj_gemm")
    return out


def _launch_padded(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], layout: int, n: int,
                   out: Optional[torch.Tensor]) -> torch.Tensor:
    """The GEMM for widths that are not multiples of 8 (its 16-byte operand
    rows need them): x, the weight and the bias are copied into zero-padded
    buffers of the next multiples of 8, the kernel runs on those, and the
    first n output columns are kept.  The padded products are exact zeros, so
    the result equals an unpadded GEMM's."""
    k = x.shape[-1]
    kp, np_ = -(-k // 8) * 8, -(-n // 8) * 8
    xp = x.new_zeros(*x.shape[:-1], kp)
    xp[..., :k] = x
    if layout == _lib.KF_WEIGHT_NK:
        wp = weight.new_zeros(np_, kp)
        wp[:n, :k] = weight
    else:
        wp = weight.new_zeros(kp, np_)
        wp[:k, :n] = weight
    bp = None
    if bias is not None:
        bp = bias.new_zeros(np_)
        bp[:n] = bias
    y = _launch(xp, wp, bp, layout, np_, None)[..., :n]
    if out is None:
        return y.contiguous()
    if out.shape != y.shape or out.dtype != x.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of the result's shape and dtype")
    return out.copy_(y)


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None, *,
           out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``x[..., K] @ weight[N, K]^T (+ bias[N])`` -> ``[..., N]`` in x's dtype
    (``torch.nn.functional.linear`` semantics, hand-written MFMA GEMM)."""
    if weight.dim() != 2 or weight.shape[1] != x.shape[-1]:
        raise ValueError(f"weight must be [N, {x.shape[-1]}], got {tuple(weight.shape)}")
    return _launch(x, weight, bias, _lib.KF_WEIGHT_NK, weight.shape[0], out)


def linear_t(x: torch.Tensor, weight_t: torch.Tensor, bias: Optional[torch.Tensor] = None, *,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``x[..., K] @ weight_t[K, N] (+ bias[N])`` -> ``[..., N]``: the same GEMM
    on the reference's prepacked ``WeightT`` layout."""
    if weight_t.dim() != 2 or weight_t.shape[0] != x.shape[-1]:
        raise ValueError(f"WeightT must be [{x.shape[-1]}, N], got {tuple(weight_t.shape)}")
    return _launch(x, weight_t, bias, _lib.KF_WEIGHT_KN, weight_t.shape[1], out)


def _torch_dtype(dtype: str) -> torch.dtype:
    dtypes = {v: k for k, v in TORCH_DTYPES.items()}
    if dtype not in dtypes:
        raise ValueError(f"unsupported projection dtype: {dtype}")
    return dtypes[dtype]


class _QKVProjection:
    """``kernel(X[B, N, C], WeightT[C, 3C]) -> QKV[B, N, 3C]`` for one shape
    (SANA_LinearAttention/custom.py:34-80)."""

    def __init__(self, batch: int, seq_len: int, channels: int, dtype: torch.dtype):
        self.shape = (batch, seq_len, channels)
        self.channels = channels
        self.dtype = dtype

    def __call__(self, X: torch.Tensor, WeightT: torch.Tensor) -> torch.Tensor:
        if tuple(X.shape) != self.shape or X.dtype != self.dtype:
            raise ValueError(f"X must be {self.dtype} of shape {self.shape}, got {X.dtype} {tuple(X.shape)}")
        if tuple(WeightT.shape) != (self.channels, 3 * self.channels) or WeightT.dtype != self.dtype:
            raise ValueError(f"WeightT must be {self.dtype} of shape ({self.channels}, {3 * self.channels})")
        return linear_t(X, WeightT)


class _OutputProjection:
    """``kernel(X[B, N, C], WeightT[C, C], Bias[C]) -> Output[B, N, C]`` for one
    shape (SANA_LinearAttention/custom.py:469-523)."""

    def __init__(self, batch: int, seq_len: int, channels: int, dtype: torch.dtype):
        self.shape = (batch, seq_len, channels)
        self.channels = channels
        self.dtype = dtype

    def __call__(self, X: torch.Tensor, WeightT: torch.Tensor, Bias: torch.Tensor) -> torch.Tensor:
        c = self.channels
        if tuple(X.shape) != self.shape or X.dtype != self.dtype:
            raise ValueError(f"X must be {self.dtype} of shape {self.shape}, got {X.dtype} {tuple(X.shape)}")
        if tuple(WeightT.shape) != (c, c) or WeightT.dtype != self.dtype:
            raise ValueError(f"WeightT must be {self.dtype} of shape ({c}, {c})")
        if tuple(Bias.shape) != (c,) or Bias.dtype != self.dtype:
            raise ValueError(f"Bias must be {self.dtype} of shape ({c},)")
        return linear_t(X, WeightT, Bias)


def qkv_projection(batch: int, seq_len: int, channels: int, dtype: str = "bfloat16") -> _QKVProjection:
    """The no-bias QKV projection for one shape, taking ``WeightT[C, 3C]``
    (SANA_LinearAttention/custom.py:83-85)."""
    return _QKVProjection(batch, seq_len, channels, _torch_dtype(dtype))


def output_projection(batch: int, seq_len: int, channels: int, dtype: str = "bfloat16") -> _OutputProjection:
    """The bias-fused output projection for one shape, taking ``WeightT[C, C]``
    and ``Bias[C]`` (SANA_LinearAttention/custom.py:457-523)."""
    return _OutputProjection(batch, seq_len, channels, _torch_dtype(dtype))
