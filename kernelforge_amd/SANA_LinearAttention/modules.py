"""LiteLA attention modules on the gfx950 kernels.

Mirrors the module API around the attention hot path:

- ``LiteLA`` -- the reference module's constructor and ``forward``
  (SANA_LinearAttention/original.py:65-145);
- ``CustomLiteLA`` -- the packed-QKV module bound to one input shape
  (SANA_LinearAttention/custom.py:391-454, exported there as ``CustomLiteLA``);
- ``JointLiteLA`` -- the same with a bias-fused output projection
  (SANA_LinearAttention/custom.py:526-592);
- ``qkv_projection`` -- the no-bias projection factory taking a prepacked
  ``WeightT[C, 3C]`` (SANA_LinearAttention/custom.py:83-85).

Data path of ``forward(x[B, N, C])``:

1. ``qkv = x @ Wqkv^T (+ b)`` -- a plain library GEMM (hipBLASLt through
   ``torch.nn.functional.linear``) into the packed ``[B, N, 3, C]`` layout.
2. ``qk_norm``: RMSNorm over the C channels of each token's q and k, in place
   in the packed buffer (``kf_rmsnorm_fwd_strided``, no copies).
3. ReLU linear attention (``kf_linattn_fwd``: split states on MFMA, fixed-order
   split reduction, MFMA output contraction), fp32 arithmetic.
4. ``y = out @ Wproj^T + b`` -- library GEMM with the bias in its epilogue.

Numerics: the attention always runs with the reference's ``fp32_attention``
semantics (ReLU on the stored 16-bit values, products and sums in fp32), so
``fp32_attention = True`` needs no separate path.  Rotary embeddings
(``rotary_emb``) are not implemented and raise ``NotImplementedError``; the
reference sends them to its eager torch path.
"""

from __future__ import annotations

import torch
from torch import nn

from .. import _lib
from ..rmsnorm.custom import RMSNorm, rms_norm_rows_
from .custom import THREADS, linear_attention

# torch dtype -> reference dtype string (SANA_LinearAttention/custom.py:16-20).
TORCH_DTYPES = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float"}


class _QKVProjection:
    """``kernel(X[B, N, C], WeightT[C, 3C]) -> QKV[B, N, 3C]`` for one shape."""

    def __init__(self, batch: int, seq_len: int, channels: int, dtype: torch.dtype):
        self.shape = (batch, seq_len, channels)
        self.channels = channels
        self.dtype = dtype

    def __call__(self, X: torch.Tensor, WeightT: torch.Tensor) -> torch.Tensor:
        if tuple(X.shape) != self.shape or X.dtype != self.dtype:
            raise ValueError(f"X must be {self.dtype} of shape {self.shape}, got {X.dtype} {tuple(X.shape)}")
        if tuple(WeightT.shape) != (self.channels, 3 * self.channels) or WeightT.dtype != self.dtype:
            raise ValueError(f"WeightT must be {self.dtype} of shape ({self.channels}, {3 * self.channels})")
        _lib.require_gpu(X, WeightT)
        return torch.matmul(X, WeightT)


def qkv_projection(batch: int, seq_len: int, channels: int, dtype: str = "bfloat16"):
    """Return the no-bias QKV projection for one shape (SANA_LinearAttention/custom.py:83-85)."""
    dtypes = {v: k for k, v in TORCH_DTYPES.items()}
    if dtype not in dtypes:
        raise ValueError(f"unsupported projection dtype: {dtype}")
    return _QKVProjection(batch, seq_len, channels, dtypes[dtype])


class LiteLA(nn.Module):
    """Lightweight ReLU linear attention (SANA_LinearAttention/original.py:65-145).

    ``qkv`` is ``Linear(in_dim, 3*in_dim, bias=use_bias)`` and ``proj`` is
    ``Linear(in_dim, in_dim)``, as the reference inherits them; heads default to
    ``out_dim // dim * heads_ratio`` and the head dim is ``out_dim // heads``.
    """

    PAD_VAL = 1

    def __init__(self, in_dim: int, out_dim: int, heads: int | None = None, heads_ratio: float = 1.0,
                 dim: int = 32, eps: float = 1e-15, use_bias: bool = False, qk_norm: bool = False,
                 norm_eps: float = 1e-5):
        super().__init__()
        heads = heads or int(out_dim // dim * heads_ratio)
        if heads <= 0 or in_dim % heads:
            raise ValueError(f"in_dim {in_dim} must split into {heads} heads")
        self.in_dim, self.out_dim, self.heads = in_dim, out_dim, heads
        self.num_heads = heads
        self.dim = out_dim // heads
        self.eps = eps
        if in_dim != heads * self.dim:
            raise ValueError(f"the packed qkv layout needs in_dim == heads * dim ({in_dim} != {heads * self.dim})")
        if self.dim <= 0 or self.dim > THREADS or THREADS % self.dim:
            raise ValueError(f"head dim {self.dim} must divide {THREADS}")
        self.qkv = nn.Linear(in_dim, in_dim * 3, bias=use_bias)
        self.proj = nn.Linear(in_dim, in_dim)
        self.kernel_func = nn.ReLU(inplace=False)
        self.qk_norm = qk_norm
        if qk_norm:
            self.q_norm = RMSNorm(in_dim, scale_factor=1.0, eps=norm_eps)
            self.k_norm = RMSNorm(in_dim, scale_factor=1.0, eps=norm_eps)
        else:
            self.q_norm = nn.Identity()
            self.k_norm = nn.Identity()

    def _packed_qkv(self, x: torch.Tensor) -> torch.Tensor:
        B, N, C = x.shape
        qkv = torch.nn.functional.linear(x, self.qkv.weight, self.qkv.bias).reshape(B, N, 3, C)
        if self.qk_norm:
            rms_norm_rows_(qkv[:, :, 0], self.q_norm.weight.detach().to(qkv.dtype), self.q_norm.eps)
            rms_norm_rows_(qkv[:, :, 1], self.k_norm.weight.detach().to(qkv.dtype), self.k_norm.eps)
        return qkv

    def _attention(self, qkv: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        # The kernel rounds its fp32 result straight to `dtype` (round to
        # nearest even), as `.to(dtype)` on the fp32 result would.
        return linear_attention(qkv, self.heads, self.dim, self.eps, dtype)

    def forward(self, x: torch.Tensor, mask=None, HW=None, rotary_emb=None, block_id=None,
                block_mask=None) -> torch.Tensor:
        if rotary_emb is not None:
            raise NotImplementedError("rotary embeddings are not implemented by the gfx950 LiteLA path")
        if x.dim() != 3 or x.shape[-1] != self.in_dim:
            raise ValueError(f"x must be [B, N, {self.in_dim}], got {tuple(x.shape)}")
        _lib.require_gpu(x)
        out = self._attention(self._packed_qkv(x), x.dtype)
        return self.proj(out)


class CustomLiteLA(LiteLA):
    """Packed-QKV LiteLA bound to one ``(batch, seq_len, dtype)`` (SANA_LinearAttention/custom.py:391-454).

    Unlike the reference's custom module, ``qk_norm=True`` is supported (the
    normalisation runs in place in the packed buffer).
    """

    def __init__(self, in_dim: int, out_dim: int, *, batch: int, seq_len: int, dtype: torch.dtype,
                 heads=None, heads_ratio: float = 1.0, dim: int = 32, eps: float = 1e-15,
                 use_bias: bool = False, qk_norm: bool = False, norm_eps: float = 1e-5):
        if dtype not in TORCH_DTYPES:
            raise ValueError(f"unsupported attention dtype: {dtype}")
        super().__init__(in_dim, out_dim, heads, heads_ratio, dim, eps, use_bias, qk_norm, norm_eps)
        self.input_shape = (batch, seq_len, in_dim)
        self.dtype = dtype

    def _validate_input(self, x: torch.Tensor) -> None:
        if tuple(x.shape) != self.input_shape:
            raise ValueError(f"expected LiteLA input shape {self.input_shape}, got {tuple(x.shape)}")
        if x.dtype != self.dtype:
            raise ValueError(f"expected LiteLA dtype {self.dtype}, got {x.dtype}")

    def forward(self, x, mask=None, HW=None, rotary_emb=None, block_id=None, block_mask=None):
        if rotary_emb is not None:
            raise NotImplementedError("rotary embeddings are not implemented by the gfx950 LiteLA path")
        self._validate_input(x)
        _lib.require_gpu(x)
        out = self._attention(self._packed_qkv(x), x.dtype)
        return self.proj(out)


class JointLiteLA(CustomLiteLA):
    """CustomLiteLA whose output projection adds the bias in the GEMM
    (SANA_LinearAttention/custom.py:526-592); needs ``in_dim == out_dim``."""

    def __init__(self, in_dim: int, out_dim: int, *, batch: int, seq_len: int, dtype: torch.dtype,
                 heads=None, heads_ratio: float = 1.0, dim: int = 32, eps: float = 1e-15,
                 use_bias: bool = False, qk_norm: bool = False, norm_eps: float = 1e-5):
        if in_dim != out_dim:
            raise ValueError("JointLiteLA requires in_dim == out_dim")
        super().__init__(in_dim, out_dim, batch=batch, seq_len=seq_len, dtype=dtype, heads=heads,
                         heads_ratio=heads_ratio, dim=dim, eps=eps, use_bias=use_bias, qk_norm=qk_norm,
                         norm_eps=norm_eps)

    def forward(self, x, mask=None, HW=None, rotary_emb=None, block_id=None, block_mask=None):
        if rotary_emb is not None:
            raise NotImplementedError("rotary embeddings are not implemented by the gfx950 LiteLA path")
        self._validate_input(x)
        _lib.require_gpu(x)
        out = self._attention(self._packed_qkv(x), x.dtype)
        bias = self.proj.bias
        if bias is None:
            bias = torch.zeros(self.out_dim, device=x.device, dtype=x.dtype)
        return torch.addmm(bias.to(x.dtype), out.reshape(-1, self.in_dim), self.proj.weight.t()).reshape(
            x.shape[0], x.shape[1], self.out_dim)
