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
3. ``rotary_emb = (cos, sin)``: rotary embedding of q and k, in place in the
   packed buffer (``kf_rope_packed``; original.py:136-138).
4. ReLU linear attention (``kf_linattn_fwd``: split states on MFMA, fixed-order
   split reduction, MFMA output contraction), fp32 arithmetic.
5. ``y = out @ Wproj^T + b`` -- library GEMM with the bias in its epilogue.

Numerics: the attention always runs with the reference's ``fp32_attention``
semantics (ReLU on the stored 16-bit values, products and sums in fp32), so
``fp32_attention = True`` needs no separate path.  The reference sends
``rotary_emb`` through its eager torch path; here it is one more in-place
kernel on the packed buffer, rounded the way the eager path rounds.

``apply_rotary_emb`` (original.py:14-58) is exported as well, as the torch
helper it is in the reference (device tensors only); LiteLA does not call it.
"""

from __future__ import annotations

import torch
from torch import nn

from .. import _lib
from ..rmsnorm.custom import RMSNorm, rms_norm_rows_
from .custom import THREADS, linear_attention

def apply_rotary_emb(x: torch.Tensor, freqs_cis, use_real: bool = True, use_real_unbind_dim: int = -1):
    """Rotary embedding with the reference's signature (SANA_LinearAttention/original.py:14-58).

    ``use_real``: ``freqs_cis = (cos, sin)`` of ``[S, D]``; channel pairs
    (2i, 2i+1) run along dim -2 of a ``[B, H, D, S]`` x (``use_real_unbind_dim
    = -2``, SANA) or along the last dim of a ``[B, H, S, D]`` x (-1) and rotate
    as ``(a, b) -> (a cos - b sin, b cos + a sin)`` with fp32 products and sum,
    rounded to x's dtype.  ``use_real=False``: complex ``freqs_cis`` of
    ``[B or 1, S, D/2]`` multiplies the pairs of a ``[B, S, H, D]`` x.
    """
    _lib.require_gpu(x)
    if not use_real:
        xf = x.float()
        z = torch.complex(xf[..., 0::2], xf[..., 1::2]) * freqs_cis.unsqueeze(2)
        return torch.stack((z.real, z.imag), dim=-1).flatten(-2).to(x.dtype)
    cos, sin = (t.to(x.device).float() for t in freqs_cis)
    if use_real_unbind_dim == -2:
        a, b = x[..., 0::2, :].float(), x[..., 1::2, :].float()
        cos, sin = cos.T, sin.T
        c_re, c_im, s_re, s_im = cos[0::2], cos[1::2], sin[0::2], sin[1::2]
        stack_dim, flat = -2, (-3, -2)
    elif use_real_unbind_dim == -1:
        a, b = x[..., 0::2].float(), x[..., 1::2].float()
        c_re, c_im, s_re, s_im = cos[..., 0::2], cos[..., 1::2], sin[..., 0::2], sin[..., 1::2]
        stack_dim, flat = -1, (-2, -1)
    else:
        raise ValueError(f"`use_real_unbind_dim={use_real_unbind_dim}` but should be -1 or -2.")
    re = a * c_re + (-b) * s_re
    im = b * c_im + a * s_im
    return torch.stack((re, im), dim=stack_dim).flatten(*flat).to(x.dtype)


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

    def _packed_qkv(self, x: torch.Tensor, rotary_emb=None) -> torch.Tensor:
        B, N, C = x.shape
        qkv = torch.nn.functional.linear(x, self.qkv.weight, self.qkv.bias).reshape(B, N, 3, C)
        if self.qk_norm:
            rms_norm_rows_(qkv[:, :, 0], self.q_norm.weight.detach().to(qkv.dtype), self.q_norm.eps)
            rms_norm_rows_(qkv[:, :, 1], self.k_norm.weight.detach().to(qkv.dtype), self.k_norm.eps)
        if rotary_emb is not None:
            self._rotate_(qkv, rotary_emb)
        return qkv

    def _rotate_(self, qkv: torch.Tensor, rotary_emb) -> None:
        """q and k of the packed qkv rotated in place (original.py:136-138)."""
        B, N, _, C = qkv.shape
        if not isinstance(rotary_emb, (tuple, list)) or len(rotary_emb) != 2:
            raise ValueError("rotary_emb must be a (cos, sin) pair of [N, head_dim] tensors")
        cos, sin = (t.detach().to(device=qkv.device, dtype=torch.float32).contiguous() for t in rotary_emb)
        if cos.shape != (N, self.dim) or sin.shape != (N, self.dim):
            raise ValueError(f"rotary_emb tensors must be [{N}, {self.dim}], got {tuple(cos.shape)}, {tuple(sin.shape)}")
        rc = _lib.load().kf_rope_packed(_lib.ptr(qkv), _lib.ptr(cos), _lib.ptr(sin), B, N, self.heads, self.dim,
                                        _lib.kf_dtype(qkv.dtype), _lib.stream_of(qkv))
        _lib.check(rc, "kf_rope_packed")

    def _attention(self, qkv: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        # The kernel rounds its fp32 result straight to `dtype` (round to
        # nearest even), as `.to(dtype)` on the fp32 result would.
        return linear_attention(qkv, self.heads, self.dim, self.eps, dtype)

    def forward(self, x: torch.Tensor, mask=None, HW=None, rotary_emb=None, block_id=None,
                block_mask=None) -> torch.Tensor:
        if x.dim() != 3 or x.shape[-1] != self.in_dim:
            raise ValueError(f"x must be [B, N, {self.in_dim}], got {tuple(x.shape)}")
        _lib.require_gpu(x)
        out = self._attention(self._packed_qkv(x, rotary_emb), x.dtype)
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
        self._validate_input(x)
        _lib.require_gpu(x)
        out = self._attention(self._packed_qkv(x, rotary_emb), x.dtype)
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
        self._validate_input(x)
        _lib.require_gpu(x)
        out = self._attention(self._packed_qkv(x, rotary_emb), x.dtype)
        bias = self.proj.bias
        if bias is None:
            bias = torch.zeros(self.out_dim, device=x.device, dtype=x.dtype)
        return torch.addmm(bias.to(x.dtype), out.reshape(-1, self.in_dim), self.proj.weight.t()).reshape(
            x.shape[0], x.shape[1], self.out_dim)
