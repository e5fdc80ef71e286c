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

Data path of ``forward(x[B, N, C])`` -- fused (fused.py), when head dim is
32, the dtype is 16-bit, there is no q/k norm or rotary embedding and the
shape has enough work (``LiteLA.fused_projection`` = None chooses, True/False
forces):

1. ``kf_litela_fused_attn``: q, k and v projected tile by tile and consumed
   in place (k/v -> ReLU -> state partials; fixed-order partial sum; q ->
   output), never written to memory;
2. ``y = out @ Wproj^T + b`` -- the projection GEMM with the bias in its
   epilogue.

Otherwise (unfused):

1. ``qkv = x @ Wqkv^T (+ b)`` -- the hand-written MFMA GEMM (``kf_proj_gemm``,
   projection.py) on the module's ``[3C, C]`` weight, into the packed
   ``[B, N, 3, C]`` layout.
2. ``qk_norm``: RMSNorm over the C channels of each token's q and k, in place
   in the packed buffer (``kf_rmsnorm_fwd_strided``, no copies).
3. ``rotary_emb = (cos, sin)``: rotary embedding of q and k, in place in the
   packed buffer (``kf_rope_packed``; original.py:136-138).
4. ReLU linear attention (``kf_linattn_fwd``: split states on MFMA, fixed-order
   split reduction, MFMA output contraction), fp32 arithmetic.
5. ``y = out @ Wproj^T + b`` -- the same GEMM with the bias in its epilogue.

Forward only: the linear-attention and rotary kernels have no backward, so
``forward`` raises ``RuntimeError`` when autograd would need one (grad mode on
and x or a parameter requiring grad); run the modules under
``torch.inference_mode()`` or ``torch.no_grad()``, as the reference's tests do
(SANA_LinearAttention/test.py:39, 73, 137).

Numerics: the attention always runs with the reference's ``fp32_attention``
semantics (ReLU on the stored 16-bit values, products and sums in fp32), so
``fp32_attention = True`` needs no separate path.  The reference sends
``rotary_emb`` through its eager torch path; here it is one more in-place
kernel on the packed buffer, rounded the way the eager path rounds.

``apply_rotary_emb`` (original.py:14-58) is exported as well, as the torch
helper it is in the reference (device tensors only); LiteLA does not call it.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from .. import _lib
from ..rmsnorm.custom import RMSNorm, rms_norm_rows_
from .custom import THREADS, attn_matmul, linear_attention
from .fused import fused_applicable, litela_fused_attention, prefer_fused
from .projection import TORCH_DTYPES, linear, qkv_projection  # noqa: F401  (re-exported)

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


def _project_qkv(x: torch.Tensor, weight: torch.Tensor, bias, q_norm_weight, k_norm_weight,
                 norm_eps: float) -> torch.Tensor:
    """``x[B, N, C] -> qkv[B, N, 3, C]``: the MFMA projection GEMM, then the
    optional q/k RMSNorm over C in place in the packed buffer (original.py:122-130)."""
    B, N, C = x.shape
    qkv = linear(x, weight.detach(), None if bias is None else bias.detach()).reshape(B, N, 3, C)
    if q_norm_weight is not None:
        rms_norm_rows_(qkv[:, :, 0], q_norm_weight.detach().to(qkv.dtype), norm_eps)
        rms_norm_rows_(qkv[:, :, 1], k_norm_weight.detach().to(qkv.dtype), norm_eps)
    return qkv


def _attention_output(x: torch.Tensor, qkv_weight: torch.Tensor, qkv_bias, q_norm_weight, k_norm_weight,
                      norm_eps: float, heads: int, dim: int, eps: float, fused: Optional[bool],
                      rotary_fn=None) -> torch.Tensor:
    """LiteLA's attention output before the output projection.  Without q/k
    norm and rotary embedding, with head dim 32 and a 16-bit dtype, the fused
    projection + attention kernels (fused.py) run when ``fused`` is True, or
    when it is None and they pay for the shape; otherwise the projection GEMM
    fills the packed qkv, the optional norm and rotation run in place, and the
    linear-attention kernel follows."""
    B, N, _ = x.shape
    if q_norm_weight is None and rotary_fn is None and fused_applicable(x.dtype, dim):
        if fused if fused is not None else prefer_fused(B, N, heads, x.device):
            return litela_fused_attention(x, qkv_weight.detach(),
                                          None if qkv_bias is None else qkv_bias.detach(), heads, eps)
    qkv = _project_qkv(x, qkv_weight, qkv_bias, q_norm_weight, k_norm_weight, norm_eps)
    if rotary_fn is not None:
        rotary_fn(qkv)
    # The kernel rounds its fp32 result straight to x's dtype (round to
    # nearest even), as `.to(dtype)` on the fp32 result would.
    return linear_attention(qkv, heads, dim, eps, x.dtype)


def _project_out(out: torch.Tensor, weight: torch.Tensor, bias) -> torch.Tensor:
    """``out[B, N, C] @ W^T + b`` with the bias added in fp32 in the GEMM's
    epilogue before its one rounding (custom.py:469-523; original.py:143's
    ``nn.Linear``)."""
    return linear(out, weight.detach(), None if bias is None else bias.detach())


@torch.library.custom_op("kernelforge_amd::joint_litela_forward", mutates_args=(), device_types="cuda")
def _joint_litela_op(x: torch.Tensor, qkv_weight: torch.Tensor, qkv_bias: Optional[torch.Tensor],
                     proj_weight: torch.Tensor, proj_bias: Optional[torch.Tensor],
                     q_norm_weight: Optional[torch.Tensor], k_norm_weight: Optional[torch.Tensor],
                     heads: int, dim: int, eps: float, norm_eps: float) -> torch.Tensor:
    """JointLiteLA's forward as one opaque operator (SANA_LinearAttention/custom.py:885-898)."""
    _lib.require_gpu(x)
    out = _attention_output(x, qkv_weight, qkv_bias, q_norm_weight, k_norm_weight, norm_eps, heads, dim, eps, None)
    return _project_out(out, proj_weight, proj_bias)


@_joint_litela_op.register_fake
def _joint_litela_op_fake(x, qkv_weight, qkv_bias, proj_weight, proj_bias, q_norm_weight, k_norm_weight,
                          heads, dim, eps, norm_eps):
    return x.new_empty((*x.shape[:-1], proj_weight.shape[0]))


def _require_inference(module: nn.Module, x: torch.Tensor) -> None:
    """Refuse a forward whose result autograd would have to differentiate: the
    attention kernels write through raw pointers and register no backward, so
    gradients would silently stop at the output projection."""
    if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in module.parameters())):
        raise RuntimeError(
            f"{type(module).__name__} runs forward-only HIP kernels with no backward; call it under "
            "torch.inference_mode() or torch.no_grad(), or freeze its parameters (requires_grad_(False))")


class LiteLA(nn.Module):
    """Lightweight ReLU linear attention (SANA_LinearAttention/original.py:65-145).

    ``qkv`` is ``Linear(in_dim, 3*in_dim, bias=use_bias)`` and ``proj`` is
    ``Linear(in_dim, in_dim)``, as the reference inherits them; heads default to
    ``out_dim // dim * heads_ratio`` and the head dim is ``out_dim // heads``.
    """

    PAD_VAL = 1
    # Fused projection + attention: None = chosen per shape, True / False = forced.
    fused_projection: Optional[bool] = None

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

    def attn_matmul(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        """ReLU linear attention of q ``[B, h, d, N]``, k ``[B, h, N, d]`` and v
        ``[B, h, d, N]`` -> fp32 ``[B, h, d, N]`` (original.py:99-117), on the
        HIP kernel with fp32 arithmetic; views of one packed qkv buffer, as
        ``forward`` makes them, are read in place (``custom.attn_matmul``)."""
        return attn_matmul(q, k, v, self.eps)

    def _norm_weights(self):
        if not self.qk_norm:
            return None, None, 1e-5
        return self.q_norm.weight, self.k_norm.weight, self.q_norm.eps

    def _attn_out(self, x: torch.Tensor, rotary_emb=None) -> torch.Tensor:
        qn, kn, norm_eps = self._norm_weights()
        rot = None if rotary_emb is None else (lambda qkv: self._rotate_(qkv, rotary_emb))
        return _attention_output(x, self.qkv.weight, self.qkv.bias, qn, kn, norm_eps, self.heads, self.dim,
                                 self.eps, self.fused_projection, rot)

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

    def forward(self, x: torch.Tensor, mask=None, HW=None, rotary_emb=None, block_id=None,
                block_mask=None) -> torch.Tensor:
        if x.dim() != 3 or x.shape[-1] != self.in_dim:
            raise ValueError(f"x must be [B, N, {self.in_dim}], got {tuple(x.shape)}")
        _lib.require_gpu(x)
        _require_inference(self, x)
        return _project_out(self._attn_out(x, rotary_emb), self.proj.weight, self.proj.bias)


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
        _require_inference(self, x)
        return _project_out(self._attn_out(x, rotary_emb), self.proj.weight, self.proj.bias)


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
        _require_inference(self, x)
        return _project_out(self._attn_out(x, rotary_emb), self.proj.weight, self.proj.bias)


class CustomOpJointLiteLA(JointLiteLA):
    """JointLiteLA exposed to Dynamo as one opaque custom operator
    (``kernelforge_amd::joint_litela_forward``; SANA_LinearAttention/custom.py:
    885-918), so ``torch.compile(..., fullgraph=True)`` traces it without
    graph breaks.  With ``rotary_emb`` the module falls back to
    ``JointLiteLA.forward``, as the reference does."""

    def forward(self, x, mask=None, HW=None, rotary_emb=None, block_id=None, block_mask=None):
        if rotary_emb is not None:
            return super().forward(x, mask, HW, rotary_emb, block_id, block_mask)
        self._validate_input(x)
        _lib.require_gpu(x)
        _require_inference(self, x)
        qn, kn, norm_eps = self._norm_weights()
        return _joint_litela_op(x, self.qkv.weight, self.qkv.bias, self.proj.weight, self.proj.bias, qn, kn,
                                self.heads, self.dim, self.eps, norm_eps)


class CUDAGraphJointLiteLA:
    """Fixed-shape HIP graph replay of a JointLiteLA (SANA_LinearAttention/
    custom.py:923-945): three warm-up calls on a side stream, one captured
    call, then ``__call__`` copies x into the static input (that copy is part
    of the measured cost) and replays.  The returned tensor is the graph's
    static output, overwritten by the next call."""

    def __init__(self, module: JointLiteLA):
        self.module = module
        self.static_input = torch.empty(module.input_shape, device=module.proj.weight.device, dtype=module.dtype)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.inference_mode():
            for _ in range(3):
                module(self.static_input)
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.inference_mode(), torch.cuda.graph(self.graph):
            self.static_output = module(self.static_input)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        self.static_input.copy_(x)
        self.graph.replay()
        return self.static_output


# The reference's single-shape fused module (SANA_LinearAttention/custom.py:
# 595-603, 812-861): B=1, N=1024, C=1152, 36 heads of 32, bf16.
GROUPED_SHAPE = (1, 1024, 1152)
GROUPED_HEADS, GROUPED_DIM = 36, 32


class GroupedFull64QOutLiteLA(JointLiteLA):
    """The reference's shape-specialised LiteLA (SANA_LinearAttention/custom.py:812-861),
    with its constructor checks: exactly B=1, N=1024, C=1152, H=36, D=32, bf16,
    ``qk_norm=False``, ``use_bias=False``, and no ``rotary_emb``.  Like the
    reference, it always runs the fused projection kernels (the k/v projection
    with ReLU and the state partials, then the q projection with the output;
    kf_litela_fused_attn), followed by the bias-fused output projection."""

    fused_projection = True

    def __init__(self, *args, **kwargs):
        batch, seq_len, dtype = kwargs.get("batch"), kwargs.get("seq_len"), kwargs.get("dtype")
        dim = kwargs.get("dim", GROUPED_DIM)
        heads = kwargs.get("heads")
        in_dim = args[0] if args else kwargs.get("in_dim")
        out_dim = args[1] if len(args) > 1 else kwargs.get("out_dim")
        if ((batch, seq_len, in_dim, out_dim) != (*GROUPED_SHAPE, GROUPED_SHAPE[2])
                or (heads is not None and heads != GROUPED_HEADS) or dtype != torch.bfloat16
                or dim != GROUPED_DIM or kwargs.get("qk_norm", False) or kwargs.get("use_bias", False)):
            raise ValueError("GroupedFull64QOutLiteLA requires exactly B=1,N=1024,C=1152,H=36,D=32, "
                             "bf16, qk_norm=False, and use_bias=False")
        super().__init__(*args, **kwargs)

    def forward(self, x, mask=None, HW=None, rotary_emb=None, block_id=None, block_mask=None):
        if rotary_emb is not None:
            raise ValueError("GroupedFull64QOutLiteLA requires rotary_emb=None")
        return super().forward(x, mask, HW, None, block_id, block_mask)


def optimized_joint_litela(in_dim: int, out_dim: int, **kwargs) -> JointLiteLA:
    """The module the reference picks for a shape (SANA_LinearAttention/custom.py:864-868)."""
    shape = (kwargs.get("batch"), kwargs.get("seq_len"), in_dim)
    module_cls = GroupedFull64QOutLiteLA if shape == GROUPED_SHAPE else JointLiteLA
    return module_cls(in_dim, out_dim, **kwargs)
