"""RMSNorm on gfx950: a one-pass row kernel behind the reference factory API.

``rms_norm(batch, seq_len, dim, eps, dtype)`` returns a callable
``kernel(X[batch, seq_len, dim], Weight[dim]) -> Output`` exactly like the
TileLang factory it replaces (rmsnorm/custom.py:11-31: the output is
allocated by the callable, ``out_idx=[-1]``).  The arithmetic is that of
``RMSNorm.forward`` (rmsnorm/original.py:38, 51-52): fp32 sum of squares,
``inv = 1/sqrt(mean + eps)``, then ``dt(float(dt(x*inv)) * float(w))``.

The kernel (kernelforge_amd/csrc/rmsnorm.hip) reads every row once with
16-byte vector loads into registers, reduces the sum of squares across the
64-lane wavefront (and through LDS when a row spans several wavefronts),
and writes the row once.
"""

from __future__ import annotations

from functools import lru_cache

import torch
from torch.autograd.function import once_differentiable

from .. import _lib

# dtype strings of the reference factory (torch names without "torch.").
DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32,
          "float": torch.float32}


def _launch(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, eps: float) -> None:
    lib = _lib.load()
    dim = x.shape[-1]
    rows = x.numel() // dim if dim else 0
    rc = lib.kf_rmsnorm_fwd(_lib.ptr(x), _lib.ptr(weight), _lib.ptr(out), rows, dim, float(eps),
                            _lib.kf_dtype(x.dtype), _lib.stream_of(x))
    _lib.check(rc, "kf_rmsnorm_fwd")


class RMSNormKernel:
    """Callable bound to one (batch, seq_len, dim, eps, dtype), like a compiled TileLang kernel."""

    def __init__(self, batch: int, seq_len: int, dim: int, eps: float, dtype: torch.dtype):
        self.batch, self.seq_len, self.dim = batch, seq_len, dim
        self.eps = float(eps)
        self.dtype = dtype

    def __call__(self, X: torch.Tensor, Weight: torch.Tensor) -> torch.Tensor:
        expect = (self.batch, self.seq_len, self.dim)
        if tuple(X.shape) != expect or X.dtype != self.dtype:
            raise ValueError(f"X must be {self.dtype} of shape {expect}, got {X.dtype} {tuple(X.shape)}")
        if tuple(Weight.shape) != (self.dim,) or Weight.dtype != self.dtype:
            raise ValueError(f"Weight must be {self.dtype} of shape ({self.dim},)")
        if Weight.device != X.device:
            raise ValueError("X and Weight must be on the same device")
        _lib.require_gpu(X)
        X = X.contiguous()
        Weight = Weight.contiguous()
        out = torch.empty_like(X)
        _launch(X, Weight, out, self.eps)
        return out


@lru_cache(maxsize=None)
def rms_norm(batch: int, seq_len: int, dim: int, eps: float = 1e-6, dtype: str = "bfloat16"):
    """Return ``kernel(X, Weight) -> Output`` (rmsnorm/custom.py:15-21)."""
    if dtype not in DTYPES:
        raise ValueError(f"dtype must be one of {sorted(DTYPES)}, got {dtype!r}")
    if min(batch, seq_len) < 0 or dim <= 0:
        raise ValueError("batch and seq_len must be >= 0 and dim > 0")
    return RMSNormKernel(batch, seq_len, dim, eps, DTYPES[dtype])


def rms_norm_tensor(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Shape-generic functional form: normalise over the last dimension of x."""
    if x.dim() < 1 or weight.shape != (x.shape[-1],) or weight.dtype != x.dtype:
        raise ValueError("weight must have shape (x.shape[-1],) and x's dtype")
    _lib.require_gpu(x, weight)
    x = x.contiguous()
    out = torch.empty_like(x)
    _launch(x, weight.contiguous(), out, eps)
    return out


def _row_layout(t: torch.Tensor) -> tuple[int, int]:
    """(rows, row stride) of a tensor whose rows (last dim) are contiguous and
    evenly spaced, e.g. the q slice ``qkv[:, :, 0]`` of a packed qkv buffer."""
    if t.stride(-1) != 1:
        raise ValueError("the last dimension must be contiguous")
    rows, ld = 1, t.shape[-1]
    for i in range(t.dim() - 2, -1, -1):
        if t.shape[i] == 1:
            continue
        if rows == 1:
            ld = t.stride(i)
        elif t.stride(i) != rows * ld:
            raise ValueError("rows must be evenly spaced in memory")
        rows *= t.shape[i]
    return rows, ld


def rms_norm_rows_(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Normalise every row of x (last dim) in place; x may be a strided view whose
    rows are evenly spaced, such as the q or k part of a packed ``qkv[B, N, 3, C]``
    (the LiteLA ``qk_norm`` of SANA_LinearAttention/original.py:91-94, 129-130).
    Same arithmetic as ``rms_norm`` (rmsnorm/original.py:38, 51-52)."""
    if x.dim() < 1 or weight.shape != (x.shape[-1],) or weight.dtype != x.dtype:
        raise ValueError("weight must have shape (x.shape[-1],) and x's dtype")
    _lib.require_gpu(x, weight)
    if x.numel() == 0:
        return x
    rows, ld = _row_layout(x)
    weight = weight.contiguous()
    rc = _lib.load().kf_rmsnorm_fwd_strided(_lib.ptr(x), _lib.ptr(weight), _lib.ptr(x), rows, x.shape[-1],
                                            ld, ld, float(eps), _lib.kf_dtype(x.dtype), _lib.stream_of(x))
    _lib.check(rc, "kf_rmsnorm_fwd_strided")
    return x


def original_tilelang_rms_norm(A: torch.Tensor, blk_m: int = 1) -> torch.Tensor:
    """fp32 weight-free RMSNorm with the two-scan baseline's semantics.

    Mirrors ``rms_norm(A, blk_m)`` of rmsnorm/original.py:55-78: ``A`` is
    fp32 ``[M, N]``, the result is ``A * rsqrt(sum(A^2)/N + 1e-12)``.  The
    row-block size ``blk_m`` only affected the TileLang schedule and is
    validated but not needed by the one-pass kernel.
    """
    if A.dim() != 2 or A.dtype != torch.float32:
        raise ValueError("A must be a 2-D float32 tensor")
    if blk_m <= 0:
        raise ValueError("blk_m must be positive")
    _lib.require_gpu(A)
    A = A.contiguous()
    B = torch.empty_like(A)
    rc = _lib.load().kf_rmsnorm_noweight_f32(_lib.ptr(A), _lib.ptr(B), A.shape[0], A.shape[1],
                                             1e-12, _lib.stream_of(A))
    _lib.check(rc, "kf_rmsnorm_noweight_f32")
    return B


def _promoted(x: torch.Tensor, weight: torch.Tensor) -> torch.dtype:
    return torch.promote_types(x.dtype, weight.dtype)


class _RMSNormFunction(torch.autograd.Function):
    """``RMSNorm.forward`` (rmsnorm/original.py:51-52) with torch's dtype
    promotion, and its gradient, on the HIP kernels (kf_rmsnorm_fwd_mixed,
    kf_rmsnorm_bwd).  x is normalised over its last dimension."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        lib = _lib.load()
        x = x.contiguous()
        weight = weight.contiguous()
        dim = x.shape[-1]
        rows = x.numel() // dim
        out = torch.empty(x.shape, device=x.device, dtype=_promoted(x, weight))
        rc = lib.kf_rmsnorm_fwd_mixed(_lib.ptr(x), _lib.ptr(weight), _lib.ptr(out), rows, dim, float(eps),
                                      _lib.kf_dtype(x.dtype), _lib.kf_dtype(weight.dtype),
                                      _lib.kf_dtype(out.dtype), _lib.stream_of(x))
        _lib.check(rc, "kf_rmsnorm_fwd_mixed")
        ctx.save_for_backward(x, weight)
        ctx.eps = float(eps)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        lib = _lib.load()
        dim = x.shape[-1]
        rows = x.numel() // dim
        dy = dy.contiguous().to(_promoted(x, weight))
        dx = torch.empty_like(x)
        dw = torch.empty_like(weight)
        ws_bytes = int(lib.kf_rmsnorm_bwd_workspace_bytes(rows, dim))
        ws = torch.empty(max(ws_bytes, 4), device=x.device, dtype=torch.uint8)
        rc = lib.kf_rmsnorm_bwd(_lib.ptr(x), _lib.ptr(weight), _lib.ptr(dy), _lib.ptr(dx), _lib.ptr(dw),
                                _lib.ptr(ws), ws_bytes, rows, dim, ctx.eps, _lib.kf_dtype(x.dtype),
                                _lib.kf_dtype(weight.dtype), _lib.stream_of(x))
        _lib.check(rc, "kf_rmsnorm_bwd")
        return dx, dw, None


def rms_norm_module_forward(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """``RMSNorm.forward`` semantics for any float dtypes of x and weight: the
    result has dtype ``promote_types(x.dtype, weight.dtype)`` and is
    differentiable with respect to x and weight."""
    if x.dim() < 1 or weight.dim() != 1 or weight.shape[0] != x.shape[-1]:
        raise ValueError("weight must have shape (x.shape[-1],)")
    for t in (x, weight):
        if t.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            raise ValueError(f"unsupported dtype {t.dtype}")
    _lib.require_gpu(x, weight)
    if weight.device != x.device:
        raise ValueError("x and weight must be on the same device")
    return _RMSNormFunction.apply(x, weight, eps)


_unit_weights: dict[tuple, torch.Tensor] = {}


def _unit_weight(dim: int, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """A cached weight of ones: y = dt(x * inv) * 1 rounds to x's dtype once."""
    key = (dim, dtype, str(device))
    w = _unit_weights.get(key)
    if w is None:
        w = _unit_weights[key] = torch.ones(dim, dtype=dtype, device=device)
    return w


class RMSNorm(torch.nn.Module):
    """``RMSNorm(dim, scale_factor=1.0, eps=1e-6)`` (rmsnorm/original.py:9-52) on the HIP kernels.

    The weight is an fp32 parameter of ones times ``scale_factor``
    (original.py:25).  ``forward`` returns ``dt(x * inv) * weight`` with
    torch's type promotion (original.py:51-52): bf16 input with the default
    fp32 weight gives an fp32 result; after ``.to(torch.bfloat16)`` the result
    is bf16.  Gradients with respect to x and the weight run on the HIP
    backward kernel.
    """

    def __init__(self, dim: int, scale_factor=1.0, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = torch.nn.Parameter(torch.ones(dim) * scale_factor)

    def _norm(self, x: torch.Tensor) -> torch.Tensor:
        """``x * rsqrt(mean(x^2, -1) + eps)`` in x's dtype (rmsnorm/original.py:27-38)
        on the HIP kernel, computed in fp32 and rounded once; differentiable in x."""
        return rms_norm_module_forward(x, _unit_weight(x.shape[-1], x.dtype, x.device), self.eps)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm_module_forward(x, self.weight, self.eps)
