"""LiteLA attention with the projections fused in (``kf_litela_fused_attn``).

``litela_fused_attention(x, qkv_weight, qkv_bias, heads, eps)`` returns the
LiteLA attention output before the output projection -- the value of
``linear_attention(linear(x, W, b).reshape(B, N, 3, C), heads, 32)`` -- without
writing q, k or v to memory.  Three launches:

1. k and v of a 256-token x 3- or 4-head tile are projected on MFMA, rounded,
   ReLU'd and staged in LDS, and the tile's state partial
   ``S = v^T relu(k)``, ``z = sum relu(k)`` is accumulated on MFMA;
2. the partials of each (batch, head) are summed in token-tile order
   (deterministic);
3. q of the same tiles is projected and contracted with the state.

This is the general-shape form of the reference's fused
``GroupedFull64QOutLiteLA`` kernels (SANA_LinearAttention/custom.py:606-809),
which exist there for one shape only.

Head dim 32, bf16 or fp16.  The partials live in a workspace kept per
(device, stream) and grown when a call needs more.

``prefer_fused`` is the modules' choice between this path and the unfused one
(projection GEMM, then the linear-attention kernel).  The fused tiles are tied
to heads, so the fused path needs about two rounds of workgroups per CU; and
at head counts that are multiples of 7 (3C a whole number of the GEMM's 224-
and, at 70 heads, 320-wide tiles) the unfused GEMM loses nothing to a partial
tile column and the fused path does not pay off.  Measured on MI355X (bf16,
us, fused against unfused): B=2, N=8192 at 36 / 48 / 64 heads 155 / 226 / 377
against 175 / 271 / 410; B=1, N=16384, 36 heads 158 against 175; B=2,
N=4096, 48 heads 132 against 153; but at 56 heads (B=2, N=8192; B=4, N=4096)
351 / 350 against 344 / 344, at 70 heads (B=2, N=4096; B=1, N=16384; B=4,
N=4096) 267 / 522 / 521 against 261 / 478 / 482, and under two rounds (B=2,
N=4096, 36 heads) 105 against 101.
"""

from __future__ import annotations

import threading
from typing import Optional

import torch

from .. import _lib

HEAD_DIM = 32
_DTYPES = (torch.bfloat16, torch.float16)

_ws_lock = threading.Lock()
_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    stream = torch.cuda.current_stream(device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream.cuda_stream)
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(nbytes, device=device, dtype=torch.uint8)
            _workspaces[key] = ws
    return ws


def fused_applicable(dtype: torch.dtype, dim: int) -> bool:
    """Whether the fused kernels cover this dtype and head dim."""
    return dtype in _DTYPES and dim == HEAD_DIM


def prefer_fused(batch: int, seq_len: int, heads: int, device: torch.device) -> bool:
    """True when the fused path has at least two rounds of (token tile,
    3-head group) workgroups per CU and the head count is not a multiple of 7
    (where the unfused projection's 3 * 32 * heads output columns fill whole
    224-wide GEMM tiles)."""
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    tiles = batch * -(-seq_len // 256) * -(-heads // 3)
    return tiles >= 2 * cus and heads % 7 != 0


def litela_fused_attention(x: torch.Tensor, qkv_weight: torch.Tensor, qkv_bias: Optional[torch.Tensor],
                           heads: int, eps: float = 1e-15, heads_per_group: Optional[int] = None) -> torch.Tensor:
    """``x[B, N, C]`` with the packed ``qkv_weight[3C, C]`` (and ``qkv_bias[3C]``)
    -> the attention output ``[B, N, C]`` in x's dtype, head dim 32.

    ``heads_per_group`` (3 or 4) forces the workgroup tile's head count, which
    is otherwise chosen per shape; the result is the same up to the fp32
    summation order of the state."""
    if heads_per_group not in (None, 3, 4):
        raise ValueError(f"heads_per_group must be None, 3 or 4, got {heads_per_group}")
    if x.dim() != 3:
        raise ValueError(f"x must be [B, N, C], got {tuple(x.shape)}")
    B, N, C = x.shape
    if C != heads * HEAD_DIM:
        raise ValueError(f"the fused path needs C == heads * {HEAD_DIM}, got C={C}, heads={heads}")
    if x.dtype not in _DTYPES:
        raise ValueError(f"the fused path needs bfloat16 or float16, got {x.dtype}")
    if qkv_weight.shape != (3 * C, C) or qkv_weight.dtype != x.dtype:
        raise ValueError(f"qkv_weight must be {x.dtype} [{3 * C}, {C}], got {qkv_weight.dtype} "
                         f"{tuple(qkv_weight.shape)}")
    if qkv_bias is not None and (qkv_bias.shape != (3 * C,) or qkv_bias.dtype != x.dtype):
        raise ValueError(f"qkv_bias must be {x.dtype} [{3 * C}]")
    _lib.require_gpu(x, qkv_weight, qkv_bias)
    lib = _lib.load()
    x = x.contiguous()
    w = qkv_weight.detach().contiguous()
    b = None if qkv_bias is None else qkv_bias.detach().contiguous()
    out = torch.empty_like(x)
    if out.numel() == 0:
        return out
    nbytes = int(lib.kf_litela_fused_workspace_bytes(B, N, heads))
    ws = _workspace(x.device, nbytes)
    args = (_lib.ptr(x), _lib.ptr(w), _lib.ptr(b), _lib.ptr(out), _lib.ptr(ws), ws.numel(), B, N, heads, HEAD_DIM,
            float(eps), _lib.kf_dtype(x.dtype))
    if heads_per_group is None:
        rc = lib.kf_litela_fused_attn(*args, _lib.stream_of(x))
    else:
        rc = lib.kfm_litela_fused_attn_heads(*args, heads_per_group, _lib.stream_of(x))
    _lib.check(rc, "kf_litela_fused_attn")
    return out
